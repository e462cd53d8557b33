// Sparse multi-head attention over gathered KV rows: the MLA decode consumer
// of the packed FP8 KV cache.
//
// Semantics (deepseek_infer/kernel.py:276-368 sparse_attn_kernel): for every
// query token (b, m) and head h, over the rows kv[b, idx[b, m, j]] (j < K;
// idx = -1, or outside [0, n), is masked):
//     s_j = (q[h] . kv_j) * scale                       (bf16 x bf16, fp32 sum)
//     blocks of 64 rows, online:  m' = max(m, max_j s_j);  a = exp(m - m')
//         l = l a + sum_j exp(s_j - m');  o = o a + sum_j bf16(exp(s_j - m')) kv_j
//     o / (l + exp(sink[h] - m))  -> bf16
// The probabilities are cast to bf16 for the P.V product and summed in fp32
// for l, as the reference kernel does (the exponentials are taken base 2 on
// log2(e)-scaled scores, the same values up to fp32 rounding).  The KV rows
// are bf16, or the 584-byte layout A rows / footer pages of
// engine/dsv4_kv_pack.py dequantized on the way in (e4m3 * 2^(e8m0-127) is
// exact in bf16; v_cvt_scalef32_pk_bf16_fp8 rounds it exactly), so the packed
// cache feeds the attention with no bf16 copy of it in HBM.
//
// One workgroup per (query token, group of 64 heads, split of the rows); a
// small batch (decode) splits its rows over several workgroups so every CU
// has one, and a second kernel merges the splits' partial maxima, sums and
// outputs.  Eight wavefronts, two per SIMD: wavefront (hg, dq) owns heads
// [32 hg, +32) of the group.  Per block of 64 rows:
//   gather:  each wavefront dequantizes 8 rows (loaded during the previous
//            block) into one row-major bf16 tile in LDS (swizzled);
//   S^T = KV . Q^T (v_mfma_f32_32x32x16_bf16, Q^T fragments parked in LDS):
//            wavefront dq = 2 dh + th the partial of the 32 tokens of half th
//            over dims [256 dh, +256); the partials meet in LDS and each of
//            the group's four wavefronts sums and finishes the softmax
//            (identically);
//   O^T += V^T . P^T: P^T is the S^T accumulator itself, cast to bf16 (the
//            32x32 output layout of S^T is the B operand layout of the next
//            MFMA), and V^T fragments come straight from the row-major tile
//            with ds_read_b64_tr_b16, so no transposed copy is stored; each
//            wavefront its 128 dims [128 dq, +128) over all 64 tokens.
// In both products lane (head c, half g) owns head c: the running max, sum
// and rescale factor of a head live in the lanes that hold its outputs.
#include "sgl_common.h"
#include "sgl_numeric.h"

namespace sgl {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef v4s __attribute__((address_space(3))) lds_v4s;

constexpr int kD = 512;     // head dim: 448 latent + 64 rope
constexpr int kBlk = 64;    // gathered rows per block
constexpr int kHG = 64;     // heads per workgroup
constexpr int kMaxSplits = 8;  // workgroups a query's rows split over, at most
constexpr int kARow = 584, kAData = 576, kANope = 448;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;   // [B, M, Hh, 512] bf16
  const uint8_t* kv;   // per batch element: bf16 [n, ld] | layout A [n, 584] | layout A pages
  int64_t n;           // rows per batch element
  int64_t kv_bstride;  // bytes between batch elements
  int64_t ld;          // bf16 rows: elements per row
  int page;            // footer pages: rows per page
  int page_shift;      // log2(page) when page is a power of two, else -1
  const float* sink;   // [Hh]
  const int32_t* idx;  // [B, M, K]
  int64_t M, K;
  int Hh;
  float scale;
  uint16_t* o;         // [B, M, Hh, 512] bf16
  int nsplit;          // > 1: the K rows are split over workgroups, partials to ws
  int bps;             // 64-row blocks per split
  float* ws_acc;       // [B, M, nsplit, Hh, 512] unnormalised outputs
  float* ws_ml;        // [B, M, nsplit, Hh, 2] running max (log2 units) and sum
};

// Row-major tile: token t, 16-byte chunk c (8 dims) at t*1024 + ((c ^ sw(t)) << 4).
// sw rotates the token's low four bits, which keeps conflict-free both the
// S^T fragment reads (16 B of one chunk from 16 consecutive tokens) and the
// transpose reads (8 B of 4 consecutive chunks from 4 consecutive tokens).
__device__ __forceinline__ uint32_t sw(int t) { return (uint32_t)(((t & 3) << 2) | ((t >> 2) & 3)); }

__device__ __forceinline__ v4s lds_tr16(const uint8_t* base, uint32_t off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(base + off));
}

template <bool HI>
__device__ __forceinline__ uint32_t cvt2_e4m3_bf16(uint32_t w, float sc) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, sc, HI));
}

template <int FMT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sparse_attn_kernel(const AttnArgs a) {
  __shared__ __align__(16) uint8_t sKV[kBlk * 1024];
  __shared__ __align__(16) uint4 sQ[2][2][16][64];   // Q^T fragments, [hg][dh][ks][lane]
  __shared__ __align__(16) float4 sS[8][4][64];      // S^T partials, [wave][quad][lane]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // wavefront (hg, dq): heads [32 hg, +32) of the group; S^T over dims
  // [256 dh, +256) for tokens [32 th, +32) of a block (dq = 2 dh + th), and
  // O^T over dims [128 dq, +128) for all 64 tokens
  const int hg = wave & 1, dq = wave >> 1, dh = dq >> 1, th = dq & 1;
  const int g2 = lane >> 5, c32 = lane & 31;
  const int64_t m = blockIdx.x, b = blockIdx.y;
  const int split = (int)(blockIdx.z % a.nsplit);
  const int h0 = (int)(blockIdx.z / a.nsplit) * kHG + 32 * hg;  // this wavefront's first head
  const bool active = h0 < a.Hh;
  const uint8_t* kvb = a.kv + b * a.kv_bstride;
  const int32_t* idxp = a.idx + (b * a.M + m) * a.K;

  // S^T A operand: token 32 th + c32, chunk 32 dh + 2 ks + g2; the swizzle
  // only touches the chunk's low four bits, so ks % 8 picks one of eight
  // bases and the rest is an immediate offset
  uint32_t qa[8];
#pragma unroll
  for (int k8 = 0; k8 < 8; ++k8)
    qa[k8] = (32 * th + c32) * 1024 + 512 * dh + ((((2 * k8 + g2) ^ sw(c32)) & 15) << 4);
  // V^T A operand by transpose read: in each 16-lane group G, source lane s
  // reads 4 dims of token 16 s4 + 8 e + 4 (G >> 1) + (s >> 2), and the read
  // hands each lane 4 consecutive tokens of one dim, i.e. 4 consecutive K
  // elements of one row of V^T.  Bases for each (e, dt).
  uint32_t va[2][4];
  {
    const int G = lane >> 4, s16 = lane & 15;
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int tok = 8 * e + 4 * (G >> 1) + (s16 >> 2);
        const int cl = 4 * dt + 2 * (G & 1) + ((s16 & 3) >> 1);
        va[e][dt] = tok * 1024 + 256 * dq + ((cl ^ sw(tok)) << 4) + 8 * (s16 & 1);
      }
  }

  v16f acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.0f;
  const float NEG_INF = -__builtin_huge_valf();
  const float c1 = a.scale * kLog2e;
  float m_run = NEG_INF, l_run = 0.0f;  // head c32: reference point (log2 units) and sum

  // layout A per-lane byte offsets: lanes < 56 take 8 e4m3 bytes and the
  // row's 8-byte scale footer, lanes 56..63 the 16 rope bytes in two halves
  const bool nope_lane = lane < 56;
  const uint32_t o0 = nope_lane ? 8 * lane : kANope + 16 * (lane - 56);
  const uint32_t o1r = kANope + 8 + 16 * (lane - 56);  // rope second half (rope lanes)
  const int sb_shift = 8 * ((lane >> 3) & 3);
  const bool sb_hi = (lane >> 3) >= 4;

  // A block's indices are loaded unconditionally (clamped to the last one)
  // and checked where they are used: the check waits for the load, and since
  // loads complete in order, a check right after the load would also wait
  // for every row gather issued before it.
  auto load_ids = [&](int j) -> int32_t {
    const int64_t p = (int64_t)j * kBlk + lane;
    return idxp[p < a.K ? p : a.K - 1];
  };
  auto check_id = [&](int j, int32_t id) -> int32_t {
    const int64_t p = (int64_t)j * kBlk + lane;
    return (p < a.K && id >= 0 && id < a.n) ? id : -1;
  };
  // this wavefront's 8 rows of the block: tokens 8 wave + rr.  The gathers
  // are unconditional (a missing row reads row 0, which store_rows zeroes),
  // so no branch splits the loads and the compiler's wait before the stores
  // counts the loads in flight instead of draining them.
  uint4 raw[8];
  auto load_rows = [&](int32_t ids) {
    if (a.n == 0) return;  // no rows at all: store_rows zeroes every row
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int idr = __builtin_amdgcn_readlane(ids, 8 * wave + rr);
      const int id = idr >= 0 ? idr : 0;
      uint4 v;
      {
        if constexpr (FMT == SGL_ATTN_KV_BF16) {
          v = *reinterpret_cast<const uint4*>(kvb + (int64_t)id * a.ld * 2 + lane * 16);
        } else {
          const uint8_t* data;
          const uint8_t* foot;
          if constexpr (FMT == SGL_ATTN_KV_A_PAGED) {
            const int pg = a.page_shift >= 0 ? id >> a.page_shift : (int)((uint32_t)id / (uint32_t)a.page);
            const int l = id - pg * a.page;
            const uint8_t* pbase = kvb + (int64_t)pg * a.page * kARow;
            data = pbase + l * kAData;
            foot = pbase + a.page * kAData + l * 8;
          } else {
            data = kvb + (int64_t)id * kARow;
            foot = data + kAData;
          }
          const uint2 x = *reinterpret_cast<const uint2*>(data + o0);
          const uint2 y = *reinterpret_cast<const uint2*>(nope_lane ? foot : data + o1r);
          v = make_uint4(x.x, x.y, y.x, y.y);
        }
      }
      raw[rr] = v;
    }
  };
  auto store_rows = [&](int32_t ids) {
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      uint4 v = raw[rr];
      if (__builtin_amdgcn_readlane(ids, 8 * wave + rr) < 0) v = make_uint4(0, 0, 0, 0);
      if constexpr (FMT != SGL_ATTN_KV_BF16) {
        const uint32_t word = sb_hi ? v.w : v.z;
        const float sc = bits_f32(((word >> sb_shift) & 0xFFu) << 23);  // 2^(e8m0 - 127)
        // word by word: a select of whole uint4 values goes through scratch
        const uint32_t c0 = cvt2_e4m3_bf16<false>(v.x, sc), c1 = cvt2_e4m3_bf16<true>(v.x, sc);
        const uint32_t c2 = cvt2_e4m3_bf16<false>(v.y, sc), c3 = cvt2_e4m3_bf16<true>(v.y, sc);
        v.x = nope_lane ? c0 : v.x;
        v.y = nope_lane ? c1 : v.y;
        v.z = nope_lane ? c2 : v.z;
        v.w = nope_lane ? c3 : v.w;
      }
      const int t = 8 * wave + rr;
      *reinterpret_cast<uint4*>(sKV + t * 1024 + ((lane ^ sw(t)) << 4)) = v;
    }
  };

  const int nblk_all = (int)((a.K + kBlk - 1) / kBlk);
  const int jb = split * a.bps;  // this split's first block
  const int nblk = jb + a.bps < nblk_all ? jb + a.bps : nblk_all;
  // indices run two blocks ahead of the MFMAs, the rows one block ahead;
  // past the last block the loads repeat it (their results are unused)
  int32_t ids = jb < nblk ? check_id(jb, load_ids(jb)) : -1;
  int32_t ids_next = jb < nblk ? load_ids(jb + 1 < nblk ? jb + 1 : jb) : -1;  // raw (none when K == 0)
  load_rows(ids);
  // Q^T B operand: lane (head c32, half g2) of step ks holds
  // q[h0 + c32][256 dh + 16 ks + 8 g2, +8); the two token halves share it.
  // Loaded after the first rows' gathers are issued, so its memory latency
  // overlaps theirs: the first block waits for two memory round trips (the
  // indices, then the rows with Q), not three
  {
    const int h = min(h0 + c32, a.Hh - 1);
    const uint16_t* qrow = a.q + ((b * a.M + m) * a.Hh + h) * (int64_t)kD + 256 * dh + 8 * g2;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int ks = 8 * th + k;
      sQ[hg][dh][ks][lane] = *reinterpret_cast<const uint4*>(qrow + 16 * ks);
    }
  }
  for (int j = jb; j < nblk; ++j) {
    const uint64_t valid = __ballot(ids >= 0);
    __syncthreads();  // the previous block's tile is consumed
    store_rows(ids);
    __syncthreads();  // block j (and, the first time, Q) is in LDS
    {
      const int jn = j + 1 < nblk ? j + 1 : j;
      ids = j + 1 < nblk ? check_id(jn, ids_next) : -1;
      ids_next = load_ids(j + 2 < nblk ? j + 2 : jn);  // before the rows it would wait behind
      load_rows(ids);
    }
    if (!active) {
      __syncthreads();  // (partials exchanged)
      continue;
    }
    // partial S^T of tile th over dims [256 dh, +256): lane (head c32, g2)
    // gets token 32 th + 8 (r / 4) + 4 g2 + r % 4 in sp[r]
    v16f sp;
#pragma unroll
    for (int r = 0; r < 16; ++r) sp[r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      const v8bf qf = __builtin_bit_cast(v8bf, sQ[hg][dh][ks][lane]);
      const v8bf kvf = *reinterpret_cast<const v8bf*>(sKV + qa[ks & 7] + 256 * (ks >> 3));
      sp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kvf, qf, sp, 0, 0, 0);
    }
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      sS[wave][q4][lane] = make_float4(sp[4 * q4], sp[4 * q4 + 1], sp[4 * q4 + 2], sp[4 * q4 + 3]);
    __syncthreads();  // partials exchanged
    // full S^T of both tiles: tile tt = partial (dh 0) + partial (dh 1), the
    // same sum in each of the head group's four wavefronts
    v16f s[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int w0 = hg + 2 * tt, w1 = hg + 4 + 2 * tt;  // (hg, dh = 0 / 1, th = tt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 x = sS[w0][q4][lane], y = sS[w1][q4][lane];
        s[tt][4 * q4] = x.x + y.x;
        s[tt][4 * q4 + 1] = x.y + y.y;
        s[tt][4 * q4 + 2] = x.z + y.z;
        s[tt][4 * q4 + 3] = x.w + y.w;
      }
    }
    if (valid != ~0ull) {
      const uint64_t vl = g2 ? (valid >> 4) : valid;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!((vl >> (32 * tt + 8 * (r >> 2) + (r & 3))) & 1ull)) s[tt][r] = NEG_INF;
    }
    // online softmax of head c32 (scale > 0: max(s) * c1 = max(s * c1))
    float mx = NEG_INF;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, s[tt][r]);
    mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32, 64));
    // The reference point moves only when the block maximum exceeds it by
    // more than 8 (log2 units): the probabilities stay <= 256 (exact range
    // in bf16, same relative rounding) and the accumulator is rarely
    // rescaled.  Any reference >= the running max gives the same softmax.
    const float m_blk = mx * c1;
    const bool move = !(m_blk <= m_run + 8.0f);  // also true while m_run = -inf
    const float m_new = move ? __builtin_fmaxf(m_run, m_blk) : m_run;
    const float ref = m_new == NEG_INF ? 0.0f : m_new;  // a fully masked prefix keeps o = 0
    const float alpha = move ? __builtin_amdgcn_exp2f(m_run - ref) : 1.0f;
    float ls = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[tt][r], c1, -ref));
        ls += p;
        s[tt][r] = p;
      }
    ls += __shfl_xor(ls, 32, 64);
    l_run = l_run * alpha + ls;
    m_run = m_new;
    // P^T B operands: K step s4 (16 tokens) = tile s4 / 2, registers 8 (s4 % 2) + e
    v8bf pb[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      v8s w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t pk = pk2_bf16(s[s4 >> 1][8 * (s4 & 1) + 2 * e], s[s4 >> 1][8 * (s4 & 1) + 2 * e + 1]);
        w[2 * e] = (short)(pk & 0xFFFFu);
        w[2 * e + 1] = (short)(pk >> 16);
      }
      pb[s4] = __builtin_bit_cast(v8bf, w);
    }
    if (j > jb && __ballot(alpha != 1.0f)) {  // (the accumulator is zero before the first block)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
    }
    // O^T += V^T . P^T over this wavefront's 4 tiles of 32 dims (K step
    // outer: four independent accumulators between dependent MFMAs)
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const v4s lo = lds_tr16(sKV, va[0][dt] + 16384 * s4);
        const v4s hi = lds_tr16(sKV, va[1][dt] + 16384 * s4);
        const v8bf vf = __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[s4], acc[dt], 0, 0, 0);
      }
    }
  }
  if (!active) return;
  const int h = h0 + c32;
  if (h >= a.Hh) return;
  // lane (head h, g2) holds dims 128 dq + 32 dt + 8 (r / 4) + 4 g2 + r % 4 in acc[dt][r]
  if (a.nsplit > 1) {
    const int64_t qs = (b * a.M + m) * a.nsplit + split;
    if (dq == 0 && g2 == 0) {
      float* ml = a.ws_ml + (qs * a.Hh + h) * 2;
      ml[0] = m_run;
      ml[1] = l_run;
    }
    float* row = a.ws_acc + (qs * a.Hh + h) * (int64_t)kD + 128 * dq + 4 * g2;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<float4*>(row + 32 * dt + 8 * q4) =
            make_float4(acc[dt][4 * q4], acc[dt][4 * q4 + 1], acc[dt][4 * q4 + 2], acc[dt][4 * q4 + 3]);
    return;
  }
  // o = acc / (l + exp(sink - m))
  const float ref = m_run == NEG_INF ? 0.0f : m_run;
  const float inv = 1.0f / (l_run + __builtin_amdgcn_exp2f(a.sink[h] * kLog2e - ref));
  uint16_t* orow = a.o + ((b * a.M + m) * a.Hh + h) * (int64_t)kD + 128 * dq + 4 * g2;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *reinterpret_cast<uint2*>(orow + 32 * dt + 8 * q4) =
          make_uint2(pk2_bf16(acc[dt][4 * q4] * inv, acc[dt][4 * q4 + 1] * inv),
                     pk2_bf16(acc[dt][4 * q4 + 2] * inv, acc[dt][4 * q4 + 3] * inv));
}

// Merge of the per-split partials, one wavefront per (query, head), maxima in
// log2 units:
//   M = max_s m_s;  o = sum_s acc_s 2^(m_s - M) / (sum_s l_s 2^(m_s - M) + e^(sink) 2^(-M))
// (splits whose rows were all masked carry m = -inf and add nothing).
__global__ __launch_bounds__(256) void sparse_attn_combine_kernel(const AttnArgs a, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= rows) return;
  const int h = (int)(w % a.Hh);
  const int64_t q = w / a.Hh;  // b * M + m
  const float NEG_INF = -__builtin_huge_valf();
  // every split's loads are issued before the first is used (at most
  // kMaxSplits splits), so their latencies overlap instead of adding up;
  // the maximum and the sums then run in split order as before
  float msp[kMaxSplits], lsp[kMaxSplits];
  float4 usp[kMaxSplits], vsp[kMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) {
    if (sp < a.nsplit) {
      const int64_t r = (q * a.nsplit + sp) * a.Hh + h;
      msp[sp] = a.ws_ml[r * 2];
      lsp[sp] = a.ws_ml[r * 2 + 1];
      const float4* src = reinterpret_cast<const float4*>(a.ws_acc + r * kD + lane * 8);
      usp[sp] = src[0];
      vsp[sp] = src[1];
    }
  }
  float mx = NEG_INF;
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp)
    if (sp < a.nsplit) mx = fmaxf_(mx, msp[sp]);
  const float ref = mx == NEG_INF ? 0.0f : mx;
  float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float l = 0.0f;
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) {
    if (sp < a.nsplit) {
      const float f = __builtin_amdgcn_exp2f(msp[sp] - ref);  // 0 for an all-masked split
      l += lsp[sp] * f;
      const float4 u = usp[sp], v = vsp[sp];
      o[0] += u.x * f; o[1] += u.y * f; o[2] += u.z * f; o[3] += u.w * f;
      o[4] += v.x * f; o[5] += v.y * f; o[6] += v.z * f; o[7] += v.w * f;
    }
  }
  const float den = l + __builtin_amdgcn_exp2f(a.sink[h] * kLog2e - ref);
  uint32_t wv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wv[i] = pk2_bf16_exact(o[2 * i] / den, o[2 * i + 1] / den);
  *reinterpret_cast<uint4*>(a.o + w * (int64_t)kD + lane * 8) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
}

// Splits of the gathered rows: enough workgroups to give every CU one, at
// most one split per 64-row block and at most 8 splits.
int attn_splits(int64_t B, int64_t M, int Hh, int64_t K) {
  const int64_t wgs = B * M * ((Hh + kHG - 1) / kHG);
  const int64_t nblk = (K + kBlk - 1) / kBlk;
  int64_t ns = (device_cu_count() + wgs - 1) / (wgs > 0 ? wgs : 1);
  if (ns > nblk) ns = nblk;
  // every split writes an fp32 partial of all its heads (128 KB per 64 heads)
  // that the merge reads back: past 8 splits that traffic costs more than the
  // parallelism gains (8 sequences x 2048 rows: 32 splits 45.7 us, 8 splits
  // 38.3 us, measured)
  if (ns > kMaxSplits) ns = kMaxSplits;
  if (ns <= 1) return 1;
  const int64_t bps = (nblk + ns - 1) / ns;
  return (int)((nblk + bps - 1) / bps);  // no empty split
}

}  // namespace
}  // namespace sgl

extern "C" size_t sgl_sparse_attn_workspace_size(int64_t B, int64_t M, int Hh, int64_t K) {
  if (B <= 0 || M <= 0 || Hh <= 0 || K <= 0) return 0;
  const int ns = sgl::attn_splits(B, M, Hh, K);
  if (ns == 1) return 0;
  return (size_t)(B * M * ns * Hh) * (sgl::kD + 2) * 4;
}

extern "C" int sgl_sparse_attn(const void* q, int64_t B, int64_t M, int Hh, const void* kv,
                               int kv_format, int page_size, int64_t n, int64_t kv_batch_stride,
                               int64_t ld, const float* attn_sink, const int32_t* topk_idxs,
                               int64_t K, float softmax_scale, void* o, void* workspace,
                               size_t workspace_bytes, sgl_stream_t stream) {
  SGL_REQUIRE(B >= 0 && M >= 0 && K >= 0 && n >= 0 && Hh >= 1, "sparse_attn: bad sizes");
  SGL_REQUIRE(softmax_scale > 0.0f, "sparse_attn: softmax_scale must be positive");
  SGL_REQUIRE(kv_format == SGL_ATTN_KV_BF16 || kv_format == SGL_ATTN_KV_A ||
                  kv_format == SGL_ATTN_KV_A_PAGED,
              "sparse_attn: bad kv_format %d", kv_format);
  SGL_REQUIRE(kv_format != SGL_ATTN_KV_A_PAGED || page_size > 0, "sparse_attn: page_size must be positive");
  SGL_REQUIRE(kv_format != SGL_ATTN_KV_BF16 || ld >= 512, "sparse_attn: bf16 kv row stride %lld < 512",
              (long long)ld);
  if (B == 0 || M == 0) return SGL_OK;
  SGL_REQUIRE(q && kv && attn_sink && o && (K == 0 || topk_idxs), "sparse_attn: null pointer");
  SGL_REQUIRE(sgl::aligned(q, 16) && sgl::aligned(o, 16) &&
                  sgl::aligned(kv, kv_format == SGL_ATTN_KV_BF16 ? 16 : 8) &&
                  (kv_format != SGL_ATTN_KV_BF16 || (ld % 8 == 0 && kv_batch_stride % 16 == 0)) &&
                  kv_batch_stride % 8 == 0,
              "sparse_attn: misaligned q / kv");
  SGL_REQUIRE(M <= 0x7FFFFFFF && B <= 65535, "sparse_attn: grid too large");
  sgl::AttnArgs a;
  a.q = (const uint16_t*)q;
  a.kv = (const uint8_t*)kv;
  a.n = n;
  a.kv_bstride = kv_batch_stride;
  a.ld = ld;
  a.page = page_size;
  a.page_shift = (page_size > 0 && (page_size & (page_size - 1)) == 0) ? __builtin_ctz((unsigned)page_size) : -1;
  a.sink = attn_sink;
  a.idx = topk_idxs;
  a.M = M;
  a.K = K;
  a.Hh = Hh;
  a.scale = softmax_scale;
  a.o = (uint16_t*)o;
  a.nsplit = K > 0 ? sgl::attn_splits(B, M, Hh, K) : 1;
  const int64_t nblk = (K + sgl::kBlk - 1) / sgl::kBlk;
  a.bps = (int)((nblk + a.nsplit - 1) / a.nsplit);
  a.ws_acc = nullptr;
  a.ws_ml = nullptr;
  if (a.nsplit > 1) {
    const size_t need = sgl_sparse_attn_workspace_size(B, M, Hh, K);
    if (workspace_bytes < need || !workspace) {
      sgl::set_error("sparse_attn: workspace %zu bytes < %zu needed", workspace_bytes, need);
      return SGL_ERR_WORKSPACE;
    }
    SGL_REQUIRE(sgl::aligned(workspace, 16), "sparse_attn: workspace must be 16-byte aligned");
    a.ws_acc = (float*)workspace;
    a.ws_ml = a.ws_acc + B * M * a.nsplit * (int64_t)Hh * sgl::kD;
  }
  dim3 grid((unsigned)M, (unsigned)B, (unsigned)(((Hh + sgl::kHG - 1) / sgl::kHG) * a.nsplit));
  hipStream_t st = (hipStream_t)stream;
  if (kv_format == SGL_ATTN_KV_BF16)
    sgl::sparse_attn_kernel<SGL_ATTN_KV_BF16><<<grid, 512, 0, st>>>(a);
  else if (kv_format == SGL_ATTN_KV_A)
    sgl::sparse_attn_kernel<SGL_ATTN_KV_A><<<grid, 512, 0, st>>>(a);
  else
    sgl::sparse_attn_kernel<SGL_ATTN_KV_A_PAGED><<<grid, 512, 0, st>>>(a);
  if (a.nsplit > 1) {
    const int64_t rows = B * M * Hh;
    sgl::sparse_attn_combine_kernel<<<(unsigned)sgl::ceil_div(rows, (int64_t)4), 256, 0, st>>>(a, rows);
  }
  return sgl::check_launch("sparse_attn");
}
