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
// for l, as the reference kernel does.  The KV rows are bf16, or the 584-byte
// layout A rows / footer pages of engine/dsv4_kv_pack.py dequantized on the
// way in (e4m3 * 2^(e8m0-127) is exact in bf16), so the packed cache feeds
// the attention with no bf16 copy of it in HBM.
//
// One workgroup per (query token, group of 64 heads, split of the rows); a
// small batch (decode) splits its rows over several workgroups so every CU
// has one, and a second kernel merges the splits' partial maxima, sums and
// outputs.  Per block of 64 rows: the eight wavefronts gather and
// dequantize the rows into LDS twice — row-major [token][d] (the A operand of
// S^T = KV . Q^T, v_mfma_f32_16x16x32_bf16) and transposed [d][token] (the B
// operand of O += P . V, v_mfma_f32_16x16x16_bf16) — both swizzled so the
// 16-lane fragment reads are conflict-free.  S^T comes out of the MFMA with
// lane (g, r) holding tokens 4g..4g+3 of head r, which is exactly the A
// fragment layout of P for the P.V MFMA: the probabilities never leave the
// registers.  Q stays in registers for the whole kernel.
#include "sgl_common.h"
#include "sgl_numeric.h"

namespace sgl {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kD = 512;     // head dim: 448 latent + 64 rope
constexpr int kBlk = 64;    // gathered rows per block
constexpr int kHG = 64;     // heads per workgroup
constexpr int kARow = 584, kAData = 576, kANope = 448;

struct AttnArgs {
  const uint16_t* q;   // [B, M, Hh, 512] bf16
  const uint8_t* kv;   // per batch element: bf16 [n, ld] | layout A [n, 584] | layout A pages
  int64_t n;           // rows per batch element
  int64_t kv_bstride;  // bytes between batch elements
  int64_t ld;          // bf16 rows: elements per row
  int page;            // footer pages: rows per page
  const float* sink;   // [Hh]
  const int32_t* idx;  // [B, M, K]
  int64_t M, K;
  int Hh;
  float scale;
  uint16_t* o;         // [B, M, Hh, 512] bf16
  int nsplit;          // > 1: the K rows are split over workgroups, partials to ws
  int bps;             // 64-row blocks per split
  float* ws_acc;       // [B, M, nsplit, Hh, 512] unnormalised outputs
  float* ws_ml;        // [B, M, nsplit, Hh, 2] running max and sum
};

// row-major copy: token t, 16-byte chunk c (8 dims) at t*1024 + ((c ^ (t & 15)) << 4)
__device__ __forceinline__ uint32_t kv_off(int t, int c) { return (uint32_t)(t * 1024 + ((c ^ (t & 15)) << 4)); }
// transposed copy: dim d, token quad q (4 tokens, 8 bytes) at d*136 + 8q: the
// 136-byte row pitch puts the 16 dims a fragment read touches on 16 distinct
// bank pairs, and keeps every offset affine in the tile indices
constexpr int kTPitch = 136;
__device__ __forceinline__ uint32_t kvt_off(int d, int q) { return (uint32_t)(d * kTPitch + 8 * q); }

__device__ __forceinline__ uint32_t word_of(const uint4& v, int c) {
  return c < 2 ? (c == 0 ? v.x : v.y) : (c == 2 ? v.z : v.w);
}

// Raw bytes of row `id` for this lane, issued early and converted later:
// bf16 rows -> 8 bf16 values; layout A -> lanes < 56: 8 e4m3 bytes in x,y and
// the group's e8m0 byte in z; lanes 56..63: 8 rope bf16 values.
template <int FMT>
__device__ __forceinline__ uint4 load_raw(const AttnArgs& a, const uint8_t* kvb, int64_t id, int lane) {
  if constexpr (FMT == SGL_ATTN_KV_BF16) {
    return *reinterpret_cast<const uint4*>(kvb + (id * a.ld + lane * 8) * 2);
  } else {
    const uint8_t* data;
    const uint8_t* foot;
    if constexpr (FMT == SGL_ATTN_KV_A_PAGED) {
      const int64_t pg = id / a.page, l = id - pg * a.page;
      const uint8_t* pbase = kvb + pg * (int64_t)a.page * kARow;
      data = pbase + l * kAData;
      foot = pbase + (int64_t)a.page * kAData + l * 8;
    } else {
      data = kvb + id * kARow;
      foot = data + kAData;
    }
    if (lane < 56) {
      const uint2 qv = *reinterpret_cast<const uint2*>(data + lane * 8);
      return make_uint4(qv.x, qv.y, foot[lane >> 3], 0u);
    }
    const uint8_t* src = data + kANope + (lane - 56) * 16;
    const uint2 x = *reinterpret_cast<const uint2*>(src);
    const uint2 y = *reinterpret_cast<const uint2*>(src + 8);
    return make_uint4(x.x, x.y, y.x, y.y);
  }
}

template <int FMT>
__device__ __forceinline__ uint4 convert_raw(const uint4 r, int lane) {
  if constexpr (FMT == SGL_ATTN_KV_BF16) {
    return r;
  } else {
    if (lane >= 56) return r;
    const uint32_t sb = r.z;
    const float sc = sb == 0xFFu ? bits_f32(0x7FC00000u) : (sb == 0 ? bits_f32(0x00400000u) : bits_f32(sb << 23));
    float d[8];
    unpack4_e4m3(r.x, d);
    unpack4_e4m3(r.y, d + 4);
    return make_uint4(pk2_bf16_exact(d[0] * sc, d[1] * sc), pk2_bf16_exact(d[2] * sc, d[3] * sc),
                      pk2_bf16_exact(d[4] * sc, d[5] * sc), pk2_bf16_exact(d[6] * sc, d[7] * sc));
  }
}

// Eight wavefronts: wavefront w owns heads [16 (w%4), +16) of the workgroup's
// group and dims [256 (w/4), +256) of the output.  Per block of 64 rows:
//   gather: each wavefront dequantizes 8 rows (its registers were loaded
//           during the previous block) into the row-major and transposed copies;
//   S^T:    each wavefront the partial over its 256 dims; the upper-half
//           wavefronts hand theirs over in LDS;
//   softmax: the lower-half wavefront of each head group, which passes the
//           bf16 probabilities and the rescale factors on in LDS;
//   P.V:    each wavefront its 256 output dims (16 tiles of 16).
template <int FMT>
__global__ __launch_bounds__(512) void sparse_attn_kernel(const AttnArgs a) {
  __shared__ __align__(16) uint8_t sKV[kBlk * 1024];
  __shared__ __align__(16) uint8_t sKVT[kD * kTPitch];
  __shared__ __align__(16) v4f sS[4][kBlk / 16][64];
  __shared__ __align__(16) v4s sP[4][kBlk / 16][64];
  __shared__ float sAlpha[4][16];
  __shared__ float sDen[4][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hg = wave & 3, dh = wave >> 2;
  const int g4 = lane >> 4, r16 = lane & 15;
  const int64_t m = blockIdx.x, b = blockIdx.y;
  const int split = (int)(blockIdx.z % a.nsplit);
  const int h0 = (int)(blockIdx.z / a.nsplit) * kHG + hg * 16;  // this wavefront's first head
  const bool active = h0 < a.Hh;
  const uint8_t* kvb = a.kv + b * a.kv_bstride;
  const int32_t* idxp = a.idx + (b * a.M + m) * a.K;
  const int d0 = 256 * dh;
  // row-major fragment bases: token r16, chunk 32 dh + 4 c + g4 (c = ks % 4)
  uint32_t qb[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) qb[c] = kv_off(r16, 32 * dh + 4 * c + g4);
  const uint32_t vbase = kvt_off(d0 + r16, g4);  // transposed fragment base

  // Q^T fragments over this wavefront's 256 dims: lane (g, r) holds
  // q[h0 + r][d0 + 32 ks + 8 g, +8)
  v8bf qf[8];
  {
    const int h = min(h0 + r16, a.Hh - 1);
    const uint16_t* qrow = a.q + ((b * a.M + m) * a.Hh + h) * (int64_t)kD + d0;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const v8bf*>(qrow + 32 * ks + 8 * g4);
  }
  v4f acc[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) acc[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const float NEG_INF = -__builtin_huge_valf();
  float m_run = NEG_INF, l_run = 0.0f;  // lower-half wavefronts: per head r16

  // block j's indices (one per lane) and this wavefront's 8 raw rows: token
  // quads wave and wave + 8
  auto load_ids = [&](int j) -> int32_t {
    const int64_t p = (int64_t)j * kBlk + lane;
    const int32_t id = p < a.K ? idxp[p] : -1;
    return (id >= 0 && id < a.n) ? id : -1;
  };
  uint4 raw[8];
  auto load_rows = [&](int32_t ids) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int t = 4 * (wave + 8 * (r >> 2)) + (r & 3);
      const int id = __builtin_amdgcn_readfirstlane(__shfl(ids, t, 64));
      raw[r] = id >= 0 ? load_raw<FMT>(a, kvb, id, lane) : make_uint4(0, 0, 0, 0);
    }
  };

  const int nblk_all = (int)((a.K + kBlk - 1) / kBlk);
  const int jb = split * a.bps;                    // this split's first block
  const int nblk = jb + a.bps < nblk_all ? jb + a.bps : nblk_all;
  // indices run two blocks ahead of the rows, the rows one block ahead of the
  // MFMAs, so neither load latency sits in front of a block's compute
  int32_t ids = jb < nblk ? load_ids(jb) : -1;
  int32_t ids_next = jb + 1 < nblk ? load_ids(jb + 1) : -1;
  load_rows(ids);
  for (int j = jb; j < nblk; ++j) {
    const uint64_t valid = __ballot(ids >= 0);
    __syncthreads();  // the previous block's LDS is consumed
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      const int qd = wave + 8 * qh;
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v[u] = convert_raw<FMT>(raw[4 * qh + u], lane);
        *reinterpret_cast<uint4*>(sKV + kv_off(4 * qd + u, lane)) = v[u];
      }
      // dim 8 lane + c of the four tokens as one 8-byte word per c
      uint2 cw[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int sh = (c & 1) * 16;
        const uint32_t t0 = (word_of(v[0], c >> 1) >> sh) & 0xFFFFu, t1 = (word_of(v[1], c >> 1) >> sh) & 0xFFFFu;
        const uint32_t t2 = (word_of(v[2], c >> 1) >> sh) & 0xFFFFu, t3 = (word_of(v[3], c >> 1) >> sh) & 0xFFFFu;
        cw[c] = make_uint2(t0 | (t1 << 16), t2 | (t3 << 16));
      }
      // lanes start at different c (a select chain, no dynamic register
      // index) so the lanes sharing a bank pair write at different steps
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const int c = (w + lane) & 7;
        uint2 x = cw[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) x = c == e ? cw[e] : x;
        *reinterpret_cast<uint2*>(sKVT + kvt_off(8 * lane + c, qd)) = x;
      }
    }
    __syncthreads();  // block j is in LDS
    if (j + 1 < nblk) {  // the next block's rows load while this one is computed
      ids = ids_next;
      load_rows(ids);
      if (j + 2 < nblk) ids_next = load_ids(j + 2);
    }

    // partial S^T over this wavefront's dims
    v4f s[kBlk / 16];
#pragma unroll
    for (int tt = 0; tt < kBlk / 16; ++tt) s[tt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (active) {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        // chunk 32 dh + 4 ks + g of token 16 tt + r: the swizzle only flips the
        // low 4 chunk bits, so the address is qb[ks % 4] plus a constant
        const uint32_t off = (uint32_t)(256 * (ks >> 2));
        v8bf kvf[kBlk / 16];
#pragma unroll
        for (int tt = 0; tt < kBlk / 16; ++tt)
          kvf[tt] = *reinterpret_cast<const v8bf*>(sKV + qb[ks & 3] + off + 16384 * tt);
#pragma unroll
        for (int tt = 0; tt < kBlk / 16; ++tt)
          s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kvf[tt], qf[ks], s[tt], 0, 0, 0);
        // (keeps the compiler from hoisting every read of the block ahead of
        // the MFMAs, which would need 128 more registers)
        if (ks & 1) __builtin_amdgcn_sched_barrier(0);
      }
      if (dh == 1) {
#pragma unroll
        for (int tt = 0; tt < kBlk / 16; ++tt) sS[hg][tt][lane] = s[tt];
      }
    }
    __syncthreads();
    v4s pk[kBlk / 16];
    if (active && dh == 0) {
      // full S^T (lane (g, r): tokens 16 tt + 4 g + i of head r), online softmax
      float mb = NEG_INF;
#pragma unroll
      for (int tt = 0; tt < kBlk / 16; ++tt) {
        const v4f o = sS[hg][tt][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * tt + 4 * g4 + i;
          const float x = ((valid >> t) & 1ull) ? (s[tt][i] + o[i]) * a.scale : NEG_INF;
          s[tt][i] = x;
          mb = fmaxf_(mb, x);
        }
      }
      mb = fmaxf_(mb, __shfl_xor(mb, 16, 64));
      mb = fmaxf_(mb, __shfl_xor(mb, 32, 64));
      const float m_new = fmaxf_(m_run, mb);
      const float ref = m_new == NEG_INF ? 0.0f : m_new;  // a fully masked prefix keeps o = 0
      const float alpha = expf(m_run - ref);
      float ls = 0.0f;
#pragma unroll
      for (int tt = 0; tt < kBlk / 16; ++tt) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = expf(s[tt][i] - ref);
          ls += p[i];
        }
        const uint32_t w0 = pk2_bf16_exact(p[0], p[1]), w1 = pk2_bf16_exact(p[2], p[3]);
        pk[tt] = v4s{(short)(w0 & 0xFFFFu), (short)(w0 >> 16), (short)(w1 & 0xFFFFu), (short)(w1 >> 16)};
        sP[hg][tt][lane] = pk[tt];
      }
      ls += __shfl_xor(ls, 16, 64);
      ls += __shfl_xor(ls, 32, 64);
      l_run = l_run * alpha + ls;
      m_run = m_new;
      if (g4 == 0) sAlpha[hg][r16] = alpha;
    }
    __syncthreads();
    if (active) {
      if (dh == 1) {
#pragma unroll
        for (int tt = 0; tt < kBlk / 16; ++tt) pk[tt] = sP[hg][tt][lane];
      }
      // O rows are heads 4 g + i
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = sAlpha[hg][4 * g4 + i];
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[dt][i] *= al[i];
      // O += P . V over this wavefront's 16 dim tiles
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) {
        v4s vb[kBlk / 16];
#pragma unroll
        for (int tt = 0; tt < kBlk / 16; ++tt) {
          const uint2 vv = *reinterpret_cast<const uint2*>(sKVT + vbase + 16 * kTPitch * dt + 32 * tt);
          vb[tt] = v4s{(short)(vv.x & 0xFFFFu), (short)(vv.x >> 16), (short)(vv.y & 0xFFFFu), (short)(vv.y >> 16)};
        }
#pragma unroll
        for (int tt = 0; tt < kBlk / 16; ++tt)
          acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pk[tt], vb[tt], acc[dt], 0, 0, 0);
        if (dt & 1) __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  if (a.nsplit > 1) {
    // partials: the running max and sum per head, the unnormalised rows
    const int64_t qs = (b * a.M + m) * a.nsplit + split;
    if (active && dh == 0 && g4 == 0 && h0 + r16 < a.Hh) {
      float* ml = a.ws_ml + (qs * a.Hh + h0 + r16) * 2;
      ml[0] = m_run;
      ml[1] = l_run;
    }
    if (!active) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = h0 + 4 * g4 + i;
      if (h >= a.Hh) continue;
      float* row = a.ws_acc + (qs * a.Hh + h) * (int64_t)kD + d0;
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) row[16 * dt + r16] = acc[dt][i];
    }
    return;
  }
  // o = acc / (l + exp(sink - m)) for heads 4 g + i, dims d0 + 16 dt + r
  if (active && dh == 0 && g4 == 0) {
    const int hs = min(h0 + r16, a.Hh - 1);
    const float ref = m_run == NEG_INF ? 0.0f : m_run;
    sDen[hg][r16] = l_run + expf(a.sink[hs] - ref);
  }
  __syncthreads();
  if (!active) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = h0 + 4 * g4 + i;
    if (h >= a.Hh) continue;
    const float dn = sDen[hg][4 * g4 + i];
    uint16_t* orow = a.o + ((b * a.M + m) * a.Hh + h) * (int64_t)kD + d0;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) orow[16 * dt + r16] = bf16_bits_exact(acc[dt][i] / dn);
  }
}

// Merge of the per-split partials, one wavefront per (query, head):
//   M = max_s m_s;  o = sum_s acc_s e^(m_s - M) / (sum_s l_s e^(m_s - M) + e^(sink - M))
// (splits whose rows were all masked carry m = -inf and add nothing).
__global__ __launch_bounds__(256) void sparse_attn_combine_kernel(const AttnArgs a, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= rows) return;
  const int h = (int)(w % a.Hh);
  const int64_t q = w / a.Hh;  // b * M + m
  const float NEG_INF = -__builtin_huge_valf();
  float mx = NEG_INF;
  for (int sp = 0; sp < a.nsplit; ++sp) mx = fmaxf_(mx, a.ws_ml[((q * a.nsplit + sp) * a.Hh + h) * 2]);
  const float ref = mx == NEG_INF ? 0.0f : mx;
  float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float l = 0.0f;
  for (int sp = 0; sp < a.nsplit; ++sp) {
    const int64_t r = (q * a.nsplit + sp) * a.Hh + h;
    const float ms = a.ws_ml[r * 2];
    const float f = expf(ms - ref);  // 0 for an all-masked split
    l += a.ws_ml[r * 2 + 1] * f;
    const float4* src = reinterpret_cast<const float4*>(a.ws_acc + r * kD + lane * 8);
    const float4 u = src[0], v = src[1];
    o[0] += u.x * f; o[1] += u.y * f; o[2] += u.z * f; o[3] += u.w * f;
    o[4] += v.x * f; o[5] += v.y * f; o[6] += v.z * f; o[7] += v.w * f;
  }
  const float den = l + expf(a.sink[h] - ref);
  uint32_t wv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wv[i] = pk2_bf16_exact(o[2 * i] / den, o[2 * i + 1] / den);
  *reinterpret_cast<uint4*>(a.o + w * (int64_t)kD + lane * 8) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
}

// Splits of the gathered rows: enough workgroups to give every CU one, at
// most one split per 64-row block.
int attn_splits(int64_t B, int64_t M, int Hh, int64_t K) {
  const int64_t wgs = B * M * ((Hh + kHG - 1) / kHG);
  const int64_t nblk = (K + kBlk - 1) / kBlk;
  int64_t ns = (device_cu_count() + wgs - 1) / (wgs > 0 ? wgs : 1);
  if (ns > nblk) ns = nblk;
  if (ns > 64) ns = 64;
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
