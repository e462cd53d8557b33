// MoE dispatch around the grouped FP8 GEMMs: router top-k, the stable
// token-to-expert permutation, the grouped gate/up and down entry points,
// the ordered unpermute-combine, and the one-call layer.
//
// Reference semantics (deepseek_infer/model.py:629-644,
// engine/v4_moe_fast.py:79-106): experts are visited in ascending id and
// torch.where(indices == e) lists that expert's slots token-ascending, so the
// permutation is a stable counting sort of slot = t*k + j by expert id; the
// combine adds the bf16 expert outputs of a token into an fp32 zero in
// ascending expert order, then adds the shared expert, then rounds to bf16.
#include <mutex>

#include "sgl_gemm.h"
#include "sgl_numeric.h"

namespace sgl {
namespace {

constexpr int kMaxRouteE = 512;    // experts per token row in route_topk
constexpr int kMaxPermE = 1024;    // experts in the permutation
constexpr int kPermThreads = 1024; // one workgroup, 16 wavefronts
constexpr int kPermWaves = kPermThreads / 64;

// ------------------------------------------------------------ route top-k

// Hash routing (deepseek_infer/model.py:576-577): the token's experts come
// from the table row tid2eid[input_ids[t]]; token ids outside [0, vocab) and
// table entries outside [0, E) are clamped into range (torch would raise).
struct HashRoute {
  const int32_t* tid2eid;  // [vocab, k], or null: score top-k
  const void* input_ids;   // [T] int32 or int64
  int ids64;
  int64_t vocab;
};

template <int EPL>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits, int64_t T,
                                                         int E, int k, int score_func,
                                                         const float* __restrict__ bias,
                                                         float route_scale, int32_t* __restrict__ ids,
                                                         float* __restrict__ weights,
                                                         const HashRoute hash) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float NEG_INF = -__builtin_huge_valf();
  float lg[EPL], sc[EPL], sel[EPL], bv[EPL];
  bool ok[EPL];
  // every load issued up front (indices past E clamped, their values dropped)
  // so the logits and the bias arrive in one memory round trip
#pragma unroll
  for (int q = 0; q < EPL; ++q) {
    const int e = lane + 64 * q;
    const int ec = e < E ? e : E - 1;
    lg[q] = logits[t * E + ec];
    bv[q] = bias ? bias[ec] : 0.0f;
  }
#pragma unroll
  for (int q = 0; q < EPL; ++q) {
    ok[q] = lane + 64 * q < E;
    lg[q] = ok[q] ? lg[q] : NEG_INF;
  }
  if (score_func == SGL_SCORE_SOFTMAX) {
    float m = NEG_INF;
#pragma unroll
    for (int q = 0; q < EPL; ++q) m = fmaxf_(m, lg[q]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf_(m, __shfl_xor(m, o, 64));
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < EPL; ++q) {
      sc[q] = ok[q] ? expf(lg[q] - m) : 0.0f;
      s += sc[q];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
#pragma unroll
    for (int q = 0; q < EPL; ++q) sc[q] = sc[q] / s;
  } else if (score_func == SGL_SCORE_SIGMOID) {
#pragma unroll
    for (int q = 0; q < EPL; ++q) sc[q] = 1.0f / (1.0f + expf(-lg[q]));
  } else {
#pragma unroll
    for (int q = 0; q < EPL; ++q) {
      const float x = lg[q];
      sc[q] = sqrtf(x > 20.0f ? x : log1pf(expf(x)));
    }
  }
  // Selection key: the scores (+ bias), which deepseek_infer/model.py:574-579
  // runs torch.topk on.  Not the logits, though every score function is
  // monotone in them: two logits can round to one fp32 score, and that tie
  // goes to the lower expert id, not to the larger logit.
#pragma unroll
  for (int q = 0; q < EPL; ++q) sel[q] = !ok[q] ? NEG_INF : (bias ? sc[q] + bv[q] : sc[q]);
  if (hash.tid2eid) {
    // weights = the original scores gathered at the table's experts, in table order
    int64_t tok = hash.ids64 ? reinterpret_cast<const int64_t*>(hash.input_ids)[t]
                             : (int64_t) reinterpret_cast<const int32_t*>(hash.input_ids)[t];
    tok = tok < 0 ? 0 : (tok >= hash.vocab ? hash.vocab - 1 : tok);
    float wsum = 0.0f;
    int my_e = 0;
    float my_s = 0.0f;
    for (int j = 0; j < k; ++j) {
      int e = hash.tid2eid[tok * k + j];
      e = (e < 0 || e >= E) ? 0 : e;
      float v = 0.0f;
#pragma unroll
      for (int q = 0; q < EPL; ++q) v = (e >> 6) == q ? sc[q] : v;
      const float bs = __shfl(v, e & 63, 64);
      if (lane == j) {
        my_e = e;
        my_s = bs;
      }
      wsum += bs;
    }
    if (lane < k) {
      float w = my_s;
      if (score_func != SGL_SCORE_SOFTMAX) w = w / wsum;
      ids[t * k + lane] = my_e;
      weights[t * k + lane] = w * route_scale;
    }
    return;
  }
  // Top-k as a radix select.  Each key becomes an unsigned image that keeps
  // the float order (-0 taken as +0, a NaN above +inf as torch.topk places it,
  // slots past E below every key); up to 32 rounds fix the k-th largest image
  // bit by bit from ballot counts, which are the same in every lane, so the
  // rounds run on scalar registers; they stop early once exactly k keys lie
  // at or above the threshold.  The keys above that threshold are taken
  // and the ties at it go to the lowest expert ids; the k picks, staged in LDS
  // in id order, then rank themselves by (key descending, id ascending):
  // torch.topk's order, ties to the lower expert id.
  __shared__ uint32_t sKey[4][16];
  __shared__ int32_t sId[4][16], sOrd[4][16];
  __shared__ float sSc[4][16];
  const int wv = threadIdx.x >> 6;
  uint32_t key[EPL];
#pragma unroll
  for (int q = 0; q < EPL; ++q) {
    uint32_t u = __float_as_uint(sel[q]);
    u = u == 0x80000000u ? 0u : u;
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    u = sel[q] != sel[q] ? 0xFFFFFFFFu : u;
    key[q] = ok[q] ? u : 0u;
  }
  uint32_t th = 0u;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = th | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int q = 0; q < EPL; ++q) cnt += __popcll(__ballot(key[q] >= cand));
    if (cnt >= k) {
      th = cand;
      if (cnt == k) break;  // exactly the k largest keys lie at or above th
    }
  }
  int need = k;
#pragma unroll
  for (int q = 0; q < EPL; ++q) need -= __popcll(__ballot(key[q] > th));
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int q = 0; q < EPL; ++q) {
    const unsigned long long eq = __ballot(key[q] == th);
    const bool pick = key[q] > th || (key[q] == th && __popcll(eq & lt_mask) < need);
    const int neq = __popcll(eq);
    need -= neq < need ? neq : need;
    const unsigned long long pm = __ballot(pick);
    if (pick) {
      const int pos = base + __popcll(pm & lt_mask);
      sKey[wv][pos] = key[q];
      sId[wv][pos] = lane + 64 * q;
      sSc[wv][pos] = sc[q];
    }
    base += __popcll(pm);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int rank = 0;
  if (lane < k) {
    const uint32_t kj = sKey[wv][lane];
    for (int i = 0; i < k; ++i) {
      const uint32_t ki = sKey[wv][i];
      rank += (ki > kj || (ki == kj && i < lane)) ? 1 : 0;
    }
    sOrd[wv][rank] = lane;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // the weight sum accumulated in rank order
  float wsum = 0.0f;
  for (int r = 0; r < k; ++r) wsum += sSc[wv][sOrd[wv][r]];
  if (lane < k) {
    float w = sSc[wv][lane];
    if (score_func != SGL_SCORE_SOFTMAX) w = w / wsum;
    ids[t * k + rank] = sId[wv][lane];
    weights[t * k + rank] = w * route_scale;
  }
}

// ------------------------------------------------------ router projection

// logits[t, e] = sum_h x[t, h] * W[e, h] for bf16 x [T, H] and bf16 W [E, H]:
// the reference computes linear(x.float(), W.float()) (deepseek_infer/model.py:
// 565); every bf16 x bf16 product is exact in fp32, so the bf16 MFMA with
// fp32 accumulation (v_mfma_f32_16x16x32_bf16) forms the same products and
// sums them in fp32 (in its own order).  A workgroup owns 16 TM tokens x 16 TE
// experts; its NWV wavefronts split K (32-deep steps w, w + NWV, ...) loading
// their operands straight from global memory, NB steps' loads in flight
// together, and the partial tiles are summed through LDS.  Rows past T / E
// re-read the last row; their outputs are dropped.
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f_r __attribute__((ext_vector_type(4)));

template <int TM, int TE, int NWV, int NB>
__global__ __launch_bounds__(64 * NWV) void router_logits_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 int64_t T, int H, int E,
                                                                 float* __restrict__ logits) {
  constexpr int RT = 16 * TM, RE = 16 * TE;
  __shared__ float sRed[NWV][RT * RE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, r16 = lane & 15;
  const int64_t t0 = (int64_t)blockIdx.y * RT;
  const int e0 = blockIdx.x * RE;
  const uint16_t* arow[TM];
  const uint16_t* brow[TE];
#pragma unroll
  for (int mi = 0; mi < TM; ++mi) {
    int64_t r = t0 + 16 * mi + r16;
    if (r > T - 1) r = T - 1;
    arow[mi] = x + r * H + 8 * g4;
  }
#pragma unroll
  for (int nj = 0; nj < TE; ++nj) {
    int r = e0 + 16 * nj + r16;
    if (r > E - 1) r = E - 1;
    brow[nj] = w + (int64_t)r * H + 8 * g4;
  }
  v4f_r acc[TM][TE];
#pragma unroll
  for (int mi = 0; mi < TM; ++mi)
#pragma unroll
    for (int nj = 0; nj < TE; ++nj) acc[mi][nj] = v4f_r{0.0f, 0.0f, 0.0f, 0.0f};
  const int steps = H / 32;
  for (int s0 = wave; s0 < steps; s0 += NWV * NB) {
    v8bf a[NB][TM], b[NB][TE];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int s = s0 + j * NWV;
      if (s < steps) {
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) a[j][mi] = *reinterpret_cast<const v8bf*>(arow[mi] + s * 32);
#pragma unroll
        for (int nj = 0; nj < TE; ++nj) b[j][nj] = *reinterpret_cast<const v8bf*>(brow[nj] + s * 32);
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (s0 + j * NWV < steps) {
#pragma unroll
        for (int mi = 0; mi < TM; ++mi)
#pragma unroll
          for (int nj = 0; nj < TE; ++nj)
            acc[mi][nj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j][mi], b[j][nj], acc[mi][nj], 0, 0, 0);
      }
    }
  }
  // lane (g4, r16) holds rows 4 g4 + r (tokens), column r16 (expert) of each 16x16 tile
#pragma unroll
  for (int mi = 0; mi < TM; ++mi)
#pragma unroll
    for (int nj = 0; nj < TE; ++nj)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sRed[wave][(16 * mi + 4 * g4 + r) * RE + 16 * nj + r16] = acc[mi][nj][r];
  __syncthreads();
  for (int i = tid; i < RT * RE; i += 64 * NWV) {
    float v = 0.0f;
#pragma unroll
    for (int q = 0; q < NWV; ++q) v += sRed[q][i];
    const int64_t t = t0 + i / RE;
    const int e = e0 + i % RE;
    if (t < T && e < E) logits[t * E + e] = v;
  }
}

// Router projection for prefill-sized batches (H % 64 == 0).  A workgroup
// of four wavefronts owns TT tokens x TE experts; the x and W rows stream
// through an NS-deep ring of 64-deep LDS stages (TT + TE rows of 128 bytes)
// by global_load_lds_dwordx4, one instruction filling 8 rows x 128 bytes, the
// 16-byte chunks swizzled (chunk c of row r at c ^ swz(r)), NS - 1 stages in
// flight.  Whole 128-byte row segments per instruction are what the L2 serves
// fastest; the register-loaded kernel above reads 16 rows x 64 bytes per
// instruction.  A wavefront computes a (TT/WT) x (TE/WE) block with
// v_mfma_f32_16x16x32_bf16: lane (g, r) reads chunks 2g and 2g + 1 of its row,
// the first MFMA takes chunk 2g's eight values and the second chunk 2g + 1's;
// x and W lanes hold the same K indices, so every MFMA sums 32 whole
// products (the 64 of a stage in two MFMAs, in the MFMA's own order).
// Tiles are numbered token-tile major, expert tile fastest, and the tiles of
// one XCD (workgroup b runs on XCD b % 8) are consecutive, so the workgroups
// reading one x tile run together on one L2.  Rows past T / E re-read the
// last row; their outputs are dropped.
template <int NI, int L>
__device__ __forceinline__ void router_wait(int later) {
  if constexpr (L == 0) {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  } else {
    if (later >= L)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(L * NI) : "memory");
    else
      router_wait<NI, L - 1>(later);
  }
}

template <int TT, int TE, int NS>
__global__ __launch_bounds__(256) void router_lds_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w, int64_t T,
                                                         int H, int E, int ntile_e, int64_t ntiles,
                                                         int64_t per_xcd, float* __restrict__ logits) {
  constexpr int WT = TT >= 32 ? 2 : 1, WE = 4 / WT;
  constexpr int ST = TT / WT, SE = TE / WE;  // a wavefront's block
  constexpr int MB = ST / 16, NB = SE / 16;
  constexpr int ROWS = TT + TE;
  constexpr int SBYTES = ROWS * 128;
  constexpr int NI = ROWS / 32;  // DMA instructions per wavefront per stage
  static_assert(ROWS % 32 == 0 && TT % 8 == 0 && ST % 16 == 0 && SE % 16 == 0, "tile shape");
  static_assert(NS >= 2 && (NS - 2) * NI <= 63, "vmcnt range");
  __shared__ __align__(16) uint8_t ring[NS * SBYTES];

  const int64_t tile = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (tile >= ntiles) return;
  const int64_t t0 = (tile / ntile_e) * TT;
  const int e0 = (int)(tile % ntile_e) * TE;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // instruction j of this wavefront fills stage rows 8 (wave + 4 j) + lane / 8
  uint64_t src[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int R = 8 * (wave + 4 * j) + (lane >> 3);
    const int c = (lane & 7) ^ swz(R);
    const uint16_t* row;
    if (R < TT) {
      const int64_t t = t0 + R < T ? t0 + R : T - 1;
      row = x + t * H;
    } else {
      const int e = e0 + R - TT < E ? e0 + R - TT : E - 1;
      row = w + (int64_t)e * H;
    }
    src[j] = (uint64_t)(uintptr_t)row + 16u * (uint32_t)c;
  }
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane(lds_u32(ring));
  const int nst = H / 64;
  auto issue = [&](int s) {
    const uint32_t slot = ring0 + (uint32_t)(s % NS) * SBYTES;
#pragma unroll
    for (int j = 0; j < NI; ++j)
      dma16v(src[j] + (uint64_t)s * 128u,
             __builtin_amdgcn_readfirstlane(slot + (uint32_t)(8 * (wave + 4 * j)) * 128u));
  };
  for (int s = 0; s < NS - 1 && s < nst; ++s) issue(s);

  const int g4 = lane >> 4, r16 = lane & 15;
  const uint32_t flo = (uint32_t)(r16 * 128 + (((2 * g4) ^ swz(r16)) << 4));
  const uint32_t fhi = (uint32_t)(r16 * 128 + (((2 * g4 + 1) ^ swz(r16)) << 4));
  const int wt = wave / WE, we = wave % WE;
  v4f_r acc[MB][NB];
#pragma unroll
  for (int mi = 0; mi < MB; ++mi)
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) acc[mi][nj] = v4f_r{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < nst; ++s) {
    // stage s has landed once at most min(NS - 2, nst - 1 - s) later stages are outstanding
    const int later = nst - 1 - s < NS - 2 ? nst - 1 - s : NS - 2;
    router_wait<NI, NS - 2>(later);
    __builtin_amdgcn_s_barrier();
    if (s + NS - 1 < nst) issue(s + NS - 1);
    const uint8_t* st = ring + (s % NS) * SBYTES;
    v8bf alo[MB], ahi[MB], blo[NB], bhi[NB];
#pragma unroll
    for (int mi = 0; mi < MB; ++mi) {
      const uint8_t* blk = st + (wt * ST + 16 * mi) * 128;
      alo[mi] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(blk + flo));
      ahi[mi] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(blk + fhi));
    }
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) {
      const uint8_t* blk = st + (TT + we * SE + 16 * nj) * 128;
      blo[nj] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(blk + flo));
      bhi[nj] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(blk + fhi));
    }
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
#pragma unroll
      for (int nj = 0; nj < NB; ++nj) {
        acc[mi][nj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo[mi], blo[nj], acc[mi][nj], 0, 0, 0);
        acc[mi][nj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi[mi], bhi[nj], acc[mi][nj], 0, 0, 0);
      }
  }
  // lane (g4, r16) holds tokens 4 g4 + r, expert r16 of each 16 x 16 block
#pragma unroll
  for (int mi = 0; mi < MB; ++mi)
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) {
      const int e = e0 + we * SE + 16 * nj + r16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t t = t0 + wt * ST + 16 * mi + 4 * g4 + r;
        if (t < T && e < E) logits[t * E + e] = acc[mi][nj][r];
      }
    }
}

// The same projection with K split over the four wavefronts (H % 128 == 0):
// 128-deep stages of 256-byte rows (one 1 KB DMA instruction fills 4 rows,
// chunk c of row r stored at c ^ (r & 15)), and wavefront w reads only its
// quarter of every row (bytes [64 w, +64): lane (g, r) the 16 bytes of chunk
// 4 w + g), one MFMA per block pair per stage over the whole TT x TE tile.
// Each stage's fragment reads then total its DMA bytes, half of what the
// 2 x 2 wavefront split reads.  After the K loop the four partial tiles meet
// in LDS and wavefront w sums rows [w TT / 4, +TT / 4) in the order
// ((p0 + p1) + p2) + p3.
template <int TT, int TE, int NS>
__global__ __launch_bounds__(256) void router_ks_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ w, int64_t T,
                                                        int H, int E, int ntile_e, int64_t ntiles,
                                                        int64_t per_xcd, float* __restrict__ logits) {
  constexpr int MB = TT / 16, NB = TE / 16;
  constexpr int ROWS = TT + TE;
  constexpr int SBYTES = ROWS * 256;
  constexpr int NI = ROWS / 16;  // DMA instructions per wavefront per stage (4 rows each)
  constexpr int RING = NS * SBYTES;
  constexpr int PART = TT * TE * 4;  // one wavefront's partial tile, fp32
  constexpr int SMEM = RING > 4 * PART ? RING : 4 * PART;
  static_assert(ROWS % 16 == 0 && TT % 16 == 0 && TE % 16 == 0 && TT % 4 == 0, "tile shape");
  static_assert(NS >= 2 && (NS - 2) * NI <= 63, "vmcnt range");
  __shared__ __align__(16) uint8_t smem[SMEM];

  const int64_t tile = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (tile >= ntiles) return;
  const int64_t t0 = (tile / ntile_e) * TT;
  const int e0 = (int)(tile % ntile_e) * TE;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // instruction j of this wavefront fills stage rows 4 (wave + 4 j) + lane / 16
  uint64_t src[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int R = 4 * (wave + 4 * j) + (lane >> 4);
    const int c = (lane & 15) ^ (R & 15);
    const uint16_t* row;
    if (R < TT) {
      const int64_t t = t0 + R < T ? t0 + R : T - 1;
      row = x + t * H;
    } else {
      const int e = e0 + R - TT < E ? e0 + R - TT : E - 1;
      row = w + (int64_t)e * H;
    }
    src[j] = (uint64_t)(uintptr_t)row + 16u * (uint32_t)c;
  }
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane(lds_u32(smem));
  const int nst = H / 128;
  auto issue = [&](int s) {
    const uint32_t slot = ring0 + (uint32_t)(s % NS) * SBYTES;
#pragma unroll
    for (int j = 0; j < NI; ++j)
      dma16v(src[j] + (uint64_t)s * 256u,
             __builtin_amdgcn_readfirstlane(slot + (uint32_t)(4 * (wave + 4 * j)) * 256u));
  };
  for (int s = 0; s < NS - 1 && s < nst; ++s) issue(s);

  const int g4 = lane >> 4, r16 = lane & 15;
  // this lane's 16 bytes of any 16-row block (blocks start at multiples of 16 rows)
  const uint32_t fo = (uint32_t)(r16 * 256 + (((4 * wave + g4) ^ r16) << 4));
  v4f_r acc[MB][NB];
#pragma unroll
  for (int mi = 0; mi < MB; ++mi)
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) acc[mi][nj] = v4f_r{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < nst; ++s) {
    const int later = nst - 1 - s < NS - 2 ? nst - 1 - s : NS - 2;
    router_wait<NI, NS - 2>(later);
    __builtin_amdgcn_s_barrier();
    if (s + NS - 1 < nst) issue(s + NS - 1);
    const uint8_t* st = smem + (s % NS) * SBYTES;
    v8bf a[MB], b[NB];
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
      a[mi] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(st + 16 * mi * 256 + fo));
#pragma unroll
    for (int nj = 0; nj < NB; ++nj)
      b[nj] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(st + (TT + 16 * nj) * 256 + fo));
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
#pragma unroll
      for (int nj = 0; nj < NB; ++nj)
        acc[mi][nj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mi], b[nj], acc[mi][nj], 0, 0, 0);
  }
  // the partial tiles meet in LDS (the ring is free once every wavefront is past its last stage)
  __syncthreads();
  float* part = reinterpret_cast<float*>(smem) + wave * (TT * TE);
#pragma unroll
  for (int mi = 0; mi < MB; ++mi)
#pragma unroll
    for (int nj = 0; nj < NB; ++nj)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[(16 * mi + 4 * g4 + r) * TE + 16 * nj + r16] = acc[mi][nj][r];
  __syncthreads();
  const float* p = reinterpret_cast<const float*>(smem);
  constexpr int RW = TT / 4;  // rows summed per wavefront
  for (int i = lane; i < RW * TE; i += 64) {
    const int row = wave * RW + i / TE, col = i % TE;
    const int o = row * TE + col;
    const float v = ((p[o] + p[TT * TE + o]) + p[2 * TT * TE + o]) + p[3 * TT * TE + o];
    const int64_t t = t0 + row;
    const int e = e0 + col;
    if (t < T && e < E) logits[t * E + e] = v;
  }
}

template <int TT, int TE, int NS>
void launch_router_ks(const uint16_t* x, const uint16_t* w, int64_t T, int H, int E,
                      float* logits, hipStream_t st) {
  const int ntile_e = (int)ceil_div(E, TE);
  const int64_t ntiles = ceil_div(T, TT) * ntile_e;
  const int64_t per_xcd = ceil_div(ntiles, 8);
  router_ks_kernel<TT, TE, NS><<<(unsigned)(8 * per_xcd), 256, 0, st>>>(x, w, T, H, E, ntile_e, ntiles,
                                                                         per_xcd, logits);
}

template <int TT, int TE, int NS>
void launch_router_lds(const uint16_t* x, const uint16_t* w, int64_t T, int H, int E,
                       float* logits, hipStream_t st) {
  const int ntile_e = (int)ceil_div(E, TE);
  const int64_t ntiles = ceil_div(T, TT) * ntile_e;
  const int64_t per_xcd = ceil_div(ntiles, 8);
  router_lds_kernel<TT, TE, NS><<<(unsigned)(8 * per_xcd), 256, 0, st>>>(x, w, T, H, E, ntile_e, ntiles,
                                                                          per_xcd, logits);
}

// -------------------------------------------------------------- permute

// Slot ranking shared by both permute forms: walk slots [lo, hi) in order,
// kPermThreads per round.  Inside a wavefront the lanes holding the same
// expert find each other with one ballot per id bit (their rank = popcount of
// lower peers), per-wavefront counts in LDS give the offset of each wavefront
// inside the round, and run[e] (the next free position of expert e) carries
// rounds forward, so equal ids keep slot order.  Writes slot_pos, and
// sorted_slot when it is non-null.  Only ids in [elo, ehi) are placed (a rank's
// local experts of an expert-sharded layer); the other slots get slot_pos -1.
__device__ void rank_slots(const int32_t* __restrict__ ids, int64_t lo, int64_t hi, int E,
                           int elo, int ehi, int* run, int (*wcnt)[kMaxPermE],
                           int32_t* __restrict__ sorted_slot, int32_t* __restrict__ slot_pos) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  for (int64_t base = lo; base < hi; base += kPermThreads) {
    const int64_t i = base + tid;
    const int e = i < hi ? ids[i] : -1;
    const bool valid = e >= elo && e < ehi;
    unsigned long long peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const unsigned long long m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    if (valid && rank == 0) wcnt[wave][e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pre = 0;
      for (int w = 0; w < wave; ++w) pre += wcnt[w][e];
      const int pos = run[e] + pre + rank;
      if (sorted_slot) sorted_slot[pos] = (int32_t)i;
      slot_pos[i] = pos;
    } else if (i < hi) {
      slot_pos[i] = -1;
    }
    __syncthreads();
    for (int x = tid; x < E; x += kPermThreads) {
      int sum = 0;
      for (int w = 0; w < kPermWaves; ++w) {
        sum += wcnt[w][x];
        wcnt[w][x] = 0;
      }
      run[x] += sum;
    }
    __syncthreads();
  }
}

// Exclusive scan of v over threads 0..E-1 of a kPermThreads workgroup (E <=
// 1024: one value per thread); returns the thread's exclusive prefix.
__device__ int block_exclusive_scan(int v, int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wsum[w];
  return base + incl - v;
}

// Small inputs: one workgroup.  Pass 1 histograms the ids in LDS, an
// exclusive scan gives the expert offsets, pass 2 ranks every slot.
__global__ __launch_bounds__(kPermThreads) void permute_kernel(const int32_t* __restrict__ ids,
                                                               int64_t P, int E,
                                                               int32_t* __restrict__ counts,
                                                               int32_t* __restrict__ offsets,
                                                               int32_t* __restrict__ sorted_slot,
                                                               int32_t* __restrict__ slot_pos,
                                                               int32_t* __restrict__ zero, int nzero,
                                                               int elo, int ehi) {
  __shared__ int cnt[kMaxPermE];
  __shared__ int run[kMaxPermE];
  __shared__ int wcnt[kPermWaves][kMaxPermE];
  __shared__ int wsum[kPermWaves];
  const int tid = threadIdx.x;
  if (zero && tid < nzero) zero[tid] = 0;
  for (int e = tid; e < E; e += kPermThreads) {
    cnt[e] = 0;
    for (int w = 0; w < kPermWaves; ++w) wcnt[w][e] = 0;
  }
  __syncthreads();
  for (int64_t i = tid; i < P; i += kPermThreads) {
    const int e = ids[i];
    if (e >= elo && e < ehi) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  {
    const int v = tid < E ? cnt[tid] : 0;
    const int excl = block_exclusive_scan(v, wsum);
    if (tid < E) {
      run[tid] = excl;
      counts[tid] = v;
      offsets[tid] = excl;
    }
    if (tid == E - 1) offsets[E] = excl + v;
  }
  __syncthreads();
  rank_slots(ids, 0, P, E, elo, ehi, run, wcnt, sorted_slot, slot_pos);
}

// Large inputs: chunks of kPermChunk slots, one workgroup each, in four
// launches.  The per-chunk tables live in the outputs before the outputs are
// final: (1) chunk histograms -> slot_pos[c*E + e]; (2) one workgroup sums
// them into counts / offsets and writes each chunk's start position per
// expert -> sorted_slot[c*E + e]; (3) each chunk ranks its slots from those
// starts and writes slot_pos; (4) sorted_slot[slot_pos[i]] = i.  Needs
// chunks * E <= P (checked by the caller).
constexpr int kPermChunk = 4096;

__global__ __launch_bounds__(kPermThreads) void permute_hist_kernel(const int32_t* __restrict__ ids,
                                                                    int64_t P, int E, int elo,
                                                                    int ehi,
                                                                    int32_t* __restrict__ hist) {
  __shared__ int cnt[kMaxPermE];
  const int tid = threadIdx.x;
  const int64_t lo = (int64_t)blockIdx.x * kPermChunk;
  const int64_t hi = lo + kPermChunk < P ? lo + kPermChunk : P;
  for (int e = tid; e < E; e += kPermThreads) cnt[e] = 0;
  __syncthreads();
  for (int64_t i = lo + tid; i < hi; i += kPermThreads) {
    const int e = ids[i];
    if (e >= elo && e < ehi) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  for (int e = tid; e < E; e += kPermThreads) hist[(int64_t)blockIdx.x * E + e] = cnt[e];
}

__global__ __launch_bounds__(kPermThreads) void permute_scan_kernel(const int32_t* __restrict__ hist,
                                                                    int nchunks, int E,
                                                                    int32_t* __restrict__ counts,
                                                                    int32_t* __restrict__ offsets,
                                                                    int32_t* __restrict__ starts,
                                                                    int32_t* __restrict__ zero,
                                                                    int nzero) {
  __shared__ int wsum[kPermWaves];
  const int tid = threadIdx.x;
  if (zero && tid < nzero) zero[tid] = 0;
  int v = 0;
  if (tid < E)
    for (int c = 0; c < nchunks; ++c) v += hist[(int64_t)c * E + tid];
  const int excl = block_exclusive_scan(v, wsum);
  if (tid < E) {
    counts[tid] = v;
    offsets[tid] = excl;
    int run = excl;
    for (int c = 0; c < nchunks; ++c) {
      const int h = hist[(int64_t)c * E + tid];
      starts[(int64_t)c * E + tid] = run;
      run += h;
    }
  }
  if (tid == E - 1) offsets[E] = excl + v;
}

__global__ __launch_bounds__(kPermThreads) void permute_rank_kernel(const int32_t* __restrict__ ids,
                                                                    int64_t P, int E, int elo,
                                                                    int ehi,
                                                                    const int32_t* __restrict__ starts,
                                                                    int32_t* __restrict__ slot_pos) {
  __shared__ int run[kMaxPermE];
  __shared__ int wcnt[kPermWaves][kMaxPermE];
  const int tid = threadIdx.x;
  const int64_t lo = (int64_t)blockIdx.x * kPermChunk;
  const int64_t hi = lo + kPermChunk < P ? lo + kPermChunk : P;
  for (int e = tid; e < E; e += kPermThreads) {
    run[e] = starts[(int64_t)blockIdx.x * E + e];
    for (int w = 0; w < kPermWaves; ++w) wcnt[w][e] = 0;
  }
  __syncthreads();
  rank_slots(ids, lo, hi, E, elo, ehi, run, wcnt, nullptr, slot_pos);
}

__global__ __launch_bounds__(256) void permute_scatter_kernel(const int32_t* __restrict__ slot_pos,
                                                              int64_t P,
                                                              int32_t* __restrict__ sorted_slot) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < P;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t p = slot_pos[i];
    if (p >= 0) sorted_slot[p] = (int32_t)i;
  }
}

// -------------------------------------------------------------- combine

// The rows are read with nontemporal loads (each once: T = 8192, 604 MB,
// 129 -> 114 us).
// One workgroup per (token, column slice): sum the token's expert rows (bf16)
// whose expert id lies in [elo, ehi) into fp32 in ascending expert id, then
// either add the shared row and round to bf16 (PARTIAL false: the whole
// layer) or store the fp32 sum (PARTIAL true: one rank's share of an
// expert-sharded layer, before the caller's all-reduce; the shared row is
// not added).  8 columns / thread; workgroup y of gridDim.y takes the column
// slices y, y + gridDim.y, ... of NT * 8 columns (small batches split the row
// over several workgroups so the launch still covers the CUs).
template <int NT, bool PARTIAL>
__global__ __launch_bounds__(NT) void combine_kernel(const uint16_t* __restrict__ out,
                                                     const int32_t* __restrict__ ids, int64_t T,
                                                     int k, int64_t H, int has_shared, int elo,
                                                     int ehi, void* __restrict__ y) {
  __shared__ int ord[16];
  __shared__ int nvalid;
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid == 0) nvalid = 0;
  __syncthreads();
  if (tid < k) {
    const int my = ids[t * k + tid];
    if (my >= elo && my < ehi) {
      int rank = 0;
      for (int j = 0; j < k; ++j) {
        const int o = ids[t * k + j];
        if (o < elo || o >= ehi) continue;
        if (o < my || (o == my && j < tid)) ++rank;
      }
      ord[rank] = tid;
      atomicAdd(&nvalid, 1);
    }
  }
  __syncthreads();
  const int nv = nvalid;
  const int stride_rows = k + has_shared;
  const uint16_t* base = out + t * stride_rows * H;
  for (int64_t col = ((int64_t)blockIdx.y * NT + tid) * 8; col < H; col += (int64_t)gridDim.y * NT * 8) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    // every row's load is issued before the first is summed (k <= 16), so
    // their latencies overlap; the sum runs in ascending expert order as
    // before, the shared row last
    uint4 rv[16];
#pragma unroll
    for (int jj = 0; jj < 16; ++jj)
      if (jj < nv) rv[jj] = ld16_stream(base + (int64_t)ord[jj] * H + col);
    const uint4 sv = !PARTIAL && has_shared ? ld16_stream(base + (int64_t)k * H + col) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      if (jj < nv) {
        const uint32_t w[4] = {rv[jj].x, rv[jj].y, rv[jj].z, rv[jj].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += bits_f32(w[i] << 16);
          acc[2 * i + 1] += bits_f32(w[i] & 0xFFFF0000u);
        }
      }
    }
    if constexpr (PARTIAL) {
      float4* yo = reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + t * H + col);
      yo[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      yo[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    } else {
      if (has_shared) {
        const uint4 v = sv;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += bits_f32(w[i] << 16);
          acc[2 * i + 1] += bits_f32(w[i] & 0xFFFF0000u);
        }
      }
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = pk2_bf16_exact(acc[2 * i], acc[2 * i + 1]);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(y) + t * H + col) =
          make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// T tokens of H columns: 256-thread workgroups, one per token, from about
// two per CU; below, 64-thread workgroups over 512-column slices (T = 64,
// H = 4096: 512 workgroups where one per token gives 64)
template <bool PARTIAL>
void launch_combine(const uint16_t* out, const int32_t* ids, int64_t T, int k, int64_t H,
                    int has_shared, int elo, int ehi, void* y, hipStream_t st) {
  if (T >= 2 * (int64_t)device_cu_count()) {
    combine_kernel<256, PARTIAL><<<dim3((unsigned)T, 1), 256, 0, st>>>(out, ids, T, k, H, has_shared,
                                                                       elo, ehi, y);
  } else {
    const unsigned slices = (unsigned)ceil_div(H, 64 * 8);
    combine_kernel<64, PARTIAL><<<dim3((unsigned)T, slices), 64, 0, st>>>(out, ids, T, k, H,
                                                                          has_shared, elo, ehi, y);
  }
}

// y[t] = bf16(y_local[t] + shared row t), the shared expert's output added
// after the caller's all-reduce of the ranks' fp32 partial sums
// (engine/v4_moe_fast.py:103-106).  One thread per 8 columns.
__global__ __launch_bounds__(256) void add_shared_kernel(const float* __restrict__ y_local,
                                                         const uint16_t* __restrict__ out, int64_t T,
                                                         int k, int64_t H,
                                                         uint16_t* __restrict__ y) {
  const int64_t n8 = T * H / 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const int64_t t = i * 8 / H, col = i * 8 - t * H;
    const float4 a = reinterpret_cast<const float4*>(y_local + t * H + col)[0];
    const float4 b = reinterpret_cast<const float4*>(y_local + t * H + col)[1];
    const uint4 v = *reinterpret_cast<const uint4*>(out + (t * (k + 1) + k) * H + col);
    const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = pk2_bf16_exact(f[2 * q] + bits_f32(w[q] << 16), f[2 * q + 1] + bits_f32(w[q] & 0xFFFF0000u));
    *reinterpret_cast<uint4*>(y + t * H + col) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

}  // namespace

// ------------------------------------------------- static layer workspace
// The workspace of sgl_moe_forward_noalloc: a file-scope device array (each
// GPU holds its own copy for the life of the process).  In host code its
// name is a stand-in, not a device address: the address comes from
// hipGetSymbolAddress, resolved once per device with that device current
// and kept in scratch_dev[]; only that pointer is ever passed to kernels.
constexpr size_t kScratchBytes = SGL_MOE_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex scratch_mu;
static void* scratch_dev[kMaxDevices] = {};

// Device address of the current device's scratch array (resolved on the
// first call for that device).
int moe_scratch_ptr(void** out) {
  int dev = 0;
  SGL_CHECK_HIP(hipGetDevice(&dev));
  SGL_REQUIRE(dev >= 0 && dev < kMaxDevices, "moe scratch: device %d above %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("moe scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                hipGetErrorString(e));
      return SGL_ERR_HIP;
    }
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return SGL_OK;
}

namespace {

struct MoeWorkspace {
  uint8_t* xq;
  float* xs;
  int32_t* counts;
  int32_t* offsets;
  int32_t* sorted_slot;
  int32_t* slot_pos;
  uint8_t* hq;
  float* hs;
  uint16_t* out;      // the down projection's rows; before down runs, the FP4
                      // layer's shared gate/up split-K partials (same stream)
  size_t out_bytes;
  int32_t* tile_ctr;  // [4][8] per-XCD tile counters of the gate/up and down GEMMs
                      // (routed + shared, or one launch each)
  size_t bytes;
};

constexpr int kTileCtrs = 32;

MoeWorkspace carve(void* base, int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  MoeWorkspace w = {};
  const int64_t P = T * k;
  const int64_t rows = P + (has_shared ? T : 0);
  uint8_t* p = reinterpret_cast<uint8_t*>(base);
  int64_t off = 0;
  auto take = [&](int64_t n) {
    uint8_t* q = p ? p + off : nullptr;
    off += align256(n);
    return q;
  };
  w.xq = take(T * H);
  w.xs = reinterpret_cast<float*>(take(T * (H / 128) * 4));
  w.counts = reinterpret_cast<int32_t*>(take((int64_t)E * 4));
  w.offsets = reinterpret_cast<int32_t*>(take((int64_t)(E + 1) * 4));
  w.sorted_slot = reinterpret_cast<int32_t*>(take(P * 4));
  w.slot_pos = reinterpret_cast<int32_t*>(take(P * 4));
  w.hq = take(rows * I);
  w.hs = reinterpret_cast<float*>(take(rows * (I / 128) * 4));
  w.out_bytes = (size_t)(T * (k + has_shared) * H * 2);
  w.out = reinterpret_cast<uint16_t*>(take(T * (k + has_shared) * H * 2));
  w.tile_ctr = reinterpret_cast<int32_t*>(take(kTileCtrs * 4));
  w.bytes = (size_t)off;
  return w;
}

// The routed experts' format without the power-of-two flag.
constexpr int kExpertFlags = SGL_EXPERT_POW2_SCALES | SGL_EXPERT_FRAG_COPY;
bool fp4_experts(int expert_format) {
  return (expert_format & ~kExpertFlags) == SGL_EXPERT_FP4_E2M1;
}

int check_moe_shapes(const char* what, int64_t T, int64_t H, int64_t I, int E, int k,
                     int expert_format) {
  SGL_REQUIRE(T >= 0 && H > 0 && I > 0, "%s: bad shape T=%lld H=%lld I=%lld", what, (long long)T,
              (long long)H, (long long)I);
  SGL_REQUIRE(H % 128 == 0 && I % 128 == 0, "%s: H and I must be multiples of 128", what);
  SGL_REQUIRE((expert_format & ~kExpertFlags) == SGL_EXPERT_FP8_BLOCK128 ||
                  (expert_format & ~kExpertFlags) == SGL_EXPERT_FP4_E2M1,
              "%s: bad expert_format %d", what, expert_format);
  SGL_REQUIRE(!fp4_experts(expert_format) || (H % 256 == 0 && I % 256 == 0),
              "%s: FP4 experts need H and I multiples of 256", what);
  SGL_REQUIRE(E >= 1 && E <= kMaxPermE, "%s: E=%d not in [1, %d]", what, E, kMaxPermE);
  SGL_REQUIRE(k >= 1 && k <= 16 && k <= E, "%s: k=%d not in [1, min(16, E)]", what, k);
  SGL_REQUIRE(T * k < 0x7FFFFFFF && T * (k + 1) * H < ((int64_t)1 << 46), "%s: too many tokens",
              what);
  // the grouped GEMMs address operand rows with 32-bit lane offsets: the
  // gate/up A operand is xq [T, H], the down A operand hq [T (k + 1), I]
  SGL_REQUIRE(T * H < ((int64_t)1 << 31) && T * (k + 1) * I < ((int64_t)1 << 31),
              "%s: T=%lld tokens exceed the 2 GiB operand limit (T*H=%lld, T*(k+1)*I=%lld)", what,
              (long long)T, (long long)(T * H), (long long)(T * (k + 1) * I));
  return SGL_OK;
}

// Also zeroes zero[0, nzero) (nzero <= 1024) on the way, for the caller's
// tile counters.  Only the slots whose expert lies in [elo, ehi) are placed
// (0 <= elo <= ehi <= E; the whole range for a layer on one rank).
int launch_permute(const int32_t* ids, int64_t T, int k, int E, int32_t* counts, int32_t* offsets,
                   int32_t* sorted_slot, int32_t* slot_pos, int32_t* zero, int nzero,
                   hipStream_t st, int elo = 0, int ehi = -1) {
  if (ehi < 0) ehi = E;
  SGL_REQUIRE(T >= 0 && k >= 1, "moe_permute: bad T=%lld k=%d", (long long)T, k);
  SGL_REQUIRE(E >= 1 && E <= kMaxPermE, "moe_permute: E=%d not in [1, %d]", E,
              kMaxPermE);
  SGL_REQUIRE(0 <= elo && elo <= ehi && ehi <= E, "moe_permute: expert range [%d, %d) not in [0, %d]",
              elo, ehi, E);
  SGL_REQUIRE(T * k < 0x7FFFFFFF, "moe_permute: T*k too large");
  SGL_REQUIRE(counts && offsets && (T == 0 || (ids && sorted_slot && slot_pos)),
              "moe_permute: null pointer");
  const int64_t P = T * k;
  const int64_t chunks = ceil_div(P, (int64_t)kPermChunk);
  if (P < 4 * kPermChunk || chunks * E > P) {
    permute_kernel<<<1, kPermThreads, 0, st>>>(ids, P, E, counts, offsets, sorted_slot, slot_pos,
                                               zero, nzero, elo, ehi);
    return check_launch("moe_permute");
  }
  permute_hist_kernel<<<(unsigned)chunks, kPermThreads, 0, st>>>(ids, P, E, elo, ehi, slot_pos);
  permute_scan_kernel<<<1, kPermThreads, 0, st>>>(slot_pos, (int)chunks, E, counts, offsets,
                                                       sorted_slot, zero, nzero);
  permute_rank_kernel<<<(unsigned)chunks, kPermThreads, 0, st>>>(ids, P, E, elo, ehi, sorted_slot,
                                                                  slot_pos);
  int64_t sblocks = ceil_div(P, (int64_t)256);
  if (sblocks > 4096) sblocks = 4096;
  permute_scatter_kernel<<<(unsigned)sblocks, 256, 0, st>>>(slot_pos, P, sorted_slot);
  return check_launch("moe_permute");
}

bool pow2_scale_mode(int scale_mode) {
  return scale_mode == SGL_SCALE_TORCH_UE8M0 || scale_mode == SGL_SCALE_TILELANG_UE8M0;
}

// FP4 layers run the FP8 shared expert in a launch of its own after the
// routed launch, on the same stream.
int run_routed_and_shared(int kind, GemmArgs& g, GemmArgs& sh, int64_t T, hipStream_t stream) {
  const int rc = launch_gemm(kind, g, g.T * g.k / g.E, stream);
  return rc ? rc : launch_gemm(kind, sh, T, stream);
}

// The routed experts in `expert_format`; the shared expert (experts[E]) is
// always FP8 128 x 128 (deepseek_infer/model.py:623-626 builds it without the
// routed experts' dtype).  FP4 routed experts run in a launch of their own,
// followed by the shared expert's FP8 launch over the rows from offsets[E].
// tile_ctr: 16 zeroed counters (or null) for the two launches.
int run_gate_up(const void* xq, const float* xs, int64_t T, int64_t H, int64_t I, int E, int k,
                const int32_t* offsets, const int32_t* sorted_slot, const float* route_w,
                const sgl_expert_ptrs* experts, int has_shared, int expert_format,
                float swiglu_limit, int scale_mode, void* hq, float* hs, int* tile_ctr,
                hipStream_t stream, void* part = nullptr, size_t part_bytes = 0) {
  int rc = check_moe_shapes("moe_gate_up", T, H, I, E, k, expert_format);
  if (rc) return rc;
  SGL_REQUIRE(scale_mode >= 0 && scale_mode <= 3, "moe_gate_up: bad scale_mode %d", scale_mode);
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(xq && xs && offsets && sorted_slot && experts && hq && hs,
              "moe_gate_up: null pointer");
  SGL_REQUIRE(aligned(xq, 16) && aligned(hq, 8), "moe_gate_up: xq/hq misaligned");
  const bool split = fp4_experts(expert_format);
  const int pow2w = (expert_format & SGL_EXPERT_POW2_SCALES) ? 1 : 0;
  GemmArgs g = {};
  g.a = (const uint8_t*)xq;
  g.sa = xs;
  g.experts = experts;
  g.offsets = offsets;
  g.sorted_slot = sorted_slot;
  g.route_w = route_w;
  g.E = E;
  g.k = k;
  g.has_shared = has_shared && !split ? 1 : 0;
  g.out_k = k + (has_shared ? 1 : 0);
  g.T = T;
  g.N = I;
  g.K = H;
  g.hq = (uint8_t*)hq;
  g.hs = hs;
  g.swiglu_limit = swiglu_limit;
  g.scale_mode = scale_mode;
  g.wfmt = split ? WF_FP4 : WF_FP8;
  g.sa_pow2 = pow2_scale_mode(scale_mode);
  g.sb_pow2 = split ? 0 : pow2w;
  g.tile_ctr = tile_ctr;
  // the fragment-layout records follow the E (+ shared) row-major ones
  const sgl_expert_ptrs* frag =
      (expert_format & SGL_EXPERT_FRAG_COPY) ? experts + E + (has_shared ? 1 : 0) : nullptr;
  g.frag = frag;
  if (!split || !has_shared) return launch_gemm(KIND_GATE_UP, g, T * k / E, stream);
  GemmArgs sh = g;  // the shared expert: one group whose rows start at offsets[E]
  sh.E = 0;
  sh.offsets = offsets + E;
  sh.experts = experts + E;
  sh.frag = frag ? frag + E : nullptr;
  sh.has_shared = 1;
  sh.wfmt = WF_FP8;
  sh.sb_pow2 = pow2w;
  sh.tile_ctr = tile_ctr ? tile_ctr + 8 : nullptr;
  // at decode sizes the shared expert's weight stream split over K, so about
  // one workgroup per CU carries it (its tiles alone are 32), in the
  // caller's spare space; the grouped launch otherwise
  if (part) {
    if ((rc = launch_gemm(KIND_GATE_UP, g, g.T * g.k / g.E, stream))) return rc;
    rc = launch_shared_gate_up_split(sh, part, part_bytes, offsets + E, stream);
    return rc == kSharedNoSplit ? launch_gemm(KIND_GATE_UP, sh, T, stream) : rc;
  }
  return run_routed_and_shared(KIND_GATE_UP, g, sh, T, stream);
}

int run_down(const void* hq, const float* hs, int64_t T, int64_t H, int64_t I, int E, int k,
             const int32_t* offsets, const int32_t* sorted_slot, const sgl_expert_ptrs* experts,
             int has_shared, int expert_format, int scale_mode, void* out, int* tile_ctr,
             hipStream_t stream) {
  int rc = check_moe_shapes("moe_down", T, H, I, E, k, expert_format);
  if (rc) return rc;
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(hq && hs && offsets && sorted_slot && experts && out, "moe_down: null pointer");
  SGL_REQUIRE(aligned(hq, 16), "moe_down: hq misaligned");
  const bool split = fp4_experts(expert_format);
  const int pow2w = (expert_format & SGL_EXPERT_POW2_SCALES) ? 1 : 0;
  GemmArgs g = {};
  g.a = (const uint8_t*)hq;
  g.sa = hs;
  g.experts = experts;
  g.offsets = offsets;
  g.sorted_slot = sorted_slot;
  g.E = E;
  g.k = k;
  g.has_shared = has_shared && !split ? 1 : 0;
  g.out_k = k + (has_shared ? 1 : 0);
  g.T = T;
  g.N = H;
  g.K = I;
  g.c = out;
  g.wfmt = split ? WF_FP4 : WF_FP8;
  g.sa_pow2 = pow2_scale_mode(scale_mode);
  g.sb_pow2 = split ? 0 : pow2w;
  g.tile_ctr = tile_ctr;
  const sgl_expert_ptrs* frag =
      (expert_format & SGL_EXPERT_FRAG_COPY) ? experts + E + (has_shared ? 1 : 0) : nullptr;
  g.frag = frag;
  if (!split || !has_shared) return launch_gemm(KIND_DOWN, g, T * k / E, stream);
  GemmArgs sh = g;
  sh.E = 0;
  sh.offsets = offsets + E;
  sh.experts = experts + E;
  sh.frag = frag ? frag + E : nullptr;
  sh.has_shared = 1;
  sh.wfmt = WF_FP8;
  sh.sb_pow2 = pow2w;
  sh.tile_ctr = tile_ctr ? tile_ctr + 8 : nullptr;
  return run_routed_and_shared(KIND_DOWN, g, sh, T, stream);
}

int launch_route(const char* what, const float* logits, int64_t T, int E, int k, int score_func,
                 const float* bias, float route_scale, int32_t* ids, float* weights,
                 const HashRoute& hash, hipStream_t st) {
  SGL_REQUIRE(T >= 0, "%s: negative T", what);
  SGL_REQUIRE(E >= 1 && E <= kMaxRouteE, "%s: E=%d not in [1, %d]", what, E, kMaxRouteE);
  SGL_REQUIRE(k >= 1 && k <= 16 && k <= E, "%s: k=%d not in [1, min(16, E)]", what, k);
  SGL_REQUIRE(score_func >= 0 && score_func <= 2, "%s: bad score_func %d", what, score_func);
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(logits && ids && weights, "%s: null pointer", what);
  const unsigned blocks = (unsigned)ceil_div(T, 4);
  const int epl = (E + 63) / 64;
#define SGL_ROUTE(n)                                                                               \
  case n:                                                                                          \
    route_topk_kernel<n><<<blocks, 256, 0, st>>>(logits, T, E, k, score_func, bias, route_scale,  \
                                                 ids, weights, hash);                              \
    break;
  switch (epl) {
    SGL_ROUTE(1) SGL_ROUTE(2) SGL_ROUTE(3) SGL_ROUTE(4) SGL_ROUTE(5) SGL_ROUTE(6) SGL_ROUTE(7)
    default:
      route_topk_kernel<8><<<blocks, 256, 0, st>>>(logits, T, E, k, score_func, bias, route_scale,
                                                   ids, weights, hash);
  }
#undef SGL_ROUTE
  return check_launch(what);
}

}  // namespace
}  // namespace sgl

extern "C" {

int sgl_moe_route_topk(const float* logits, int64_t T, int E, int k, int score_func,
                       const float* bias, float route_scale, int32_t* ids, float* weights,
                       sgl_stream_t stream) {
  return sgl::launch_route("route_topk", logits, T, E, k, score_func, bias, route_scale, ids,
                           weights, sgl::HashRoute{nullptr, nullptr, 0, 0}, (hipStream_t)stream);
}

int sgl_moe_gate(const void* x, const void* w, int64_t T, int64_t H, int E, int k, int score_func,
                 const float* bias, float route_scale, const int32_t* tid2eid, int64_t vocab,
                 const void* input_ids, int input_ids_int64, float* logits, int32_t* ids,
                 float* weights, sgl_stream_t stream) {
  SGL_REQUIRE(T >= 0 && H > 0 && H % 32 == 0, "moe_gate: H=%lld must be a positive multiple of 32",
              (long long)H);
  SGL_REQUIRE(E >= 1 && E <= sgl::kMaxRouteE, "moe_gate: E=%d not in [1, %d]", E, sgl::kMaxRouteE);
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(x && w && logits, "moe_gate: null pointer");
  SGL_REQUIRE(sgl::aligned(x, 16) && sgl::aligned(w, 16), "moe_gate: x and W must be 16-byte aligned");
  SGL_REQUIRE(!tid2eid || (input_ids && vocab >= 1), "moe_gate: hash routing needs input_ids and vocab");
  SGL_REQUIRE(T < ((int64_t)1 << 31) / 16, "moe_gate: T too large");
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  const uint16_t* wb = (const uint16_t*)w;
  // T > 256 with H % 64 == 0: the LDS-staged kernels, the largest of their
  // tiles that still gives about a workgroup per CU; K split over the four
  // wavefronts for the 32 x 64 and 32 x 32 tiles when H % 128 == 0 (H = 4096,
  // E = 256 projection: T = 512 13.0 -> 9.4 us, T = 2048 18.3 -> 15.0 us; for
  // 32 x 128 even, for 64 x 128 31.4 -> 33.6 us, so those keep 2 x 2
  // wavefronts over 64-deep stages).  Decode-sized batches: the
  // register-loaded kernel with 16 tokens x 16 experts per workgroup and 16
  // wavefronts with all their K steps in flight (many small workgroups spread
  // the weight read); it also serves H % 64 != 0 (64 x 64 or 64 x 128 tiles).
  auto tiles = [&](int64_t tt, int64_t te) { return sgl::ceil_div(T, tt) * sgl::ceil_div(E, te); };
  if (T > 256 && H % 128 == 0 && tiles(32, 128) < 240) {
    if (tiles(32, 64) >= 240)
      sgl::launch_router_ks<32, 64, 6>(xb, wb, T, (int)H, E, logits, st);
    else
      sgl::launch_router_ks<32, 32, 8>(xb, wb, T, (int)H, E, logits, st);
  } else if (T > 256 && H % 64 == 0) {
    if (tiles(64, 128) >= 240)
      sgl::launch_router_lds<64, 128, 4>(xb, wb, T, (int)H, E, logits, st);
    else if (tiles(32, 128) >= 240)
      sgl::launch_router_lds<32, 128, 4>(xb, wb, T, (int)H, E, logits, st);
    else if (tiles(32, 64) >= 240)
      sgl::launch_router_lds<32, 64, 6>(xb, wb, T, (int)H, E, logits, st);
    else
      sgl::launch_router_lds<32, 32, 8>(xb, wb, T, (int)H, E, logits, st);
  } else if (T <= 256) {
    dim3 grid((unsigned)E / 16 + (E % 16 != 0), (unsigned)sgl::ceil_div(T, 16));
    sgl::router_logits_kernel<1, 1, 16, 8><<<grid, 1024, 0, st>>>(xb, wb, T, (int)H, E, logits);
  } else if (T >= 4096) {
    dim3 grid((unsigned)sgl::ceil_div((int64_t)E, 128), (unsigned)sgl::ceil_div(T, 64));
    sgl::router_logits_kernel<4, 8, 4, 2><<<grid, 256, 0, st>>>(xb, wb, T, (int)H, E, logits);
  } else {
    dim3 grid((unsigned)sgl::ceil_div((int64_t)E, 64), (unsigned)sgl::ceil_div(T, 64));
    sgl::router_logits_kernel<4, 4, 8, 4><<<grid, 512, 0, st>>>(xb, wb, T, (int)H, E, logits);
  }
  int rc = sgl::check_launch("moe_gate");
  if (rc) return rc;
  return sgl::launch_route("moe_gate", logits, T, E, k, score_func, bias, route_scale, ids, weights,
                           sgl::HashRoute{tid2eid, input_ids, input_ids_int64 ? 1 : 0, vocab}, st);
}

int sgl_moe_permute(const int32_t* ids, int64_t T, int k, int E, int32_t* counts, int32_t* offsets,
                    int32_t* sorted_slot, int32_t* slot_pos, sgl_stream_t stream) {
  return sgl::launch_permute(ids, T, k, E, counts, offsets, sorted_slot, slot_pos, nullptr, 0,
                             (hipStream_t)stream);
}

int sgl_moe_gate_up(const void* xq, const float* xs, int64_t T, int64_t H, int64_t I, int E, int k,
                    const int32_t* offsets, const int32_t* sorted_slot, const float* route_w,
                    const sgl_expert_ptrs* experts, int has_shared, int expert_format,
                    float swiglu_limit, int scale_mode, void* hq, float* hs, sgl_stream_t stream) {
  return sgl::run_gate_up(xq, xs, T, H, I, E, k, offsets, sorted_slot, route_w, experts, has_shared,
                          expert_format, swiglu_limit, scale_mode, hq, hs, nullptr,
                          (hipStream_t)stream);
}

int sgl_moe_down(const void* hq, const float* hs, int64_t T, int64_t H, int64_t I, int E, int k,
                 const int32_t* offsets, const int32_t* sorted_slot,
                 const sgl_expert_ptrs* experts, int has_shared, int expert_format, int scale_mode,
                 void* out, sgl_stream_t stream) {
  return sgl::run_down(hq, hs, T, H, I, E, k, offsets, sorted_slot, experts, has_shared,
                       expert_format, scale_mode, out, nullptr, (hipStream_t)stream);
}

int sgl_moe_combine(const void* out, const int32_t* ids, int64_t T, int k, int64_t H,
                    int has_shared, void* y, sgl_stream_t stream) {
  SGL_REQUIRE(T >= 0 && k >= 1 && k <= 16 && H > 0 && H % 8 == 0, "moe_combine: bad shape");
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(out && ids && y, "moe_combine: null pointer");
  SGL_REQUIRE(sgl::aligned(out, 16) && sgl::aligned(y, 16), "moe_combine: out/y misaligned");
  sgl::launch_combine<false>((const uint16_t*)out, ids, T, k, H, has_shared ? 1 : 0, 0, 0x7FFFFFFF, y,
                             (hipStream_t)stream);
  return sgl::check_launch("moe_combine");
}

size_t sgl_moe_workspace_size(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return sgl::carve(nullptr, T, H, I, E, k, has_shared ? 1 : 0).bytes;
}

int sgl_moe_forward_noalloc(const void* x, int64_t T, int64_t H, int64_t I, int E, int k,
                            const int32_t* ids, const float* weights,
                            const sgl_expert_ptrs* experts, int has_shared, int expert_format,
                            float swiglu_limit, int scale_mode, void* y, sgl_stream_t stream) {
  int rc = sgl::check_moe_shapes("moe_forward_noalloc", T, H, I, E, k, expert_format);
  if (rc) return rc;
  const size_t need = sgl::carve(nullptr, T, H, I, E, k, has_shared ? 1 : 0).bytes;
  if (need > sgl::kScratchBytes) {
    sgl::set_error("moe_forward_noalloc: T=%lld needs %zu bytes of workspace, above the static "
                   "%zu (SGL_MOE_SCRATCH_BYTES); use sgl_moe_forward with a caller workspace",
                   (long long)T, need, sgl::kScratchBytes);
    return SGL_ERR_WORKSPACE;
  }
  if (T == 0) return SGL_OK;
  void* ws = nullptr;
  if ((rc = sgl::moe_scratch_ptr(&ws))) return rc;
  // every buffer the layer reads is written first inside the call (the
  // permute kernel zeroes the GEMM tile counters), so the array needs no clear
  return sgl_moe_forward(x, T, H, I, E, k, ids, weights, experts, has_shared, expert_format,
                         swiglu_limit, scale_mode, ws, sgl::kScratchBytes, y, stream);
}

int sgl_moe_forward(const void* x, int64_t T, int64_t H, int64_t I, int E, int k,
                    const int32_t* ids, const float* weights, const sgl_expert_ptrs* experts,
                    int has_shared, int expert_format, float swiglu_limit, int scale_mode,
                    void* workspace, size_t workspace_bytes, void* y, sgl_stream_t stream) {
  int rc = sgl::check_moe_shapes("moe_forward", T, H, I, E, k, expert_format);
  if (rc) return rc;
  SGL_REQUIRE(scale_mode >= 0 && scale_mode <= 3, "moe_forward: bad scale_mode %d", scale_mode);
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(x && ids && weights && experts && workspace && y, "moe_forward: null pointer");
  has_shared = has_shared ? 1 : 0;
  const sgl::MoeWorkspace w = sgl::carve(workspace, T, H, I, E, k, has_shared);
  if (workspace_bytes < w.bytes) {
    sgl::set_error("moe_forward: workspace %zu bytes < %zu needed", workspace_bytes, w.bytes);
    return SGL_ERR_WORKSPACE;
  }
  SGL_REQUIRE(sgl::aligned(workspace, 256), "moe_forward: workspace must be 256-byte aligned");
  if ((rc = sgl_act_quant(x, T, H, H, w.xq, H, w.xs, H / 128, 128, scale_mode, 0, 0, stream)))
    return rc;
  hipStream_t st = (hipStream_t)stream;
  // the permute also zeroes the GEMMs' tile counters
  if ((rc = sgl::launch_permute(ids, T, k, E, w.counts, w.offsets, w.sorted_slot, w.slot_pos,
                                w.tile_ctr, sgl::kTileCtrs, st)))
    return rc;
  if ((rc = sgl::run_gate_up(w.xq, w.xs, T, H, I, E, k, w.offsets, w.sorted_slot, weights, experts,
                             has_shared, expert_format, swiglu_limit, scale_mode, w.hq, w.hs,
                             w.tile_ctr, st, w.out, w.out_bytes)))
    return rc;
  if ((rc = sgl::run_down(w.hq, w.hs, T, H, I, E, k, w.offsets, w.sorted_slot, experts, has_shared,
                          expert_format, scale_mode, w.out, w.tile_ctr + 16, st)))
    return rc;
  sgl::launch_combine<false>(w.out, ids, T, k, H, has_shared, 0, E, y, st);
  return sgl::check_launch("moe_combine");
}

int sgl_moe_forward_local(const void* x, int64_t T, int64_t H, int64_t I, int E, int k,
                          const int32_t* ids, const float* weights, const sgl_expert_ptrs* experts,
                          int expert_begin, int expert_end, int has_shared, int expert_format,
                          float swiglu_limit, int scale_mode, void* workspace,
                          size_t workspace_bytes, float* y_local, sgl_stream_t stream) {
  int rc = sgl::check_moe_shapes("moe_forward_local", T, H, I, E, k, expert_format);
  if (rc) return rc;
  SGL_REQUIRE(scale_mode >= 0 && scale_mode <= 3, "moe_forward_local: bad scale_mode %d", scale_mode);
  SGL_REQUIRE(0 <= expert_begin && expert_begin <= expert_end && expert_end <= E,
              "moe_forward_local: expert range [%d, %d) not in [0, %d]", expert_begin, expert_end, E);
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(x && ids && weights && experts && workspace && y_local,
              "moe_forward_local: null pointer");
  has_shared = has_shared ? 1 : 0;
  const sgl::MoeWorkspace w = sgl::carve(workspace, T, H, I, E, k, has_shared);
  if (workspace_bytes < w.bytes) {
    sgl::set_error("moe_forward_local: workspace %zu bytes < %zu needed", workspace_bytes, w.bytes);
    return SGL_ERR_WORKSPACE;
  }
  SGL_REQUIRE(sgl::aligned(workspace, 256) && sgl::aligned(y_local, 16),
              "moe_forward_local: workspace must be 256-byte and y_local 16-byte aligned");
  if ((rc = sgl_act_quant(x, T, H, H, w.xq, H, w.xs, H / 128, 128, scale_mode, 0, 0, stream)))
    return rc;
  hipStream_t st = (hipStream_t)stream;
  // only the local experts' slots are placed; offsets[E] counts them, and the
  // shared expert's rows follow them as in the whole layer
  if ((rc = sgl::launch_permute(ids, T, k, E, w.counts, w.offsets, w.sorted_slot, w.slot_pos,
                                w.tile_ctr, sgl::kTileCtrs, st, expert_begin, expert_end)))
    return rc;
  if ((rc = sgl::run_gate_up(w.xq, w.xs, T, H, I, E, k, w.offsets, w.sorted_slot, weights, experts,
                             has_shared, expert_format, swiglu_limit, scale_mode, w.hq, w.hs,
                             w.tile_ctr, st, w.out, w.out_bytes)))
    return rc;
  if ((rc = sgl::run_down(w.hq, w.hs, T, H, I, E, k, w.offsets, w.sorted_slot, experts, has_shared,
                          expert_format, scale_mode, w.out, w.tile_ctr + 16, st)))
    return rc;
  sgl::launch_combine<true>(w.out, ids, T, k, H, has_shared, expert_begin, expert_end, y_local, st);
  return sgl::check_launch("moe_forward_local");
}

int sgl_moe_add_shared(const float* y_local, const void* workspace, size_t workspace_bytes,
                       int64_t T, int64_t H, int64_t I, int E, int k, void* y,
                       sgl_stream_t stream) {
  SGL_REQUIRE(T >= 0 && H > 0 && H % 128 == 0 && I > 0 && E >= 1 && k >= 1 && k <= 16,
              "moe_add_shared: bad shape");
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(y_local && workspace && y, "moe_add_shared: null pointer");
  const sgl::MoeWorkspace w = sgl::carve(const_cast<void*>(workspace), T, H, I, E, k, 1);
  if (workspace_bytes < w.bytes) {
    sgl::set_error("moe_add_shared: workspace %zu bytes < %zu needed", workspace_bytes, w.bytes);
    return SGL_ERR_WORKSPACE;
  }
  SGL_REQUIRE(sgl::aligned(y_local, 16) && sgl::aligned(y, 16),
              "moe_add_shared: y_local and y must be 16-byte aligned");
  int64_t blocks = sgl::ceil_div(T * H / 8, (int64_t)256);
  const int64_t cap = 16 * (int64_t)sgl::device_cu_count();
  if (blocks > cap) blocks = cap;
  sgl::add_shared_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(
      y_local, w.out, T, k, H, (uint16_t*)y);
  return sgl::check_launch("moe_add_shared");
}

}  // extern "C"
