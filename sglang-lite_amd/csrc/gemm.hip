// Block-scaled FP8 (e4m3) GEMMs on gfx950 MFMA: dense, grouped gate/up with
// the fused SwiGLU + 1x128 requant epilogue, and grouped down.
//
// Math (deepseek_infer/kernel.py:203-254): for every 128-deep K block kb
//     P = A[:, kb] . B[:, kb]^T            (one v_mfma_f32_16x16x128_f8f6f4 per
//                                           16x16 output tile: K = 128 exactly)
//     C += P * (sa[m, kb] * sb[n/128, kb]) (fp32 promotion of the block partial)
// so the fp32 partial of each K block is scaled once, as the reference's
// two-accumulator structure does.
//
// Tiling: a workgroup owns a BM x BN output tile and streams K in 128-byte
// steps through a double-buffered LDS stage (A: BM x 128 B, B: BN x 128 B).
// Rows are 128 B = 8 chunks of 16 B, stored with the chunk index XORed by
// (row & 7) so the 16 lanes that read one 16x128 MFMA operand (16 rows, same
// chunk) hit distinct banks.  Each wavefront owns a (BM/WM) x (BN/WN) sub-tile
// of 16x16 MFMA tiles; lane l holds row l%16 and K bytes [32*(l/16), +32) of
// every operand it feeds (A and B use the same K assignment, so the product
// is the full 128-deep dot product whatever order the hardware pairs them in).
//
// MoE tiles: an M tile never straddles two experts.  Wavefront 0 of each
// workgroup turns its linear M-tile index into (expert, first row, rows) with
// a wave-wide prefix sum over ceil(count_e / BM) read from the expert offsets,
// so the grid can be sized from T*k alone and nothing is read back to the host.
#include "sgl_gemm.h"
#include "sgl_numeric.h"

namespace sgl {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ float e8m0_value(uint32_t b) {
  return b == 0xFFu ? bits_f32(0x7FC00000u) : (b == 0 ? bits_f32(0x00400000u) : bits_f32(b << 23));
}

__device__ __forceinline__ float load_scale(const void* s, int64_t idx, int e8m0) {
  if (e8m0) return e8m0_value(reinterpret_cast<const uint8_t*>(s)[idx]);
  return reinterpret_cast<const float*>(s)[idx];
}

__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

struct TileInfo {
  int e;
  int row0;
  int rows;
};

// Executed by wavefront 0 only.  Groups are the E routed experts followed by
// the shared expert (T rows at offsets[E]) when has_shared.
__device__ void resolve_moe_tile(const int32_t* __restrict__ offsets, int E, int has_shared,
                                 int64_t T, int BM, int mt, TileInfo* out) {
  const int lane = threadIdx.x & 63;
  const int G = E + (has_shared ? 1 : 0);
  const int per = (G + 63) / 64;
  int local = 0;
  for (int q = 0; q < per; ++q) {
    const int g = lane * per + q;
    int cnt = 0;
    if (g < E)
      cnt = offsets[g + 1] - offsets[g];
    else if (g == E && has_shared)
      cnt = (int)T;
    local += (cnt + BM - 1) / BM;
  }
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  const int excl = incl - local;
  const bool mine = mt >= excl && mt < incl;
  const unsigned long long mask = __ballot(mine);
  if (lane == 0 && mask == 0ull) out->e = -1;
  if (mine) {
    int start = excl;
    for (int q = 0; q < per; ++q) {
      const int g = lane * per + q;
      const int cnt = g < E ? offsets[g + 1] - offsets[g] : ((g == E && has_shared) ? (int)T : 0);
      const int nt = (cnt + BM - 1) / BM;
      if (mt < start + nt) {
        const int lt = mt - start;
        const int base = g < E ? offsets[g] : offsets[E];
        out->e = g;
        out->row0 = base + lt * BM;
        out->rows = min(BM, cnt - lt * BM);
        break;
      }
      start += nt;
    }
  }
}

template <int KIND, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_fp8_kernel(const GemmArgs args) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / (WM * 16);
  constexpr int TN = BN / (WN * 16);
  constexpr int A_CH = BM * 8 / NT;  // 16-byte chunks each thread moves per K step
  constexpr int B_CH = BN * 8 / NT;
  constexpr int HALF = BN / 2;       // gate_up: gate columns, then the same up columns
  constexpr int HW = HALF / WN;      // gate_up: h columns per wavefront
  static_assert(TM >= 1 && TN >= 1 && A_CH >= 1 && B_CH >= 1, "tile too small for the block");
  static_assert(KIND != KIND_GATE_UP || (TN % 2 == 0 && HALF == 128), "gate_up needs 128 h columns");

  __shared__ __align__(16) uint8_t sA[2][BM * 128];
  __shared__ __align__(16) uint8_t sB[2][BN * 128];
  __shared__ float sSa[2][BM];
  __shared__ int sSrc[BM];
  __shared__ int sDst[BM];
  __shared__ float sW[BM];
  __shared__ TileInfo sTile;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int mt = (int)(blockIdx.x / (unsigned)args.n_tiles);
  const int nt = (int)(blockIdx.x % (unsigned)args.n_tiles);
  const int64_t K = args.K, N = args.N;
  const int KB = (int)(K / 128);

  // ---- which rows this tile covers
  int e = 0, row0 = 0, rows = 0;
  int64_t shared_base = 0;
  if constexpr (KIND == KIND_DENSE) {
    row0 = mt * BM;
    rows = (int)min((int64_t)BM, args.M - row0);
    if (rows <= 0) return;
  } else {
    if (wave == 0) resolve_moe_tile(args.offsets, args.E, args.has_shared, args.T, BM, mt, &sTile);
    __syncthreads();
    e = sTile.e;
    if (e < 0) return;
    row0 = sTile.row0;
    rows = sTile.rows;
    shared_base = args.offsets[args.E];
  }
  for (int i = tid; i < BM; i += NT) {
    int src = -1, dst = -1;
    float w = 1.0f;
    if (i < rows) {
      const int p = row0 + i;
      if constexpr (KIND == KIND_DENSE) {
        src = p;
        dst = p;
      } else if (e < args.E) {
        const int slot = args.sorted_slot[p];
        const int t = slot / args.k;
        const int j = slot - t * args.k;
        if constexpr (KIND == KIND_GATE_UP) {
          src = t;
          dst = p;
          if (args.route_w) w = args.route_w[slot];
        } else {
          src = p;
          dst = t * (args.k + args.has_shared) + j;
        }
      } else {
        const int t = p - (int)shared_base;
        if constexpr (KIND == KIND_GATE_UP) {
          src = t;
          dst = p;
        } else {
          src = p;
          dst = t * (args.k + 1) + args.k;
        }
      }
    }
    sSrc[i] = src;
    sDst[i] = dst;
    sW[i] = w;
  }
  __syncthreads();

  // ---- operand sources
  const uint8_t* b0;
  const uint8_t* b1 = nullptr;
  const void* sb0;
  const void* sb1 = nullptr;
  int sb_e8m0 = 0;
  int64_t n0;
  if constexpr (KIND == KIND_DENSE) {
    b0 = args.b;
    sb0 = args.sb;
    sb_e8m0 = args.sb_e8m0;
    n0 = (int64_t)nt * BN;
  } else if constexpr (KIND == KIND_GATE_UP) {
    const sgl_expert_ptrs ex = args.experts[e];
    b0 = reinterpret_cast<const uint8_t*>(ex.w_gate);
    b1 = reinterpret_cast<const uint8_t*>(ex.w_up);
    sb0 = ex.s_gate;
    sb1 = ex.s_up;
    n0 = (int64_t)nt * HALF;
  } else {
    const sgl_expert_ptrs ex = args.experts[e];
    b0 = reinterpret_cast<const uint8_t*>(ex.w_down);
    sb0 = ex.s_down;
    n0 = (int64_t)nt * BN;
  }
  const int64_t sb_row = (n0 / 128) * KB;

  // Every lane always loads from a valid address (a row of this tile) and
  // zeroes what it loaded for rows outside the tile, so the loads stay plain
  // global loads with no pointer select.
  const uint8_t* pa[A_CH];
  int la[A_CH];
  unsigned amask = 0u;
  const int src0 = sSrc[0];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c >> 3, ch = c & 7;
    const int src = sSrc[r];
    if (src >= 0) amask |= 1u << i;
    pa[i] = args.a + (int64_t)(src >= 0 ? src : src0) * K + ch * 16;
    la[i] = swz(r, ch);
  }
  const uint8_t* pb[B_CH];
  int lb[B_CH];
  unsigned bmask = 0u;
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c >> 3, ch = c & 7;
    const bool up_half = KIND == KIND_GATE_UP && r >= HALF;
    const int64_t n = n0 + (up_half ? r - HALF : r);
    if (n < N) bmask |= 1u << i;
    pb[i] = (up_half ? b1 : b0) + (n < N ? n : n0) * K + ch * 16;
    lb[i] = swz(r, ch);
  }
  const int my_src = tid < BM ? sSrc[tid] : -1;
  const int64_t my_sa_row = (int64_t)(my_src >= 0 ? my_src : src0) * KB;

  uint4 ra[A_CH], rb[B_CH];
  float rsa = 0.0f;

#define SGL_GLOAD(kb_)                                                                   \
  do {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i) {                                   \
      const uint4 v = *reinterpret_cast<const uint4*>(pa[i] + (kb_) * 128);              \
      const bool ok = (amask >> i) & 1u;                                                 \
      ra[i] = make_uint4(ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u);     \
    }                                                                                    \
    _Pragma("unroll") for (int i = 0; i < B_CH; ++i) {                                   \
      const uint4 v = *reinterpret_cast<const uint4*>(pb[i] + (kb_) * 128);              \
      const bool ok = (bmask >> i) & 1u;                                                 \
      rb[i] = make_uint4(ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u);     \
    }                                                                                    \
    if (tid < BM) {                                                                      \
      const float sv = load_scale(args.sa, my_sa_row + (kb_), args.sa_e8m0);             \
      rsa = my_src >= 0 ? sv : 0.0f;                                                     \
    }                                                                                    \
  } while (0)
#define SGL_SSTORE(st_)                                                                  \
  do {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i)                                     \
        *reinterpret_cast<uint4*>(&sA[(st_)][la[i]]) = ra[i];                            \
    _Pragma("unroll") for (int i = 0; i < B_CH; ++i)                                     \
        *reinterpret_cast<uint4*>(&sB[(st_)][lb[i]]) = rb[i];                            \
    if (tid < BM) sSa[(st_)][tid] = rsa;                                                 \
  } while (0)

  const int wm = wave / WN, wn = wave % WN;
  const int g4 = lane >> 4, r16 = lane & 15;
  auto tile_col = [&](int nj) -> int {
    if constexpr (KIND == KIND_GATE_UP) {
      return nj < TN / 2 ? wn * HW + nj * 16 : HALF + wn * HW + (nj - TN / 2) * 16;
    } else {
      return (wn * TN + nj) * 16;
    }
  };

  v4f acc[TM][TN];
#pragma unroll
  for (int mi = 0; mi < TM; ++mi)
#pragma unroll
    for (int nj = 0; nj < TN; ++nj) acc[mi][nj] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const v4f vzero = {0.0f, 0.0f, 0.0f, 0.0f};

  SGL_GLOAD(0);
  SGL_SSTORE(0);
  __syncthreads();

  for (int kb = 0; kb < KB; ++kb) {
    const int st = kb & 1;
    if (kb + 1 < KB) SGL_GLOAD(kb + 1);
    const float sbv0 = load_scale(sb0, sb_row + kb, sb_e8m0);
    const float sbv1 = KIND == KIND_GATE_UP ? load_scale(sb1, sb_row + kb, 0) : 0.0f;

    v8i af[TM];
    float sav[TM][4];
#pragma unroll
    for (int mi = 0; mi < TM; ++mi) {
      const int row = (wm * TM + mi) * 16 + r16;
      const uint4 lo = *reinterpret_cast<const uint4*>(&sA[st][swz(row, 2 * g4)]);
      const uint4 hi = *reinterpret_cast<const uint4*>(&sA[st][swz(row, 2 * g4 + 1)]);
      af[mi] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                   (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) sav[mi][r] = sSa[st][(wm * TM + mi) * 16 + 4 * g4 + r];
    }
#pragma unroll
    for (int nj = 0; nj < TN; ++nj) {
      const int col = tile_col(nj) + r16;
      const uint4 lo = *reinterpret_cast<const uint4*>(&sB[st][swz(col, 2 * g4)]);
      const uint4 hi = *reinterpret_cast<const uint4*>(&sB[st][swz(col, 2 * g4 + 1)]);
      const v8i bf = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                         (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      const float sbv = (KIND == KIND_GATE_UP && nj >= TN / 2) ? sbv1 : sbv0;
#pragma unroll
      for (int mi = 0; mi < TM; ++mi) {
        const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[mi], bf, vzero, 0, 0, 0,
                                                                        0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mi][nj][r] = fmaf(p[r], sav[mi][r] * sbv, acc[mi][nj][r]);
      }
    }
    if (kb + 1 < KB) SGL_SSTORE(st ^ 1);
    __syncthreads();
  }

  if constexpr (KIND != KIND_GATE_UP) {
    // ---- bf16 / fp32 output rows
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = (wm * TM + mi) * 16 + 4 * g4 + r;
        const bool row_ok = row < rows;
        const int64_t dst = row_ok ? sDst[row] : 0;
#pragma unroll
        for (int nj = 0; nj < TN; ++nj) {
          const int64_t col = n0 + tile_col(nj) + r16;
          const float v = acc[mi][nj][r];
          if (row_ok && col < N) {
            if (KIND == KIND_DENSE && args.out_f32)
              reinterpret_cast<float*>(args.c)[dst * N + col] = v;
            else
              reinterpret_cast<uint16_t*>(args.c)[dst * N + col] = f32_to_bf16(v);
          }
        }
      }
  } else {
    // ---- SwiGLU epilogue: h = bf16(silu(bf16(gate)) * bf16(up) * w), staged in
    // LDS as bf16 [BM][128], then 1x128 requant of each row (16 lanes per row).
    uint16_t* hbuf = reinterpret_cast<uint16_t*>(&sB[0][0]);
    const float lim = args.swiglu_limit;
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = (wm * TM + mi) * 16 + 4 * g4 + r;
        const float w = sW[row];
#pragma unroll
        for (int j = 0; j < TN / 2; ++j) {
          float gt = bf16r(acc[mi][j][r]);
          float up = bf16r(acc[mi][j + TN / 2][r]);
          if (lim > 0.0f) {
            up = clampf_(up, -lim, lim);
            gt = gt > lim ? lim : gt;
          }
          const float silu = gt / (1.0f + expf(-gt));
          const float h = w * (silu * up);
          hbuf[row * HALF + wn * HW + j * 16 + r16] = f32_to_bf16(h);
        }
      }
    __syncthreads();
    constexpr int LPR = HALF / 8;  // 16 lanes per 128-column row
    static_assert((BM * LPR) % NT == 0, "requant loop must be uniform");
    const int64_t NB = N / 128;
#pragma unroll
    for (int it = 0; it < BM * LPR / NT; ++it) {
      const int task = tid + it * NT;
      const int row = task / LPR, sub = task % LPR;
      const uint4 v = *reinterpret_cast<const uint4*>(hbuf + row * HALF + sub * 8);
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
      float f[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = bits_f32(wv[i] << 16);
        f[2 * i + 1] = bits_f32(wv[i] & 0xFFFF0000u);
      }
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf_(amax, fabsf(f[i]));
#pragma unroll
      for (int o = LPR / 2; o > 0; o >>= 1) amax = fmaxf_(amax, __shfl_xor(amax, o, 64));
      if (row < rows) {
        const float sf = group_scale(args.scale_mode, amax);
        const float inv = 1.0f / sf;
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo |= (uint32_t)quant_elem(args.scale_mode, f[i], sf, inv) << (8 * i);
          hi |= (uint32_t)quant_elem(args.scale_mode, f[i + 4], sf, inv) << (8 * i);
        }
        const int64_t p = row0 + row;
        *reinterpret_cast<uint2*>(args.hq + p * N + n0 + sub * 8) = make_uint2(lo, hi);
        if (sub == 0) args.hs[p * NB + n0 / 128] = sf;
      }
    }
  }
}

#undef SGL_GLOAD
#undef SGL_SSTORE

template <int KIND, int BM, int BN, int WM, int WN>
int launch_cfg(GemmArgs& a, hipStream_t stream) {
  const int64_t half = KIND == KIND_GATE_UP ? BN / 2 : BN;
  a.n_tiles = (int)ceil_div(a.N, half);
  if constexpr (KIND == KIND_DENSE) {
    a.m_tiles = (int)ceil_div(a.M, BM);
  } else {
    const int64_t P = a.T * a.k;
    int64_t mt = P / BM + (P < a.E ? P : a.E) + 1;
    if (a.has_shared) mt += ceil_div(a.T, BM);
    a.m_tiles = (int)mt;
  }
  const int64_t blocks = (int64_t)a.m_tiles * a.n_tiles;
  if (blocks == 0) return SGL_OK;
  if (blocks > 0x7FFFFFFF) {
    set_error("gemm: grid of %lld blocks too large", (long long)blocks);
    return SGL_ERR_UNSUPPORTED;
  }
  gemm_fp8_kernel<KIND, BM, BN, WM, WN><<<(unsigned)blocks, 64 * WM * WN, 0, stream>>>(a);
  return check_launch("gemm_fp8");
}

}  // namespace

int launch_gemm(int kind, GemmArgs& a, int64_t rows_hint, hipStream_t stream) {
  const bool big = rows_hint >= 64;
  switch (kind) {
    case KIND_DENSE:
      return big ? launch_cfg<KIND_DENSE, 128, 128, 2, 2>(a, stream)
                 : launch_cfg<KIND_DENSE, 32, 128, 1, 2>(a, stream);
    case KIND_GATE_UP:
      return big ? launch_cfg<KIND_GATE_UP, 128, 256, 2, 4>(a, stream)
                 : launch_cfg<KIND_GATE_UP, 32, 256, 1, 4>(a, stream);
    default:
      return big ? launch_cfg<KIND_DOWN, 128, 128, 2, 2>(a, stream)
                 : launch_cfg<KIND_DOWN, 32, 128, 1, 2>(a, stream);
  }
}

}  // namespace sgl

extern "C" int sgl_fp8_gemm(const void* a, const void* sa, int a_scale_e8m0, const void* b,
                            const void* sb, int b_scale_e8m0, void* c, int out_dtype, int64_t M,
                            int64_t N, int64_t K, sgl_stream_t stream) {
  SGL_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fp8_gemm: negative shape");
  SGL_REQUIRE(out_dtype == SGL_BF16 || out_dtype == SGL_F32, "fp8_gemm: out_dtype must be bf16/f32");
  SGL_REQUIRE(K % 128 == 0, "fp8_gemm: K=%lld must be a multiple of 128", (long long)K);
  SGL_REQUIRE(N % 16 == 0, "fp8_gemm: N=%lld must be a multiple of 16", (long long)N);
  if (M == 0 || N == 0) return SGL_OK;
  SGL_REQUIRE(a && sa && b && sb && c, "fp8_gemm: null pointer");
  SGL_REQUIRE(sgl::aligned(a, 16) && sgl::aligned(b, 16),
              "fp8_gemm: A and B must be 16-byte aligned");
  SGL_REQUIRE(a_scale_e8m0 || sgl::aligned(sa, 4), "fp8_gemm: fp32 sa must be 4-byte aligned");
  SGL_REQUIRE(b_scale_e8m0 || sgl::aligned(sb, 4), "fp8_gemm: fp32 sb must be 4-byte aligned");
  sgl::GemmArgs g = {};
  g.a = (const uint8_t*)a;
  g.sa = sa;
  g.sa_e8m0 = a_scale_e8m0;
  g.b = (const uint8_t*)b;
  g.sb = sb;
  g.sb_e8m0 = b_scale_e8m0;
  g.M = M;
  g.N = N;
  g.K = K;
  g.c = c;
  g.out_f32 = out_dtype == SGL_F32;
  return sgl::launch_gemm(sgl::KIND_DENSE, g, M, (hipStream_t)stream);
}
