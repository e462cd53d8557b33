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
// Data movement: operand tiles go global -> LDS with global_load_lds_dwordx4
// (each lane moves 16 bytes straight into LDS, no register staging) through
// an NSTAGE-deep ring of LDS stages.  One 1 KB DMA instruction fills 8 rows x
// 128 bytes of a stage; a row's 16-byte chunk c is stored at c ^ swz(row) with
// swz(row) = (row & 6) | ((row >> 3) & 1).  A ds_read_b128 of an MFMA operand
// has 16 lanes read one chunk column of 16 consecutive rows; with this swizzle
// those reads are conflict-free on gfx950's 64-bank LDS (measured: 4 LDS
// cycles per wavefront read, like a contiguous 1 KB read; the plain
// (row >> 1) & 7 rotation measures 8, two-way conflicted).  The swizzle is
// applied to each lane's global address, so the DMA keeps reading whole
// 128-byte row segments.  The
// waits are explicit s_waitcnt vmcnt(n) counts plus a bare s_barrier, so
// NSTAGE-1 stages of loads stay in flight while the MFMAs run.
//
// Work split: a workgroup of WM x WN wavefronts owns a BM x BN tile; each
// wavefront a (BM/WM) x (BN/WN) block of 16x16 MFMA tiles (lane l holds row
// l%16 and K bytes [32*(l/16), +32) of every operand; A and B use the same K
// assignment, so the product is the full 128-deep dot product).  A
// wavefront whose rows lie wholly past the tile's last row skips its MFMAs.
// The kernel is persistent: each workgroup walks the tiles assigned to its
// XCD (workgroup b runs on XCD b % 8) in a contiguous range, expert-major with
// the M tiles of one N slice adjacent, so the tiles sharing a weight slice or
// an activation block run close together on one XCD's L2.
//
// MoE tiles: an M tile never straddles two experts.  The workgroup first
// prefix-sums ceil(count_e / BM) over the expert offsets into LDS, so the
// grid is sized without reading routing data on the host.
#include <algorithm>
#include <type_traits>

#include "sgl_gemm.h"
#include "sgl_numeric.h"

namespace sgl {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kMaxGroups = 1025;  // 1024 routed experts + shared

// nontemporal loads for the weight streams that are read once per launch
#ifndef SGL_NT_WEIGHTS
#define SGL_NT_WEIGHTS 1
#endif
// MoE tiles of one wavefront row: compute only the 16-row blocks a group fills
#ifndef SGL_DEAD_SKIP
#define SGL_DEAD_SKIP 1
#endif

constexpr int kMaxKB = 128;       // K <= 16384: weight scales of a tile staged in LDS

__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// Lane i of the wavefront copies 16 bytes from base + voff to LDS m0 + 16 i.
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(lds) : "memory");
}
// dma16 with the nontemporal cache policy: for operand bytes read once per
// launch (a nontemporal read stream on gfx950 moves 7.0 TB/s, a plain one 6.2)
__device__ __forceinline__ void dma16nt(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
               :: "v"(voff), "s"(base), "s"(lds) : "memory");
}
// Lane i copies 4 bytes from base + voff to LDS m0 + 4 i.
__device__ __forceinline__ void dma4(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(base), "s"(lds) : "memory");
}

// The same with a per-lane 64-bit address (no scalar base): lane i copies 4
// bytes from addr to LDS m0 + 4 i (dma16v, 16 bytes, is in sgl_common.h).
__device__ __forceinline__ void dma4v(uint64_t addr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(addr), "s"(lds) : "memory");
}


template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" :: "n"(N) : "memory");
}

__device__ __forceinline__ float e8m0_value(uint32_t b) {
  return b == 0xFFu ? bits_f32(0x7FC00000u) : (b == 0 ? bits_f32(0x00400000u) : bits_f32(b << 23));
}



__device__ __forceinline__ float load_scale(const void* s, int64_t idx, int e8m0) {
  if (e8m0) return e8m0_value(reinterpret_cast<const uint8_t*>(s)[idx]);
  return reinterpret_cast<const float*>(s)[idx];
}

// Lane l's two 16-byte chunks of a 16-row operand block: row l % 16, logical
// chunks 2 (l / 16) and 2 (l / 16) + 1.  Blocks start at multiples of 16 rows,
// where the swizzle repeats, so the lane's byte offsets inside any block are
// the same two numbers; the block's own offset (row0 * 128) is a constant.
struct FragLane {
  uint32_t lo, hi;
};
__device__ __forceinline__ FragLane frag_lane(int r16, int g4) {
  return FragLane{(uint32_t)(r16 * 128 + (((2 * g4) ^ swz(r16)) << 4)),
                  (uint32_t)(r16 * 128 + (((2 * g4 + 1) ^ swz(r16)) << 4))};
}
// With a packed e2m1 B operand the MFMA pairs A's K differently: lane l
// holds A bytes [16 (l/16), +16) and [64 + 16 (l/16), +16) of its row, i.e.
// logical chunks l/16 and 4 + l/16 (B lane l holds K [32 (l/16), +32) of its
// column as 16 packed bytes).
__device__ __forceinline__ FragLane frag_lane_fp4a(int r16, int g4) {
  return FragLane{(uint32_t)(r16 * 128 + ((g4 ^ swz(r16)) << 4)),
                  (uint32_t)(r16 * 128 + (((4 + g4) ^ swz(r16)) << 4))};
}
__device__ __forceinline__ v8i read_frag(const uint8_t* block, FragLane fl) {
  const uint4 lo = *reinterpret_cast<const uint4*>(block + fl.lo);
  const uint4 hi = *reinterpret_cast<const uint4*>(block + fl.hi);
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

template <int KIND, int BM, int BN, int WM, int WN, int NSTAGE, int WF, bool SAHW, int LW>
struct Cfg {
  // LW > 0: LW loader wavefronts (after the WM x WN compute wavefronts) issue
  // every stage DMA and compute nothing, so no compute wavefront ever stalls
  // behind the CU's address unit; LW == 0: the DMAs are issued by compute
  // wavefronts (with 8, by the second half, one per SIMD)
  static constexpr int NWC = WM * WN;        // compute wavefronts
  static constexpr int NW = NWC + LW;        // all wavefronts
  static constexpr int NT = 64 * NW;
  static constexpr int TM = BM / (WM * 16);
  static constexpr int TN = BN / (WN * 16);
  static constexpr int HALF = BN / 2;   // gate_up: gate columns, then the same up columns
  static constexpr int HW = HALF / WN;  // gate_up: h columns per wavefront
  // 128-deep K steps per stage: a stage always holds 128-byte B rows, which
  // is 128 K of e4m3 or 256 K of packed e2m1
  static constexpr int KS = WF == WF_FP4 ? 2 : 1;
  static constexpr int A_BYTES = BM * 128 * KS;  // KS sub-blocks of BM x 128 bytes
  static constexpr int B_BYTES = BN * 128;
  static constexpr int SB_BYTES = WF == WF_FP4 ? BN * 8 : 0;  // e8m0 weight scales: 8 per column
  // DMA issuers: with 8 wavefronts (two per SIMD) only the second half, one
  // wavefront per SIMD, issues a stage's loads; the first half starts its
  // MFMAs right after the stage barrier instead of queueing behind the CU's
  // address unit with every other wavefront
  static constexpr int IW = LW > 0 ? LW : (NWC == 8 ? NWC / 2 : NWC);
  static constexpr int SBI = SB_BYTES / (IW * 256);  // weight-scale dword DMAs per issuer
  static constexpr int SA_ROWS = BM / NWC;  // row scales per compute wavefront slot per stage
  static constexpr int STAGE = A_BYTES + B_BYTES + SB_BYTES;
  static constexpr int SA_SLOT = NWC * 256;          // one stage of row scales
  static constexpr int ACH = BM * KS / 8;            // 1 KB DMA chunks of A per stage
  static constexpr int CHUNKS = ACH + BN / 8;        // ... of A and B
  static constexpr int CPW = CHUNKS / IW;       // per issuer
  static constexpr int SAI = NWC / IW;          // row-scale DMAs per issuer (one per slot)
  static constexpr int QA = BM / 8 / IW;        // distinct A row groups per issuer
  static constexpr int LPS = CPW + SAI + SBI;   // DMA instructions per issuer per stage
  static constexpr int NSA = NSTAGE;  // row-scale slots (a ring of their own)
  static constexpr int RING = NSTAGE * STAGE;
  static constexpr int SMEM = RING + NSA * SA_SLOT;
  static_assert(CHUNKS % IW == 0, "chunks must split evenly over the issuers");
  static_assert(NWC % IW == 0, "row-scale slots must split evenly over the issuers");
  static_assert(IW % 2 == 0 && (BM / 8) % IW == 0 && (HALF / 8) % IW == 0,
                "every chunk index of an issuer maps to one operand, half and swizzle parity");
  static_assert(SA_ROWS >= 1 && SA_ROWS * KS <= 64, "row scales per wavefront");
  static_assert(SB_BYTES % (IW * 256) == 0, "weight-scale DMAs must split evenly");
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  static_assert(KIND != KIND_GATE_UP || (TN % 2 == 0 && HALF == 128), "gate_up needs 128 h columns");
  static_assert(LW > 0 || (KIND == KIND_GATE_UP ? BM * HALF * 2 <= RING : BM * BN * 4 <= RING),
                "epilogue staging must fit in the stage ring");
  static_assert(NSTAGE >= 2 && NSTAGE <= 6, "stages");
  static_assert(WF == WF_FP4 || !SAHW || KIND == KIND_DENSE, "e8m0 activation scales: dense only");
};

template <int KIND, int BM, int BN, int WM, int WN, int NSTAGE, int WF, bool SAHW, int LW>
__global__ __launch_bounds__(64 * (WM * WN + LW)) void gemm_fp8_kernel(const GemmArgs args) {
  using C = Cfg<KIND, BM, BN, WM, WN, NSTAGE, WF, SAHW, LW>;
  constexpr int NT = C::NT, NW = C::NW, NWC = C::NWC, TM = C::TM, TN = C::TN, HALF = C::HALF,
                HW = C::HW;
  constexpr int KS = C::KS;
  constexpr bool FP4 = WF == WF_FP4;
  // SAHW: FP4 weights, power-of-two row scales applied inside the MFMA
  // (fp32, or e8m0 bytes when sa_e8m0); FP8 weights (dense), e8m0 row scales
  // as bytes, with e8m0 weight scales both applied inside the MFMA, else
  // promoted in fp32.  The other instantiations read fp32 row scales.
  const int sa_e8 = (KIND == KIND_DENSE && SAHW) ? (FP4 ? args.sa_e8m0 : 1) : 0;
  const bool pow2 = KIND == KIND_DENSE && !FP4 && SAHW && args.sb_e8m0;

  __shared__ __align__(16) uint8_t smem[C::SMEM];
  __shared__ int sTstart[KIND == KIND_DENSE ? 1 : kMaxGroups + 1];
  __shared__ int sSrc[BM];
  __shared__ int sDst[BM];
  __shared__ float sW[BM];
  __shared__ float sSb[2][FP4 ? 1 : kMaxKB];  // fp8: the tile's weight scales per K block
  // register epilogue of gate/up (LW > 0): each compute wavefront's row |h| maximum
  __shared__ float sAmax[KIND == KIND_GATE_UP && LW > 0 ? WN : 1][KIND == KIND_GATE_UP && LW > 0 ? BM : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool computes = LW == 0 || wave < NWC;  // loader wavefronts (LW > 0) compute nothing
  const int wm = computes ? wave / WN : 0, wn = computes ? wave % WN : 0;
  const int g4 = lane >> 4, r16 = lane & 15;
  const FragLane fl = frag_lane(r16, g4);
  const FragLane fla = FP4 ? frag_lane_fp4a(r16, g4) : fl;
  const int64_t K = args.K, N = args.N;
  const int64_t KROW = FP4 ? K / 2 : K;  // bytes per B row
  const int KB = (int)(K / 128);
  const int NST = KB / KS;  // stages along K
  const int n_tiles = args.n_tiles;

  // ---- M-tile prefix over the expert groups (E routed, then the shared one)
  int G = 0, total_mt;
  int64_t shared_base = 0;
  if constexpr (KIND == KIND_DENSE) {
    total_mt = (int)((args.M + BM - 1) / BM);
  } else {
    G = args.E + (args.has_shared ? 1 : 0);
    shared_base = args.offsets[args.E];
    if (wave == 0) {
      int carry = 0;
      if (lane == 0) sTstart[0] = 0;
      for (int base = 0; base < G; base += 64) {
        const int g = base + lane;
        int cnt = 0;
        if (g < args.E)
          cnt = args.offsets[g + 1] - args.offsets[g];
        else if (g < G)
          cnt = (int)args.T;
        const int v = (cnt + BM - 1) / BM;
        int incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int u = __shfl_up(incl, o, 64);
          if (lane >= o) incl += u;
        }
        if (g < G) sTstart[g + 1] = carry + incl;
        carry += __shfl(incl, 63, 64);
      }
    }
    __syncthreads();
    total_mt = sTstart[G];
  }
  const int total = total_mt * n_tiles;
  const int nwg = gridDim.x;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per_xcd = nwg >> 3;
  const int per = (total + 7) >> 3;
  const int t_begin = xcd * per;
  const int t_end = min(t_begin + per, total);

  // Static order: slot s of an XCD takes tiles s, s + per_xcd, ...  With
  // tile counters the workgroups of an XCD take the next tile when they
  // finish one, so tiles that are adjacent in the order (the M tiles sharing
  // a weight slice) start together even when tile costs differ.
  __shared__ int sNext;
  for (int iter = 0;; ++iter) {
    int local;
    if (args.tile_ctr) {
      if (tid == 0) sNext = atomicAdd(&args.tile_ctr[xcd], 1);
      __syncthreads();
      local = __builtin_amdgcn_readfirstlane(sNext);
    } else {
      local = slot + iter * per_xcd;
    }
    const int L = t_begin + local;
    if (L >= t_end) break;
    // ---- resolve the tile: group g, its M tile mt, N tile nt (M tiles adjacent)
    int e = 0, row0, rows, nt;
    if constexpr (KIND == KIND_DENSE) {
      nt = L / total_mt;
      const int mt = L - nt * total_mt;
      row0 = mt * BM;
      rows = (int)min((int64_t)BM, args.M - row0);
    } else {
      int lo = 0, hi = G;  // find g: sTstart[g]*n_tiles <= L < sTstart[g+1]*n_tiles
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (sTstart[mid] * n_tiles <= L) lo = mid; else hi = mid;
      }
      e = lo;
      const int m_in_g = sTstart[e + 1] - sTstart[e];
      const int local = L - sTstart[e] * n_tiles;
      nt = local / m_in_g;
      const int mt = local - nt * m_in_g;
      const int cnt = e < args.E ? args.offsets[e + 1] - args.offsets[e] : (int)args.T;
      const int base = e < args.E ? args.offsets[e] : (int)shared_base;
      row0 = base + mt * BM;
      rows = min(BM, cnt - mt * BM);
    }
    e = __builtin_amdgcn_readfirstlane(e);
    nt = __builtin_amdgcn_readfirstlane(nt);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    rows = __builtin_amdgcn_readfirstlane(rows);
    // ---- operand bases (wave-uniform) and per-lane DMA offsets
    const uint8_t* baseA = uniform_ptr(args.a);
    const uint8_t* b0;
    const uint8_t* b1 = nullptr;
    const void* sb0;
    const void* sb1 = nullptr;
    int sb_e8m0 = 0;
    int64_t n0;
    if constexpr (KIND == KIND_DENSE) {
      b0 = uniform_ptr(args.b);
      sb0 = args.sb;
      sb_e8m0 = args.sb_e8m0;
      n0 = (int64_t)nt * BN;
    } else if constexpr (KIND == KIND_GATE_UP) {
      const sgl_expert_ptrs* ex = args.experts + e;
      b0 = uniform_ptr(ex->w_gate);
      b1 = uniform_ptr(ex->w_up);
      sb0 = uniform_ptr(ex->s_gate);
      sb1 = uniform_ptr(ex->s_up);
      n0 = (int64_t)nt * HALF;
    } else {
      const sgl_expert_ptrs* ex = args.experts + e;
      b0 = uniform_ptr(ex->w_down);
      sb0 = uniform_ptr(ex->s_down);
      n0 = (int64_t)nt * BN;
    }
    // weight-scale row: gate_up tiles are 128 columns per half; dense / down
    // tiles span BN/128 scale blocks, one per wavefront column group
    // (TN*16 <= 128 columns), clamped for a ragged last tile
    const int64_t sb_blk = n0 / 128;
    static_assert(FP4 || KIND == KIND_GATE_UP ||
                      (TN * 16 <= 128 && 128 % (TN * 16) == 0 && BN <= 256),
                  "a wavefront's columns must sit in one 128-column scale block");
    const int wave_blk = KIND == KIND_GATE_UP ? 0 : (wn * TN * 16) / 128;
    // fp8: the tile's weight scales -> LDS (row 0: gate / first block, row 1:
    // up / second block), so the K loop issues no vector loads besides the
    // DMAs; fp4 weight scales travel with each stage
    for (int i = tid; i < (FP4 ? 0 : 2 * KB); i += NT) {
      const int j = i / KB, kb = i - j * KB;
      float v;
      if constexpr (KIND == KIND_GATE_UP) {
        v = load_scale(j ? sb1 : sb0, sb_blk * KB + kb, 0);
      } else {
        const int64_t nb = (N + 127) / 128;
        int64_t blk = n0 / 128 + j;
        if (blk > nb - 1) blk = nb - 1;
        v = load_scale(sb0, blk * KB + kb, sb_e8m0);
      }
      sSb[j][kb] = v;
    }
    // ---- per-row tables
    for (int i = tid; i < BM; i += NT) {
      int src = -1, dst = -1;
      float w = 1.0f;
      if (i < rows) {
        const int p = row0 + i;
        if constexpr (KIND == KIND_DENSE) {
          src = p;
          dst = p;
        } else if (e < args.E) {
          const int sl = args.sorted_slot[p];
          const int t = sl / args.k;
          const int j = sl - t * args.k;
          if constexpr (KIND == KIND_GATE_UP) {
            src = t;
            dst = p;
            if (args.route_w) w = args.route_w[sl];
          } else {
            src = p;
            dst = t * args.out_k + j;
          }
        } else {
          const int t = p - (int)shared_base;
          if constexpr (KIND == KIND_GATE_UP) {
            src = t;
            dst = p;
          } else {
            src = p;
            dst = t * args.out_k + args.k;
          }
        }
      }
      sSrc[i] = src;
      sDst[i] = dst;
      sW[i] = w;
    }
    __syncthreads();

    const int src0 = __builtin_amdgcn_readfirstlane(sSrc[0]);

    // Issuer iw (wavefront NW - IW + iw) moves chunks c = iw + j * IW of
    // every stage, A's first: A chunk c holds rows [8c', 8c'+8) of K
    // sub-block c / (BM/8) (c' = c % (BM/8)), its lane offsets one register
    // per distinct c' (the sub-block adds 128 bytes); B chunk b = c - ACH
    // holds weight rows [8b, 8b+8).  Since IW is even, every B chunk of an
    // issuer has the same swizzle parity (b & 1 = iw & 1), so the B lane
    // offset is one register plus a wave-uniform row base.  The other
    // wavefronts issue nothing (their offsets are issuer 0's, never used).
    const bool issuer = wave >= NW - C::IW;  // the loaders, or the last IW compute wavefronts
    const int iw = issuer ? wave - (NW - C::IW) : 0;
    const int rr = lane >> 3, pc = lane & 7;
    uint32_t voffA[C::QA];
#pragma unroll
    for (int q = 0; q < C::QA; ++q) {
      const int r = (iw + q * C::IW) * 8 + rr;
      const int s = sSrc[r] >= 0 ? sSrc[r] : src0;
      voffA[q] = (uint32_t)((int64_t)s * K + ((pc ^ swz(r)) << 4));
    }
    const uint32_t chunkB = (uint32_t)((pc ^ ((rr & 6) | (iw & 1))) << 4);
    const uint32_t laneB = (uint32_t)(rr * KROW) + chunkB;
    const uint32_t clampB = (uint32_t)(n0 * KROW) + chunkB;  // rows past N re-read row n0
    // row scales of wavefront w = iw + q IW (its 256-byte slot): lane l <
    // KS * SA_ROWS loads row w * SA_ROWS + l % SA_ROWS, K step l / SA_ROWS of
    // the stage (the other lanes repeat lane 0's load)
    const int sa_l = lane < KS * C::SA_ROWS ? lane : 0;
    uint32_t sa_off[C::SAI];
#pragma unroll
    for (int q = 0; q < C::SAI; ++q) {
      const int sa_row = (iw + q * C::IW) * C::SA_ROWS + sa_l % C::SA_ROWS;
      const int sa_src = sSrc[sa_row] >= 0 ? sSrc[sa_row] : src0;
      // byte offsets of e8m0 scales (one byte each), else of fp32 ones
      sa_off[q] = (uint32_t)(((int64_t)sa_src * KB + sa_l / C::SA_ROWS) * (sa_e8 ? 1 : 4));
    }
    const uint8_t* sa_base = uniform_ptr(args.sa);
    const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_u32(smem));
    // fp4 weight scales: dword d = (q IW + iw) 64 + lane of the stage's
    // [BN][8] bytes is column d / 2, half d % 2 (32 columns per instruction,
    // so a gate_up instruction is wholly gate or wholly up)
    uint32_t sb_off[C::SBI > 0 ? C::SBI : 1];
#pragma unroll
    for (int q = 0; q < C::SBI; ++q) {
      const int d = (q * C::IW + iw) * 64 + lane;
      const int col = d >> 1;
      const bool up_half = KIND == KIND_GATE_UP && col >= HALF;
      int64_t n = n0 + (up_half ? col - HALF : col);
      if (n >= N) n = n0;
      sb_off[q] = (uint32_t)(n * (K / 32) + (d & 1) * 4);
    }
    const uint8_t* sbp0 = FP4 ? uniform_ptr(sb0) : nullptr;
    const uint8_t* sbp1 = FP4 && KIND == KIND_GATE_UP ? uniform_ptr(sb1) : nullptr;

    // DMA stage st (K steps st*KS ...) into operand slot `slot` and
    // row-scale slot `sa_slot` (defaults: st % NSTAGE, st % NSA)
    auto issue = [&](int st, int slot = -1, int sa_slot = -1) {
      if (!issuer) return;
      if (slot < 0) slot = st % NSTAGE;
      if (sa_slot < 0) sa_slot = st % C::NSA;
      const uint32_t sl = smem_lds + (uint32_t)(slot * C::STAGE);
      // chunk j of every issuer is of the same kind: decided at compile time
#pragma unroll
      for (int j = 0; j < C::CPW; ++j) {
        const int c = iw + j * C::IW;
        if (j < C::ACH / C::IW) {
          const int q = j % C::QA, sub = j / C::QA;
          dma16(baseA, voffA[q] + (uint32_t)(sub * 128) + (uint32_t)st * (128u * KS),
                sl + (uint32_t)c * 1024u);
        } else {
          const int b = c - C::ACH;
          const bool up_half = KIND == KIND_GATE_UP && j >= (C::ACH + HALF / 8) / C::IW;
          const int64_t nrow = n0 + (up_half ? b * 8 - HALF : b * 8);
          const uint32_t vo = nrow + rr < N ? (uint32_t)(nrow * KROW) + laneB : clampB;
          // the decode tiles (32 rows) stream the weights with nontemporal
          // loads (same box, T = 64 / 256 / 512: FP8 layer 0.62 / 0.99 /
          // 1.18 ms, FP4 0.43 / 0.68 / 0.85; with nt only for experts that
          // fit in one tile 0.61 / 1.00 / 1.19 and 0.44 / 0.72 / 0.88)
          if (KIND != KIND_DENSE && BM == 32 && SGL_NT_WEIGHTS)
            dma16nt(up_half ? b1 : b0, vo + (uint32_t)st * 128u, sl + (uint32_t)c * 1024u);
          else
            dma16(up_half ? b1 : b0, vo + (uint32_t)st * 128u, sl + (uint32_t)c * 1024u);
        }
      }
#pragma unroll
      for (int q = 0; q < C::SBI; ++q) {
        const bool up_half = KIND == KIND_GATE_UP && (q * C::IW + iw) * 32 >= HALF;
        dma4(up_half ? sbp1 : sbp0, sb_off[q] + (uint32_t)st * 8u,
             sl + (uint32_t)(C::A_BYTES + C::B_BYTES + (q * C::IW + iw) * 256));
      }
#pragma unroll
      for (int q = 0; q < C::SAI; ++q)
        if (sa_e8)  // the aligned dword holding the byte
          dma4(sa_base, (sa_off[q] + (uint32_t)st * KS) & ~3u,
               smem_lds + (uint32_t)(C::RING + sa_slot * C::SA_SLOT + (iw + q * C::IW) * 256));
        else
          dma4(sa_base, sa_off[q] + (uint32_t)st * (4u * KS),
             smem_lds + (uint32_t)(C::RING + sa_slot * C::SA_SLOT + (iw + q * C::IW) * 256));
    };

    v4f acc[TM][TN];
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
      for (int nj = 0; nj < TN; ++nj) acc[mi][nj] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const v4f vzero = {0.0f, 0.0f, 0.0f, 0.0f};

    auto tile_col = [&](int nj) -> int {
      if constexpr (KIND == KIND_GATE_UP)
        return nj < TN / 2 ? wn * HW + nj * 16 : HALF + wn * HW + (nj - TN / 2) * 16;
      else
        return (wn * TN + nj) * 16;
    };

    // DMA waits: the loads of stage st are the oldest in flight; allow the younger ones
    auto wait_stage = [&](int st) {
      const int younger = min(NSTAGE - 2, NST - 1 - st);
      if (NSTAGE >= 6 && younger >= 4) wait_vmcnt<(NSTAGE >= 6 ? 4 : 0) * C::LPS>();
      else if (NSTAGE >= 5 && younger == 3) wait_vmcnt<(NSTAGE >= 5 ? 3 : 0) * C::LPS>();
      else if (younger >= 2) wait_vmcnt<2 * C::LPS>();
      else if (younger == 1) wait_vmcnt<C::LPS>();
      else wait_vmcnt<0>();
    };
    // the MFMAs (and promotion) of stage st, from the stage's LDS slot
    auto compute_stage = [&](int st) {
      const uint8_t* stg = smem + (st % NSTAGE) * C::STAGE;
      const uint8_t* tB = stg + C::A_BYTES;
      const float* tS = reinterpret_cast<const float*>(smem + C::RING + (st % C::NSA) * C::SA_SLOT);
      // row scale of tile row `row`, K step ks of the stage
      auto row_scale = [&](int row, int ks) -> float {  // fp32 row scales
        return tS[(row / C::SA_ROWS) * 64 + ks * C::SA_ROWS + row % C::SA_ROWS];
      };
      // SAHW: the row scale's exponent, for the MFMA's scale operand: the
      // e8m0 byte (source row) KB + K step of the scale tensor, taken from
      // the aligned dword the DMA staged (dense rows past the tile's last
      // read the tile's first; their outputs are dropped), or the exponent
      // field of a power-of-two fp32 scale
      auto row_exp = [&](int row, int ks) -> int {
        const uint32_t raw = __float_as_uint(row_scale(row, ks));
        if (!sa_e8) return (int)(raw >> 23);
        const int src = row0 + (row < rows ? row : 0);
        return (int)((raw >> (((uint32_t)(src * KB + st * KS + ks) & 3u) * 8u)) & 0xFFu);
      };

      // the MFMAs of the wavefront's first NL 16-row blocks: a tile's rows
      // past its last are not computed (their outputs are dropped)
      auto blocks = [&](auto nl_c) __attribute__((always_inline)) {
        constexpr int NL = decltype(nl_c)::value;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint8_t* tA = stg + ks * (BM * 128);
          v8i af[NL];
#pragma unroll
          for (int mi = 0; mi < NL; ++mi) af[mi] = read_frag(tA + (wm * TM + mi) * 16 * 128, fla);
          if constexpr (!FP4 && LW > 0) {
            // two compute wavefronts share each SIMD (the loaders issue the
            // DMAs), so the MFMAs of one overlap the other's promotion and
            // LDS reads: no software pipelining, which keeps the live set in
            // the 168-VGPR budget of three wavefronts per SIMD.
            // Transposed product: the weight fragment is the MFMA's A operand
            // (16 columns n), the activation fragment its B operand (16 rows
            // m), so lane (g4, r16) accumulates row r16 of each 16-row block
            // and columns 4 g4 .. 4 g4 + 3 of each 16-column block: one row
            // scale per lane and block, and four consecutive output columns
            // for the epilogue's vector stores.  Per half (gate, then up; one
            // half for dense / down): the products sa * sb, then per column
            // block the weight fragment, TM MFMAs and TM x 4 promotion FMAs.
            const int kb = st;
            constexpr int HALVES = KIND == KIND_GATE_UP ? 2 : 1;
            // the row scale of row (wm TM + mi) 16 + r16 sits in slot
            // wm TM + mi at position r16 (16 rows per slot); all scales of
            // the stage are read up front with the A fragments, and the
            // weight fragment of block nj + 1 is read while the MFMAs of
            // block nj run (two fragment buffers), so no MFMA waits on LDS
            static_assert(C::SA_ROWS == 16, "row-scale slot layout");
            float sa1[NL];
#pragma unroll
            for (int mi = 0; mi < NL; ++mi) sa1[mi] = tS[(wm * TM + mi) * 64 + r16];  // fp32 (grouped)
            float sbh[HALVES];
#pragma unroll
            for (int hv = 0; hv < HALVES; ++hv) sbh[hv] = sSb[KIND == KIND_GATE_UP ? hv : wave_blk][kb];
            v8i bf[2];
            bf[0] = read_frag(tB + tile_col(0) * 128, fl);
#pragma unroll
            for (int hv = 0; hv < HALVES; ++hv) {
              float ss[NL];
#pragma unroll
              for (int mi = 0; mi < NL; ++mi) ss[mi] = sa1[mi] * sbh[hv];
#pragma unroll
              for (int nh = 0; nh < TN / HALVES; ++nh) {
                const int nj = hv * (TN / HALVES) + nh;
                if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + tile_col(nj + 1) * 128, fl);
                v4f pr[NL];
#pragma unroll
                for (int mi = 0; mi < NL; ++mi)
                  pr[mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[nj & 1], af[mi], vzero, 0, 0,
                                                                            0, 0, 0, 0);
#pragma unroll
                for (int mi = 0; mi < NL; ++mi)
#pragma unroll
                  for (int r = 0; r < 4; ++r) acc[mi][nj][r] = fmaf(pr[mi][r], ss[mi], acc[mi][nj][r]);
              }
            }
          } else if constexpr (!FP4) {
            const int kb = st;
            const float sbv0 = sSb[wave_blk][kb];
            const float sbv1 = KIND == KIND_GATE_UP ? sSb[1][kb] : 0.0f;
            if constexpr (KIND == KIND_DENSE && SAHW) {
              // e8m0 row scales: the exponent goes into the MFMA (activation
              // rows = operand A, lane r16's row), exact for a power of two.
              // e8m0 weight scales too (operand B, one per wavefront's
              // 128-column block): the MFMA accumulates in place, no
              // promotion; fp32 weight scales: C += P' sb, which is the
              // promotion's C += P (sa sb) to the bit
              int sae[NL];
#pragma unroll
              for (int mi = 0; mi < NL; ++mi) sae[mi] = row_exp((wm * TM + mi) * 16 + r16, 0);
              v8i bf[2];
              bf[0] = read_frag(tB + tile_col(0) * 128, fl);
              if (pow2) {
                const int sbe = (int)(__float_as_uint(sbv0) >> 23);
#pragma unroll
                for (int nj = 0; nj < TN; ++nj) {
                  if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + tile_col(nj + 1) * 128, fl);
#pragma unroll
                  for (int mi = 0; mi < NL; ++mi)
                    acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        af[mi], bf[nj & 1], acc[mi][nj], 0, 0, 0, sae[mi], 0, sbe);
                }
              } else {
#pragma unroll
                for (int nj = 0; nj < TN; ++nj) {
                  if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + tile_col(nj + 1) * 128, fl);
                  v4f pr[NL];
#pragma unroll
                  for (int mi = 0; mi < NL; ++mi)
                    pr[mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[mi], bf[nj & 1], vzero, 0, 0,
                                                                              0, sae[mi], 0, 127);
#pragma unroll
                  for (int mi = 0; mi < NL; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[mi][nj][r] = fmaf(pr[mi][r], sbv0, acc[mi][nj][r]);
                }
              }
              continue;
            }
            float sav[NL][4];
#pragma unroll
            for (int mi = 0; mi < NL; ++mi)
#pragma unroll
              for (int r = 0; r < 4; ++r) sav[mi][r] = row_scale((wm * TM + mi) * 16 + 4 * g4 + r, 0);
            // software pipeline: B fragment nj+1 is read while the MFMAs of
            // column block nj run, and block nj-1 is promoted after block
            // nj's MFMAs are issued, so neither the LDS latency nor the MFMA
            // latency sits in front of a dependent instruction
            v8i bf[2];
            v4f pr[2][NL];
            bf[0] = read_frag(tB + tile_col(0) * 128, fl);
#pragma unroll
            for (int nj = 0; nj < TN; ++nj) {
              if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + tile_col(nj + 1) * 128, fl);
#pragma unroll
              for (int mi = 0; mi < NL; ++mi)
                pr[nj & 1][mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    af[mi], bf[nj & 1], vzero, 0, 0, 0, 0, 0, 0);
              if (nj > 0) {
                const float sbv = (KIND == KIND_GATE_UP && nj - 1 >= TN / 2) ? sbv1 : sbv0;
#pragma unroll
                for (int mi = 0; mi < NL; ++mi) {
                  // updated as a whole vector, so the accumulators stay in registers
                  v4f t = acc[mi][nj - 1];
#pragma unroll
                  for (int r = 0; r < 4; ++r) t[r] = fmaf(pr[(nj - 1) & 1][mi][r], sav[mi][r] * sbv, t[r]);
                  acc[mi][nj - 1] = t;
                }
              }
            }
            const float sbv = (KIND == KIND_GATE_UP && TN - 1 >= TN / 2) ? sbv1 : sbv0;
#pragma unroll
            for (int mi = 0; mi < NL; ++mi) {
              v4f t = acc[mi][TN - 1];
#pragma unroll
              for (int r = 0; r < 4; ++r) t[r] = fmaf(pr[(TN - 1) & 1][mi][r], sav[mi][r] * sbv, t[r]);
              acc[mi][TN - 1] = t;
            }
          } else {
            // fp4 B: lane (r16, g4) of column block nj reads 16 bytes = K
            // [32 g4, 32 g4 + 32) of the step from column tile_col(nj) + r16,
            // and that column's e8m0 scale of the same 32-deep block
            const uint32_t bl = (uint32_t)(r16 * 128 + (((4 * ks + g4) ^ swz(r16)) << 4));
            const uint8_t* tSB = stg + C::A_BYTES + C::B_BYTES + ks * 4;
            auto read_b = [&](int nj) -> v8i {
              const uint4 v = *reinterpret_cast<const uint4*>(tB + tile_col(nj) * 128 + bl);
              return v8i{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
            };
            auto read_sb = [&](int nj) -> int {
              const uint32_t w = *reinterpret_cast<const uint32_t*>(tSB + (tile_col(nj) + r16) * 8);
              return (int)(w >> (8 * g4));
            };
            v8i bf[2];
            int sbb[2];
            bf[0] = read_b(0);
            sbb[0] = read_sb(0);
            if constexpr (SAHW) {
              // power-of-two row scales: e8m0 = the fp32 exponent field; both
              // scales are applied inside the MFMA, which accumulates in place
              int sae[NL];
#pragma unroll
              for (int mi = 0; mi < NL; ++mi) sae[mi] = row_exp((wm * TM + mi) * 16 + r16, ks);
#pragma unroll
              for (int nj = 0; nj < TN; ++nj) {
                if (nj + 1 < TN) {
                  bf[(nj + 1) & 1] = read_b(nj + 1);
                  sbb[(nj + 1) & 1] = read_sb(nj + 1);
                }
#pragma unroll
                for (int mi = 0; mi < NL; ++mi)
                  acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                      af[mi], bf[nj & 1], acc[mi][nj], 0, 4, 0, sae[mi], 0, sbb[nj & 1]);
              }
            } else {
              // fp32 row scales: the weight scales inside the MFMA, the row
              // scale promoted once per 128-deep step as in the fp8 path
              float sav[NL][4];
#pragma unroll
              for (int mi = 0; mi < NL; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) sav[mi][r] = row_scale((wm * TM + mi) * 16 + 4 * g4 + r, ks);
              v4f pr[2][NL];
#pragma unroll
              for (int nj = 0; nj < TN; ++nj) {
                if (nj + 1 < TN) {
                  bf[(nj + 1) & 1] = read_b(nj + 1);
                  sbb[(nj + 1) & 1] = read_sb(nj + 1);
                }
#pragma unroll
                for (int mi = 0; mi < NL; ++mi)
                  pr[nj & 1][mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                      af[mi], bf[nj & 1], vzero, 0, 4, 0, 127, 0, sbb[nj & 1]);
                if (nj > 0) {
#pragma unroll
                  for (int mi = 0; mi < NL; ++mi)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                      acc[mi][nj - 1][r] = fmaf(pr[(nj - 1) & 1][mi][r], sav[mi][r], acc[mi][nj - 1][r]);
                }
              }
#pragma unroll
              for (int mi = 0; mi < NL; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  acc[mi][TN - 1][r] = fmaf(pr[(TN - 1) & 1][mi][r], sav[mi][r], acc[mi][TN - 1][r]);
            }
          }
        }
      };
      // a wavefront whose rows all lie past the tile's last row has no work;
      // a 32-row decode tile (one wavefront row) that holds at most 16 rows
      // (a group's last tile) computes only its first 16-row block
      const int live = rows - wm * TM * 16;
      if (!computes || live <= 0) return;
      if constexpr (SGL_DEAD_SKIP && KIND != KIND_DENSE && WM == 1 && TM == 2) {
        if (live > 16) blocks(std::integral_constant<int, 2>{});
        else blocks(std::integral_constant<int, 1>{});
      } else {
        blocks(std::integral_constant<int, TM>{});
      }
    };

    if constexpr (LW > 0) {
      // loaders and compute wavefronts run separate loops with the same
      // barriers, so neither keeps the other's registers live: the loaders
      // wait for stage st's DMAs, meet the barrier, then refill the slot
      // stage st - 1 used; the compute wavefronts meet the barrier with
      // their reads of stage st - 1 complete, then compute stage st
      if (!computes) {
#pragma unroll
        for (int s = 0; s < NSTAGE - 1; ++s)
          if (s < NST) issue(s);
        for (int st = 0; st < NST; ++st) {
          wait_stage(st);
          __builtin_amdgcn_s_barrier();
          if (st + NSTAGE - 1 < NST) issue(st + NSTAGE - 1);
        }
      } else {
        for (int st = 0; st < NST; ++st) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();
          compute_stage(st);
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < NSTAGE - 1; ++s)
        if (s < NST) issue(s);
      for (int st = 0; st < NST; ++st) {
        wait_stage(st);
        __builtin_amdgcn_s_barrier();
        if (st + NSTAGE - 1 < NST) issue(st + NSTAGE - 1);
        compute_stage(st);
      }
    }
    __syncthreads();  // every wavefront is done with the stage ring

    if constexpr (LW > 0 && KIND != KIND_GATE_UP) {
      // ---- transposed layout: lane (g4, r16) holds row (wm TM + mi) 16 + r16,
      // columns tile_col(nj) + 4 g4 .. + 3: four consecutive outputs per
      // store (8 bytes bf16 / 16 bytes fp32), a wavefront's 64 columns of a
      // row in four stores
      const bool f32out = KIND == KIND_DENSE && args.out_f32;
      if (computes) {
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
          const int row = (wm * TM + mi) * 16 + r16;
          if (row < rows) {
            const int64_t drow = sDst[row];
#pragma unroll
            for (int nj = 0; nj < TN; ++nj) {
              const int64_t col = n0 + tile_col(nj) + 4 * g4;
              if (col < N) {
                const v4f v = acc[mi][nj];
                if (f32out) {
                  *reinterpret_cast<float4*>(reinterpret_cast<float*>(args.c) + drow * N + col) =
                      make_float4(v[0], v[1], v[2], v[3]);
                } else {
                  *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(args.c) + drow * N + col) =
                      make_uint2(pk2_bf16_exact(v[0], v[1]), pk2_bf16_exact(v[2], v[3]));
                }
              }
            }
          }
        }
      }
    } else if constexpr (LW > 0) {
      // ---- SwiGLU + 1x128 requant in registers (transposed layout): lane
      // (g4, r16) holds h of row (wm TM + mi) 16 + r16 at columns
      // wn HW + 16 j + 4 g4 .. + 3 (j < TN/2), gate and up of the same
      // columns in the same lane.  h = bf16(w * silu(bf16(gate)) * bf16(up)),
      // silu(g) = g / (1 + 2^(-g log2 e)) with the hardware exp2 and
      // reciprocal.  The row's |h| maximum over its 128 columns: the lane's
      // 8 values, the 4 lanes of the row (xor 16, 32), then the WN
      // wavefronts through sAmax.  Each lane quantizes its 8 values and
      // stores them as two 4-byte runs.
      const float lim = args.swiglu_limit;
      float h[TM][8];
      auto swiglu = [&](auto clamp_c) {
        constexpr bool CLAMP = decltype(clamp_c)::value;
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
          const int row = (wm * TM + mi) * 16 + r16;
          const float w = sW[row];
          float am = 0.0f;
#pragma unroll
          for (int j = 0; j < TN / 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float gt = bf16_round(acc[mi][j][r]);
              float up = bf16_round(acc[mi][j + TN / 2][r]);
              if constexpr (CLAMP) {
                up = clampf_(up, -lim, lim);
                gt = gt > lim ? lim : gt;
              }
              const float ex = __builtin_amdgcn_exp2f(gt * -1.4426950408889634f);
              const float silu = gt * __builtin_amdgcn_rcpf(1.0f + ex);
              const float hv = bits_f32((uint32_t)bf16_bits_exact(w * (silu * up)) << 16);
              h[mi][4 * j + r] = hv;
              // IEEE maximum (v_maximum_f32): a NaN element makes the row's
              // amax NaN, as the reference's amax does
              am = __builtin_elementwise_maximum(am, fabsf(hv));
            }
          am = __builtin_elementwise_maximum(am, __shfl_xor(am, 16, 64));
          am = __builtin_elementwise_maximum(am, __shfl_xor(am, 32, 64));
          if (g4 == 0) sAmax[wn][row] = am;
        }
      };
      static_assert(TN == 4, "the register epilogue packs 2 x 4 h values per row and lane");
      if (!computes) {
      } else if (lim > 0.0f) {
        swiglu(std::true_type{});
      } else {
        swiglu(std::false_type{});
      }
      __syncthreads();
      const int64_t NB = N / 128;
      auto requant = [&](auto mode_c) {
        constexpr int MODE = decltype(mode_c)::value;
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
          const int row = (wm * TM + mi) * 16 + r16;
          if (row < rows) {
            float am = sAmax[0][row];
#pragma unroll
            for (int q = 1; q < WN; ++q) am = __builtin_elementwise_maximum(am, sAmax[q][row]);
            const float sf = group_scale(MODE, am);
            const uint2 qv = quant8_e4m3(MODE, h[mi], sf);
            const int64_t p = row0 + row;
            uint8_t* dst = args.hq + p * N + n0 + wn * HW + 4 * g4;
            *reinterpret_cast<uint32_t*>(dst) = qv.x;
            *reinterpret_cast<uint32_t*>(dst + 16) = qv.y;
            if (wn == 0 && g4 == 0) args.hs[p * NB + n0 / 128] = sf;
          }
        }
      };
      if (computes) {
        switch (args.scale_mode) {
          case SCALE_TORCH_FP32: requant(std::integral_constant<int, SCALE_TORCH_FP32>{}); break;
          case SCALE_TORCH_UE8M0: requant(std::integral_constant<int, SCALE_TORCH_UE8M0>{}); break;
          case SCALE_TILELANG_FP32: requant(std::integral_constant<int, SCALE_TILELANG_FP32>{}); break;
          default: requant(std::integral_constant<int, SCALE_TILELANG_UE8M0>{}); break;
        }
      }
    } else if constexpr (KIND != KIND_GATE_UP) {
      // ---- stage the tile in LDS, then coalesced 16-byte row stores
      const bool f32out = KIND == KIND_DENSE && args.out_f32;
      const int esz = f32out ? 4 : 2;
      if (computes) {
#pragma unroll
        for (int mi = 0; mi < TM; ++mi)
#pragma unroll
          for (int nj = 0; nj < TN; ++nj)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = (wm * TM + mi) * 16 + 4 * g4 + r;
              const int col = tile_col(nj) + r16;
              const float v = acc[mi][nj][r];
              if (f32out)
                reinterpret_cast<float*>(smem)[row * BN + col] = v;
              else
                reinterpret_cast<uint16_t*>(smem)[row * BN + col] = bf16_bits_exact(v);
            }
      }
      __syncthreads();
      const int chunks_per_row = BN * esz / 16;
      for (int task = tid; task < BM * chunks_per_row; task += NT) {
        const int row = task / chunks_per_row, ch = task - row * chunks_per_row;
        const int64_t col = n0 + ch * (16 / esz);
        if (row < rows && col < N) {
          const uint4 v = *reinterpret_cast<const uint4*>(smem + (row * BN) * esz + ch * 16);
          uint8_t* dst = reinterpret_cast<uint8_t*>(args.c) + ((int64_t)sDst[row] * N + col) * esz;
          *reinterpret_cast<uint4*>(dst) = v;
        }
      }
    } else {
      // ---- SwiGLU epilogue: h = bf16(w * silu(bf16(gate)) * bf16(up)), staged in
      // LDS as bf16 [BM][128], then 1x128 requant of each row (16 lanes per row).
      // silu(g) = g / (1 + 2^(-g log2 e)) with the hardware exp2 and
      // reciprocal (about 1 ulp each, far below the bf16 rounding of h).
      uint16_t* hbuf = reinterpret_cast<uint16_t*>(smem);
      const float lim = args.swiglu_limit;
      auto swiglu = [&](auto clamp_c) {
        constexpr bool CLAMP = decltype(clamp_c)::value;
#pragma unroll
        for (int mi = 0; mi < TM; ++mi)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = (wm * TM + mi) * 16 + 4 * g4 + r;
            const float w = sW[row];
#pragma unroll
            for (int j = 0; j < TN / 2; ++j) {
              float gt = bf16_round(acc[mi][j][r]);
              float up = bf16_round(acc[mi][j + TN / 2][r]);
              if constexpr (CLAMP) {
                up = clampf_(up, -lim, lim);
                gt = gt > lim ? lim : gt;
              }
              const float ex = __builtin_amdgcn_exp2f(gt * -1.4426950408889634f);
              const float silu = gt * __builtin_amdgcn_rcpf(1.0f + ex);
              hbuf[row * HALF + wn * HW + j * 16 + r16] = bf16_bits_exact(w * (silu * up));
            }
          }
      };
      if (!computes) {
      } else if (lim > 0.0f) {
        swiglu(std::true_type{});
      } else {
        swiglu(std::false_type{});
      }
      __syncthreads();
      constexpr int LPR = HALF / 8;  // 16 lanes per 128-column row
      // a wavefront's 64 tasks are 4 whole rows, in range or not together
      static_assert((BM * LPR) % 64 == 0, "requant rows must fill wavefronts");
      constexpr int RQ_IT = (BM * LPR + NT - 1) / NT;
      const int64_t NB = N / 128;
      // the scale mode is a compile-time constant inside (one copy per mode),
      // so the scale formula and the quantization fold to straight-line code
      auto requant = [&](auto mode_c) {
        constexpr int MODE = decltype(mode_c)::value;
#pragma unroll
        for (int it = 0; it < RQ_IT; ++it) {
          const int task = tid + it * NT;
          if ((BM * LPR) % NT != 0 && task >= BM * LPR) break;  // wave-uniform
          const int row = task / LPR, sub = task % LPR;
          const uint4 v = *reinterpret_cast<const uint4*>(hbuf + row * HALF + sub * 8);
          const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
          float f[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            f[2 * i] = bits_f32(wv[i] << 16);
            f[2 * i + 1] = bits_f32(wv[i] & 0xFFFF0000u);
          }
          // IEEE maximum (v_maximum3_f32): a NaN element makes the group's
          // amax NaN, as the reference's amax does
          float amax = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) amax = __builtin_elementwise_maximum(amax, fabsf(f[i]));
#pragma unroll
          for (int o = LPR / 2; o > 0; o >>= 1)
            amax = __builtin_elementwise_maximum(amax, __shfl_xor(amax, o, 64));
          if (row < rows) {
            const float sf = group_scale(MODE, amax);
            const uint2 qv = quant8_e4m3(MODE, f, sf);
            const int64_t p = row0 + row;
            *reinterpret_cast<uint2*>(args.hq + p * N + n0 + sub * 8) = qv;
            if (sub == 0) args.hs[p * NB + n0 / 128] = sf;
          }
        }
      };
      switch (args.scale_mode) {
        case SCALE_TORCH_FP32: requant(std::integral_constant<int, SCALE_TORCH_FP32>{}); break;
        case SCALE_TORCH_UE8M0: requant(std::integral_constant<int, SCALE_TORCH_UE8M0>{}); break;
        case SCALE_TILELANG_FP32: requant(std::integral_constant<int, SCALE_TILELANG_FP32>{}); break;
        default: requant(std::integral_constant<int, SCALE_TILELANG_UE8M0>{}); break;
      }
    }
    __syncthreads();  // the next tile's DMA overwrites the stage ring
  }
}

// ------------------------------------------------------------ pipelined tiles
// The grouped FP8 GEMMs at prefill sizes: 128 x 256 tiles (gate/up: 128 rows
// x (128 gate + 128 up) columns; down: 128 x 256), eight compute wavefronts
// (2 x 4, 64 x 64 each) and four loader wavefronts, a 3-stage ring of 48 KB.
//
// The loaders run one tile ahead.  During tile i's K loop they DMA tile
// i+1's row slots and weight scales into the second table buffer; after
// tile i's last stage they issue tile i+1's first two stages while the
// compute wavefronts run tile i's epilogue (which keeps everything in
// registers and leaves the ring alone) and fetch the index of tile i+2.  So
// neither the table loads nor the first stages' latency separate two tiles.
// Every loader global access is an LDS DMA counted by the explicit vmcnt
// waits, except the tile-counter atomic, issued where nothing else is in
// flight that its wait could hold up.
//
// Compute (as in the loader form of gemm_fp8_kernel): the transposed product
// (weight fragment = MFMA A operand), lane (g4, r16) accumulating row
// (wm 4 + mi) 16 + r16 and columns 16 nj + 4 g4 .. + 3; per 128-deep K
// block C += P (sa sb); SwiGLU + 1x128 requant (gate/up) or bf16 stores
// (down) from registers.
namespace pipe {
constexpr int BM = 128, BN = 256, WM = 2, WN = 4, TM = 4, TN = 4, NWC = 8, LW = 4, NW = 12;
constexpr int NT = 64 * NW, NSTAGE = 3, HALF = 128, HW = HALF / WN;
constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128, STAGE = A_BYTES + B_BYTES;
constexpr int SA_ROWS = BM / NWC;     // rows per 256-byte row-scale slot
constexpr int SA_SLOT = NWC * 256;    // one stage of row scales
constexpr int RING = NSTAGE * STAGE;
constexpr int SMEM = RING + NSTAGE * SA_SLOT;
constexpr int CPW = (BM / 8 + BN / 8) / LW;  // 1 KB operand DMAs per loader per stage
constexpr int QA = BM / 8 / LW;              // A row groups per loader
constexpr int SAI = NWC / LW;                // row-scale DMAs per loader per stage
constexpr int LPS = CPW + SAI;               // DMA instructions per loader per stage
constexpr int kMaxKBp = 64;                  // K <= 8192: the tile's weight scales in LDS
static_assert(SA_ROWS == 16 && CPW == 12 && QA == 4, "layout");
static_assert(WM * WN == NWC && WM * TM * 16 == BM && WN * TN * 16 == BN, "compute wavefront grid");
}  // namespace pipe

// POW2: every row scale and weight scale is a power of two; both go into the
// MFMA as e8m0 exponents (the fp32 exponent field) and the accumulators are
// its C operand, so no fp32 promotion runs.
template <int KIND, bool POW2>
__global__ __launch_bounds__(pipe::NT) void gemm_pipe_kernel(const GemmArgs args) {
  using namespace pipe;
  static_assert(KIND == KIND_GATE_UP || KIND == KIND_DOWN, "grouped GEMMs only");
  __shared__ __align__(16) uint8_t smem[SMEM];
  __shared__ int sTstart[kMaxGroups + 1];
  __shared__ int sSlot[BM];                // next tile's sorted slots (routed rows)
  // per table buffer: the epilogue's routing weight (gate/up) or output row (down) per tile row
  __shared__ float sRow[2][BM];
  __shared__ float sSb[2][2][kMaxKBp];     // per table buffer: weight scales per K block
  __shared__ float sAmax[KIND == KIND_GATE_UP ? WN : 1][BM];
  __shared__ int sTile[2][5];              // per table buffer: valid, e, row0, rows, nt
  __shared__ uint32_t sExp[2][12];         // per table buffer: the tile expert's sgl_expert_ptrs
  __shared__ int sPend[5];                 // the tile after the next one, resolved

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = wave >= NWC;
  const int iw = loader ? wave - NWC : 0;
  const int wm = loader ? 0 : wave / WN, wn = loader ? 0 : wave % WN;
  const int g4 = lane >> 4, r16 = lane & 15;
  const int64_t K = args.K, N = args.N;
  const int KB = (int)(K / 128);
  const int NST = KB;
  const int n_tiles = args.n_tiles;
  const int G = args.E + (args.has_shared ? 1 : 0);
  const int64_t shared_base = args.offsets[args.E];

  // ---- M-tile prefix over the expert groups (E routed, then the shared one)
  if (wave == 0) {
    int carry = 0;
    if (lane == 0) sTstart[0] = 0;
    for (int base = 0; base < G; base += 64) {
      const int g = base + lane;
      int cnt = 0;
      if (g < args.E)
        cnt = args.offsets[g + 1] - args.offsets[g];
      else if (g < G)
        cnt = (int)args.T;
      int incl = (cnt + BM - 1) / BM;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
      }
      if (g < G) sTstart[g + 1] = carry + incl;
      carry += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
  const int total = sTstart[G] * n_tiles;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per_xcd = gridDim.x >> 3;
  const int per = (total + 7) >> 3;
  const int t_begin = xcd * per;
  const int t_end = min(t_begin + per, total);

  // the workgroup's next tile (wave-uniform local index): the XCD's tile
  // counter, or the static order slot, slot + per_xcd, ...
  int static_next = slot;
  auto take_tile = [&]() -> int {
    if (args.tile_ctr) return atomicAdd(&args.tile_ctr[xcd], 1);
    const int l = static_next;
    static_next += per_xcd;
    return l;
  };
  struct Tile {
    int valid, e, row0, rows, nt;
  };
  auto resolve = [&](int local) -> Tile {
    Tile t = {0, 0, 0, 0, 0};
    const int L = t_begin + local;
    if (local < 0 || L >= t_end) return t;
    int lo = 0, hi = G;  // g with sTstart[g] * n_tiles <= L < sTstart[g + 1] * n_tiles
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (sTstart[mid] * n_tiles <= L) lo = mid; else hi = mid;
    }
    const int m_in_g = sTstart[lo + 1] - sTstart[lo];
    const int loc = L - sTstart[lo] * n_tiles;
    const int nt = loc / m_in_g;
    const int mt = loc - nt * m_in_g;
    const int cnt = lo < args.E ? args.offsets[lo + 1] - args.offsets[lo] : (int)args.T;
    const int base = lo < args.E ? args.offsets[lo] : (int)shared_base;
    // the search reads LDS per lane: make the fields wave-uniform again
    t.valid = 1;
    t.e = __builtin_amdgcn_readfirstlane(lo);
    t.row0 = __builtin_amdgcn_readfirstlane(base + mt * BM);
    t.rows = __builtin_amdgcn_readfirstlane(min(BM, cnt - mt * BM));
    t.nt = __builtin_amdgcn_readfirstlane(nt);
    return t;
  };
  auto read_tile = [&](int buf) -> Tile {
    Tile t;
    t.valid = __builtin_amdgcn_readfirstlane(sTile[buf][0]);
    t.e = __builtin_amdgcn_readfirstlane(sTile[buf][1]);
    t.row0 = __builtin_amdgcn_readfirstlane(sTile[buf][2]);
    t.rows = __builtin_amdgcn_readfirstlane(sTile[buf][3]);
    t.nt = __builtin_amdgcn_readfirstlane(sTile[buf][4]);
    return t;
  };
  auto write_tile = [&](int buf, const Tile& t) {
    sTile[buf][0] = t.valid;
    sTile[buf][1] = t.e;
    sTile[buf][2] = t.row0;
    sTile[buf][3] = t.rows;
    sTile[buf][4] = t.nt;
  };
  auto write_pend = [&](const Tile& t) {
    sPend[0] = t.valid;
    sPend[1] = t.e;
    sPend[2] = t.row0;
    sPend[3] = t.rows;
    sPend[4] = t.nt;
  };
  auto read_pend = [&]() -> Tile {
    Tile t;
    t.valid = __builtin_amdgcn_readfirstlane(sPend[0]);
    t.e = __builtin_amdgcn_readfirstlane(sPend[1]);
    t.row0 = __builtin_amdgcn_readfirstlane(sPend[2]);
    t.rows = __builtin_amdgcn_readfirstlane(sPend[3]);
    t.nt = __builtin_amdgcn_readfirstlane(sPend[4]);
    return t;
  };
  // pointer field f of table buffer buf's expert record (w_gate 0, w_up 1,
  // w_down 2, s_gate 3, s_up 4, s_down 5)
  static_assert(sizeof(sgl_expert_ptrs) == 48, "expert record layout");
  auto exp_ptr = [&](int buf, int f) -> uint64_t {
    return ((uint64_t)sExp[buf][2 * f + 1] << 32) | sExp[buf][2 * f];
  };
  // address of weight scale kb of half j of tile t (record in buffer buf):
  // gate/up tiles read row n0/128 of the gate and up scales; down tiles the
  // (clamped) blocks n0/128 and n0/128 + 1
  auto scale_addr = [&](int buf, const Tile& t, int j, int kb) -> uint64_t {
    if constexpr (KIND == KIND_GATE_UP) {
      return exp_ptr(buf, j ? 4 : 3) + (uint64_t)(((int64_t)t.nt * HALF / 128) * KB + kb) * 4;
    } else {
      const int64_t nb = (N + 127) / 128;
      int64_t blk = (int64_t)t.nt * BN / 128 + j;
      if (blk > nb - 1) blk = nb - 1;
      return exp_ptr(buf, 5) + (uint64_t)(blk * KB + kb) * 4;
    }
  };

  // the epilogue value of tile row i (routed rows: from its sorted slot sl):
  // gate/up the routing weight, down the output row t (k + shared) + j
  auto row_value = [&](const Tile& t, int i, int sl) -> float {
    if constexpr (KIND == KIND_GATE_UP) {
      return (t.e < args.E && args.route_w) ? args.route_w[sl] : 1.0f;
    } else {
      const int p = t.row0 + (i < t.rows ? i : 0);
      const int tok = t.e < args.E ? sl / args.k : p - (int)shared_base;
      const int j = t.e < args.E ? sl - tok * args.k : args.k;
      return __int_as_float(tok * args.out_k + j);
    }
  };

  // ---- the first tile's tables, with plain loads (nothing else in flight);
  // loader 0 alone, the barrier below publishes them
  if (loader && iw == 0) {
    int first = 0, second = 0;
    if (lane == 0) {
      first = take_tile();
      second = take_tile();
    }
    const Tile t0 = resolve(__builtin_amdgcn_readfirstlane(__shfl(first, 0, 64)));
    const Tile t1 = resolve(__builtin_amdgcn_readfirstlane(__shfl(second, 0, 64)));
    if (lane == 0) {
      write_tile(0, t0);
      write_pend(t1);
    }
    if (t0.valid) {
      if (lane < 12) sExp[0][lane] = reinterpret_cast<const uint32_t*>(args.experts + t0.e)[lane];
      for (int i = lane; i < BM; i += 64) {
        const int sl = (t0.e < args.E && i < t0.rows) ? args.sorted_slot[t0.row0 + i] : 0;
        sSlot[i] = sl;
        sRow[0][i] = row_value(t0, i, sl);
      }
    }
  }
  __syncthreads();
  if (loader && iw == 0) {
    const Tile t0 = read_tile(0);
    if (t0.valid)
      for (int j = 0; j < 2; ++j)
        for (int kb = lane; kb < KB; kb += 64)
          sSb[0][j][kb] = *reinterpret_cast<const float*>(scale_addr(0, t0, j, kb));
  }
  __syncthreads();

  const v4f vzero = {0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_u32(smem));
  const int rr = lane >> 3, pc = lane & 7;

  // ---- loader state of the tile whose stages it issues
  // per-lane 64-bit DMA addresses (stage 0) -- no scalar base pointers, so
  // nothing of the loader's state competes for SGPRs with the tile loop's
  struct LoadState {
    uint64_t a[QA];     // A row group q
    uint64_t sa[SAI];   // row-scale slot q
    uint64_t b0, b1;    // weight bases (gate / up, or down twice)
    uint32_t laneB, clampB;
    int64_t n0;
  };
  auto setup = [&](int buf, const Tile& t) -> LoadState {
    LoadState ls;
    // A row of tile row r: the token (gate/up routed: slot / k; shared:
    // p - shared_base) or the h row p (down); rows past the tile's last row
    // re-read its first row
    auto src_of = [&](int r) -> int {
      const int rc = r < t.rows ? r : 0;
      const int p = t.row0 + rc;
      if constexpr (KIND == KIND_GATE_UP) return t.e < args.E ? sSlot[rc] / args.k : p - (int)shared_base;
      else return p;
    };
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int r = (iw + q * LW) * 8 + rr;
      ls.a[q] = (uint64_t)(uintptr_t)args.a + (uint64_t)((int64_t)src_of(r) * K + ((pc ^ swz(r)) << 4));
    }
    const int sa_l = lane < SA_ROWS ? lane : 0;
#pragma unroll
    for (int q = 0; q < SAI; ++q) {
      const int sa_row = (iw + q * LW) * SA_ROWS + sa_l;
      ls.sa[q] = (uint64_t)(uintptr_t)args.sa + (uint64_t)((int64_t)src_of(sa_row) * KB * 4);
    }
    if constexpr (KIND == KIND_GATE_UP) {
      ls.b0 = exp_ptr(buf, 0);
      ls.b1 = exp_ptr(buf, 1);
      ls.n0 = (int64_t)t.nt * HALF;
    } else {
      ls.b0 = exp_ptr(buf, 2);
      ls.b1 = ls.b0;
      ls.n0 = (int64_t)t.nt * BN;
    }
    const uint32_t chunkB = (uint32_t)((pc ^ ((rr & 6) | (iw & 1))) << 4);
    ls.laneB = (uint32_t)(rr * K) + chunkB;
    ls.clampB = (uint32_t)(ls.n0 * K) + chunkB;  // rows past N re-read row n0
    return ls;
  };
  // DMA stage st of the tile: loader iw moves 1 KB chunks c = iw + 4 j (A's
  // 16 chunks first, then B's 32) into slot st % 3 and its two row-scale
  // slots; the swizzle as in gemm_fp8_kernel
  auto issue = [&](const LoadState& ls, int st) {
    const uint32_t sl = __builtin_amdgcn_readfirstlane(smem_lds + (uint32_t)((st % NSTAGE) * STAGE));
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int c = iw + j * LW;
      if (j < QA) {
        dma16v(ls.a[j] + (uint64_t)st * 128u, __builtin_amdgcn_readfirstlane(sl + (uint32_t)c * 1024u));
      } else {
        const int b = c - BM / 8;
        const bool up_half = KIND == KIND_GATE_UP && b * 8 >= HALF;
        const int64_t nrow = ls.n0 + (up_half ? b * 8 - HALF : b * 8);
        const uint32_t vo = nrow + rr < N ? (uint32_t)(nrow * K) + ls.laneB : ls.clampB;
        // plain loads: the two or three M tiles of an expert share its weight
        // slice through L2 (nontemporal DMAs here: gate/up 1.82 -> 2.26 ms)
        dma16v((up_half ? ls.b1 : ls.b0) + vo + (uint64_t)st * 128u,
               __builtin_amdgcn_readfirstlane(sl + (uint32_t)c * 1024u));
      }
    }
#pragma unroll
    for (int q = 0; q < SAI; ++q)
      dma4v(ls.sa[q] + (uint64_t)st * 4u,
            __builtin_amdgcn_readfirstlane(
                smem_lds + (uint32_t)(RING + (st % NSTAGE) * SA_SLOT + (iw + q * LW) * 256)));
  };
  auto wait_stage = [&](int st) {
    if (st + 1 < NST) wait_vmcnt<LPS>();
    else wait_vmcnt<0>();
  };
  static_assert(NSTAGE == 3, "the waits allow exactly one younger stage in flight");
  // The next tile's tables by DMA, after the barrier of stage 1 (step 1)
  // and stage 2 (step 2) of the current tile; every loader DMA of a step is
  // older than that iteration's stage DMAs, so the next stage wait covers it.
  //   step 1: loaders 0 and 1 its 128 row slots (64 each; routed rows),
  //           loader 2 its expert record (12 dwords)
  //   step 2: loaders 0 and 1 the epilogue row values (routing weights by a
  //           gather; output rows computed), loaders 2 and 3 its gate / up
  //           (or two down) weight-scale rows
  auto prep_step1 = [&](int buf, const Tile& t) {
    if (!t.valid) return;
    if (iw < 2) {
      const bool routed = t.e < args.E;
      const int i = iw * 64 + lane;
      const int ic = routed ? (i < t.rows ? i : t.rows - 1) : 0;
      dma4v((uint64_t)(uintptr_t)args.sorted_slot + (uint64_t)(routed ? t.row0 + ic : 0) * 4u,
            __builtin_amdgcn_readfirstlane(lds_u32(&sSlot[iw * 64])));
    } else if (iw == 2 && lane < 12) {
      // the DMA writes one dword per ACTIVE lane (m0 + 4 lane): only the 12
      // lanes that own a dword of the 48-byte record may be active
      dma4v((uint64_t)(uintptr_t)(args.experts + t.e) + (uint64_t)lane * 4u,
            __builtin_amdgcn_readfirstlane(lds_u32(&sExp[buf][0])));
    }
  };
  auto prep_step2 = [&](int buf, const Tile& t) {
    if (!t.valid) return;
    if (iw < 2) {
      const int i = iw * 64 + lane;
      const int sl = sSlot[i < t.rows ? i : 0];
      if constexpr (KIND == KIND_GATE_UP) {
        if (t.e < args.E && args.route_w)
          dma4v((uint64_t)(uintptr_t)args.route_w + (uint64_t)sl * 4u,
                __builtin_amdgcn_readfirstlane(lds_u32(&sRow[buf][iw * 64])));
        else
          sRow[buf][i] = 1.0f;
      } else {
        sRow[buf][i] = row_value(t, i, sl);
      }
    } else {
      const int j = iw - 2;
      dma4v(scale_addr(buf, t, j, lane < KB ? lane : KB - 1),
            __builtin_amdgcn_readfirstlane(lds_u32(&sSb[buf][j][0])));
    }
  };

  // The two roles run separate tile loops (separate register live ranges:
  // the loader state never coexists with the accumulators) that meet at the
  // same barriers: per tile NST stage barriers, the ring-free barrier, the
  // row-maxima barrier (gate/up only) and the epilogue-done barrier. Both
  // read the same tile sequence from LDS, so they leave together.
  if (loader) {
    LoadState ls = {};
    int cur = 0;
    {
      const Tile t0 = read_tile(0);
      if (t0.valid) {
        ls = setup(0, t0);
        issue(ls, 0);
        if (NST > 1) issue(ls, 1);
      }
    }
    for (;;) {
      if (!read_tile(cur).valid) break;
      for (int st = 0; st < NST; ++st) {
        wait_stage(st);
        __builtin_amdgcn_s_barrier();
        if (st == 1) {
          // this tile's sSlot was last read by setup() before its first
          // stage; the next tile was resolved before this tile
          const Tile tn = read_pend();
          prep_step1(cur ^ 1, tn);
          if (iw == 0 && lane == 0) write_tile(cur ^ 1, tn);
        } else if (st == 2) {
          // step 1's DMAs have landed (the stage-2 wait and barrier)
          prep_step2(cur ^ 1, read_tile(cur ^ 1));
        }
        if (st + 2 < NST) issue(ls, st + 2);
      }
      __syncthreads();  // the ring is free; the next tile's tables are in LDS
      // the next tile's first two stages, then (loader 0) the tile after
      // it, taken and resolved: its loads wait for those DMAs too, which the
      // next tile's first stage waits for anyway; all of it overlaps the
      // compute wavefronts' epilogue
      const Tile tn = read_tile(cur ^ 1);
      if (tn.valid) {
        ls = setup(cur ^ 1, tn);
        issue(ls, 0);
        if (NST > 1) issue(ls, 1);
      }
      if (iw == 0) {
        int idx = -1;
        if (lane == 0 && tn.valid) idx = take_tile();
        const Tile tp = resolve(__builtin_amdgcn_readfirstlane(__shfl(idx, 0, 64)));
        if (lane == 0) write_pend(tp);
      }
      if constexpr (KIND == KIND_GATE_UP) __syncthreads();  // row maxima
      __syncthreads();  // epilogue done
      cur ^= 1;
    }
    return;
  }

  int cur = 0;
  for (;;) {
    const Tile tc = read_tile(cur);
    if (!tc.valid) break;
    const int row0 = tc.row0, rows = tc.rows;
    const int64_t n0 = KIND == KIND_GATE_UP ? (int64_t)tc.nt * HALF : (int64_t)tc.nt * BN;

    const FragLane fl = frag_lane(r16, g4);
    auto tile_col = [&](int nj) -> int {
      if constexpr (KIND == KIND_GATE_UP)
        return nj < TN / 2 ? wn * HW + nj * 16 : HALF + wn * HW + (nj - TN / 2) * 16;
      else
        return (wn * TN + nj) * 16;
    };
    const int wave_blk = KIND == KIND_GATE_UP ? 0 : (wn * TN * 16) / 128;

    v4f acc[TM][TN];
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
      for (int nj = 0; nj < TN; ++nj) acc[mi][nj] = vzero;

    // The wavefront's 16-row blocks that hold rows of the tile (an expert's
    // last M tile is partly padding): only those get fragment reads and
    // MFMAs (TML of the TM blocks, a compile-time count per K loop), so the
    // padding costs whole 16-row blocks, not the wavefront's 64 rows.
    const int tml = min(TM, max(0, (rows - wm * TM * 16 + 15) >> 4));
    auto kloop = [&](auto tml_c) {
      constexpr int TML = decltype(tml_c)::value;
      for (int st = 0; st < NST; ++st) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if constexpr (TML > 0) {
          const uint8_t* stg = smem + (st % NSTAGE) * STAGE;
          const uint8_t* tB = stg + A_BYTES;
          const float* tS = reinterpret_cast<const float*>(smem + RING + (st % NSTAGE) * SA_SLOT);
          // LDS reads in the order the MFMAs consume them (A0, B0 and the
          // scales, then A1..): the reads complete in order, so the first
          // MFMA waits for two fragments, not for the whole stage's burst of
          // all eight wavefronts
          v8i af[TML];
          v8i bf[2];
          constexpr int HALVES = KIND == KIND_GATE_UP ? 2 : 1;
          float sa1[TML];
          float sbh[HALVES];
          af[0] = read_frag(stg + (wm * TM) * 16 * 128, fl);
          bf[0] = read_frag(tB + tile_col(0) * 128, fl);
#pragma unroll
          for (int mi = 0; mi < TML; ++mi) sa1[mi] = tS[(wm * TM + mi) * 64 + r16];
#pragma unroll
          for (int hv = 0; hv < HALVES; ++hv) sbh[hv] = sSb[cur][KIND == KIND_GATE_UP ? hv : wave_blk][st];
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int mi = 1; mi < TML; ++mi) af[mi] = read_frag(stg + (wm * TM + mi) * 16 * 128, fl);
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (POW2) {
            // operand A = the weight fragment (one scale per 16-column
            // fragment: the 128 x 128 block), operand B = the activation rows
            // (lane r16's row scale); the scale of lane (g4, r16) covers its
            // 32-deep K quarter, the same for all four quarters here
            int sae[TML], sbe[HALVES];
#pragma unroll
            for (int mi = 0; mi < TML; ++mi) sae[mi] = (int)(__float_as_uint(sa1[mi]) >> 23);
#pragma unroll
            for (int hv = 0; hv < HALVES; ++hv) sbe[hv] = (int)(__float_as_uint(sbh[hv]) >> 23);
#pragma unroll
            for (int hv = 0; hv < HALVES; ++hv)
#pragma unroll
              for (int nh = 0; nh < TN / HALVES; ++nh) {
                const int nj = hv * (TN / HALVES) + nh;
                if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + tile_col(nj + 1) * 128, fl);
#pragma unroll
                for (int mi = 0; mi < TML; ++mi)
                  acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                      bf[nj & 1], af[mi], acc[mi][nj], 0, 0, 0, sbe[hv], 0, sae[mi]);
              }
          } else {
#pragma unroll
            for (int hv = 0; hv < HALVES; ++hv) {
              float ss[TML];
#pragma unroll
              for (int mi = 0; mi < TML; ++mi) ss[mi] = sa1[mi] * sbh[hv];
#pragma unroll
              for (int nh = 0; nh < TN / HALVES; ++nh) {
                const int nj = hv * (TN / HALVES) + nh;
                if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + tile_col(nj + 1) * 128, fl);
                v4f pr[TML];
#pragma unroll
                for (int mi = 0; mi < TML; ++mi)
                  pr[mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[nj & 1], af[mi], vzero, 0, 0,
                                                                            0, 0, 0, 0);
#pragma unroll
                for (int mi = 0; mi < TML; ++mi)
#pragma unroll
                  for (int r = 0; r < 4; ++r) acc[mi][nj][r] = fmaf(pr[mi][r], ss[mi], acc[mi][nj][r]);
              }
            }
          }
        }
      }
    };
    switch (tml) {
      case 0: kloop(std::integral_constant<int, 0>{}); break;
      case 1: kloop(std::integral_constant<int, 1>{}); break;
      case 2: kloop(std::integral_constant<int, 2>{}); break;
      case 3: kloop(std::integral_constant<int, 3>{}); break;
      default: kloop(std::integral_constant<int, TM>{}); break;
    }
    __syncthreads();  // the ring is free; the next tile's tables are in LDS

    if constexpr (KIND == KIND_DOWN) {
      {
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
          const int row = (wm * TM + mi) * 16 + r16;
          if (row < rows) {
            const int64_t drow = __float_as_int(sRow[cur][row]);
#pragma unroll
            for (int nj = 0; nj < TN; ++nj) {
              const int64_t col = n0 + tile_col(nj) + 4 * g4;
              if (col < N) {
                const v4f v = acc[mi][nj];
                // plain stores (nontemporal ones: down 1.01 -> 1.17 ms)
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(args.c) + drow * N + col) =
                    make_uint2(pk2_bf16_exact(v[0], v[1]), pk2_bf16_exact(v[2], v[3]));
              }
            }
          }
        }
      }
    } else {
      // SwiGLU + 1x128 requant from registers (see gemm_fp8_kernel)
      // h is bf16-exact: kept as packed pairs (16 registers, not 32) across
      // the barrier that publishes the row maxima
      const float lim = args.swiglu_limit;
      uint32_t h2[TM][4];
      auto swiglu = [&](auto clamp_c) {
        constexpr bool CLAMP = decltype(clamp_c)::value;
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
          const int row = (wm * TM + mi) * 16 + r16;
          const float w = sRow[cur][row];
          float am = 0.0f;
#pragma unroll
          for (int j = 0; j < TN / 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float gt = bf16_round(acc[mi][j][r]);
              float up = bf16_round(acc[mi][j + TN / 2][r]);
              if constexpr (CLAMP) {
                up = clampf_(up, -lim, lim);
                gt = gt > lim ? lim : gt;
              }
              const float ex = __builtin_amdgcn_exp2f(gt * -1.4426950408889634f);
              const float silu = gt * __builtin_amdgcn_rcpf(1.0f + ex);
              const uint32_t hb = bf16_bits_exact(w * (silu * up));
              const int q = 4 * j + r;
              if (q & 1)
                h2[mi][q >> 1] |= hb << 16;
              else
                h2[mi][q >> 1] = hb;
              am = __builtin_elementwise_maximum(am, fabsf(bits_f32(hb << 16)));
            }
          am = __builtin_elementwise_maximum(am, __shfl_xor(am, 16, 64));
          am = __builtin_elementwise_maximum(am, __shfl_xor(am, 32, 64));
          if (g4 == 0) sAmax[wn][row] = am;
        }
      };
      if (lim > 0.0f) {
        swiglu(std::true_type{});
      } else {
        swiglu(std::false_type{});
      }
      __syncthreads();
      const int64_t NB = N / 128;
      auto requant = [&](auto mode_c) {
        constexpr int MODE = decltype(mode_c)::value;
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
          const int row = (wm * TM + mi) * 16 + r16;
          if (row < rows) {
            float am = sAmax[0][row];
#pragma unroll
            for (int q = 1; q < WN; ++q) am = __builtin_elementwise_maximum(am, sAmax[q][row]);
            const float sf = group_scale(MODE, am);
            float hf[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              hf[2 * q] = bits_f32(h2[mi][q] << 16);
              hf[2 * q + 1] = bits_f32(h2[mi][q] & 0xFFFF0000u);
            }
            const uint2 qv = quant8_e4m3(MODE, hf, sf);
            const int64_t p = row0 + row;
            uint8_t* dst = args.hq + p * N + n0 + wn * HW + 4 * g4;
            *reinterpret_cast<uint32_t*>(dst) = qv.x;
            *reinterpret_cast<uint32_t*>(dst + 16) = qv.y;
            if (wn == 0 && g4 == 0) args.hs[p * NB + n0 / 128] = sf;
          }
        }
      };
      switch (args.scale_mode) {
        case SCALE_TORCH_FP32: requant(std::integral_constant<int, SCALE_TORCH_FP32>{}); break;
        case SCALE_TORCH_UE8M0: requant(std::integral_constant<int, SCALE_TORCH_UE8M0>{}); break;
        case SCALE_TILELANG_FP32: requant(std::integral_constant<int, SCALE_TILELANG_FP32>{}); break;
        default: requant(std::integral_constant<int, SCALE_TILELANG_UE8M0>{}); break;
      }
    }
    __syncthreads();  // epilogue done (sAmax, the table buffer cur free)
    cur ^= 1;
  }
}

template <int KIND, bool POW2>
int launch_pipe(GemmArgs& a, hipStream_t stream) {
  using namespace pipe;
  a.n_tiles = (int)ceil_div(a.N, KIND == KIND_GATE_UP ? HALF : BN);
  const int64_t P = a.E > 0 ? a.T * a.k : 0;
  const int64_t mt_bound = P / BM + (P < a.E ? P : a.E) + (a.has_shared ? ceil_div(a.T, BM) : 0);
  const int64_t tiles = mt_bound * a.n_tiles;
  if (tiles == 0) return SGL_OK;
  constexpr int kLds = SMEM + 4 * (kMaxGroups + 1) + BM * 4 + 2 * BM * 4 + 2 * 2 * kMaxKBp * 4 +
                       (KIND == KIND_GATE_UP ? WN * BM * 4 : 4) + 2 * 5 * 4 + 2 * 12 * 4 + 5 * 4;
  static_assert(kLds <= 160 * 1024, "pipelined tile exceeds the LDS of a CU");
  int64_t wgs = (int64_t)device_cu_count();
  wgs = (wgs + 7) / 8 * 8;
  const int64_t need = (tiles + 7) / 8 * 8;
  if (need < wgs) wgs = need;
  a.m_tiles = (int)mt_bound;
  gemm_pipe_kernel<KIND, POW2><<<(unsigned)wgs, NT, 0, stream>>>(a);
  return check_launch("gemm_pipe");
}

// ------------------------------------------------------------ register-fed weights
// The grouped FP8 GEMMs at prefill sizes with the expert weights in the MFMA
// fragment layout (weight_to_frag_kernel below: per 16 rows x 128-deep block,
// 2 KB that hold lane l's 32 bytes of the block as two 1 KB halves, so each
// half is one fully coalesced 1 KB load straight into registers).
//
// The weight fragments go from memory into registers D = 4 stages ahead of
// the MFMAs that use them: the register file (512 KB per CU) holds the weight
// bytes in flight, where the LDS-staged kernels are capped by 160 KB of LDS
// at two 48 KB stages in flight.  Only the activation rows, which all eight
// wavefronts share, pass through LDS: loaded into registers four stages
// ahead, written into one of four 16 KB LDS slots two stages ahead.
//
// 128 x 256 tiles (gate/up: 128 rows x (128 gate + 128 up) columns; down:
// 128 x 256), eight wavefronts side by side along N: wavefront w owns all 128
// rows and 16 gate + 16 up columns (gate/up) or 32 columns (down), so no
// weight byte is loaded twice.  Per 128-deep K block the transposed product
// and fp32 promotion of gemm_pipe_kernel (C += P (sa sb), K blocks in
// order), so the outputs are bit-identical to it.
//
// Every load is an ordinary compiler-visible load, so the compiler's vmcnt
// waits count them.  The waits stay partial (vmcnt(n) with the younger
// stages still in flight) only if the count is the same on every path:
// every stage issues its activation, row-scale and weight loads
// unconditionally (the last tile re-reads its own first stages for the
// tile that does not follow), and the output stores are issued outside the
// compiler's accounting (store_b32 / store_b64: a store the compiler saw
// would turn its next wait into vmcnt(0), draining the next tile's loads;
// an extra store in flight can only delay, never satisfy early, a wait for
// an older load, since loads return in order).  Tiles follow a static order
// per XCD (no atomic counter, for the same reason; every tile runs all eight
// row blocks, so the tiles take the same time).  The next tile's tables are
// prepared at fixed stages of the current tile (K >= 2048: at least 16
// stages): resolved at stage 5, its row slots and expert record loaded at 6
// and stored at 10 (with its weight scales and routing weights loaded), its
// row addresses formed at 12, its weight scales and routing weights stored
// at 14; its first stages load from stage NST - 4.
//
// Stores the compiler does not count (see above).  At most 8 bytes of data:
// wider stores have a data-overwrite hazard the compiler would not cover.
__device__ __forceinline__ void store_b32(void* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off" :: "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_b64(void* p, uint2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off" :: "v"(p), "v"(v) : "memory");
}

#ifndef SGL_RB_DBG
#define SGL_RB_DBG 2
#endif
namespace rb {
constexpr int BM = 128;  // tile rows (the tile columns: 256 NJ, set per launch)
constexpr int SLOTS = 4;  // LDS slots of 128-deep activation stages
constexpr int A_BYTES = BM * 128;
constexpr int kMinKB = 16, kMaxKBr = 64;
static_assert(SLOTS == 4, "the stage loop is unrolled by four");
}  // namespace rb

// Eight wavefronts (two per SIMD), each owning NJ 16-column fragments of the
// gate and of the up half (gate/up) or 2 NJ fragments (down): a tile is 128
// rows x 128 NJ gate + 128 NJ up columns (down: 256 NJ columns).  NJ = 2
// halves the LDS fragment reads per MFMA (each activation fragment feeds
// four MFMAs, not two) and keeps DB = 2 weight stages in registers; NJ = 1
// keeps four.
//
// POW2: every row scale and weight scale is a power of two; both go into the
// MFMA as e8m0 exponents with the accumulators as its C operand (no fp32
// promotion), as in gemm_pipe_kernel<POW2>.
//
// W4: packed e2m1 weights (the FP4 fragment layout: 16 bytes per lane and
// 128-deep block, the fp4 MFMA operand) with their e8m0 1 x 32 scales, which
// the MFMA applies (one dword per lane holds a lane's scales for four
// stages); the activation fragment pairs its K as the FP4 kernels do (chunks
// l/16 and 4 + l/16); the row scales as for FP8 (POW2: in the MFMA, else one
// fp32 promotion per 128-deep block).
//
// NTW: the weight fragments by nontemporal loads (decode batches, where an
// expert's rows rarely fill two tiles and each weight byte is read once).
template <int KIND, int NJ, bool POW2, bool W4, bool NTW>
__global__ __launch_bounds__(512) void gemm_rb_kernel(const GemmArgs args) {
  using namespace rb;
  static_assert(KIND == KIND_GATE_UP || KIND == KIND_DOWN, "grouped GEMMs only");
  static_assert(NJ == 1 || NJ == 2, "one or two fragments per half");
  static_assert(!W4 || NJ == 1, "fp4 weights: 16-column fragments per half");
  constexpr int NW = 8, NT = 64 * NW;
  // stages of weight fragments in registers: four for down and for fp4
  // (half the registers per fragment); fp8 gate/up (whose epilogue holds more
  // registers across the tile boundary) SGL_RB_DBG
  constexpr int DB = NJ == 2 ? 2 : ((KIND == KIND_GATE_UP && !W4) ? SGL_RB_DBG : 4);
  constexpr uint32_t WBLK = W4 ? 1024 : 2048;  // weight bytes per 16-row x 128-deep block
  constexpr int GC = 128 * NJ;         // gate/up: gate columns of a tile
  constexpr int TC = KIND == KIND_GATE_UP ? GC : 256 * NJ;  // output columns of a tile (per half)
  constexpr int NB = 2 * NJ;           // weight-scale rows of a tile (gate/up: NJ per half)
  constexpr int NF = 2 * NJ;        // weight fragments per wavefront and stage
  constexpr int RPW = BM / NW;      // tile rows whose activations a wavefront loads
  constexpr int AQ = RPW / 8;       // 1 KB activation loads per wavefront and stage
  __shared__ __align__(16) uint8_t sA[SLOTS * A_BYTES];
  __shared__ __align__(16) float sSa[2][BM * 4];  // row scales of four stages, [row][4]
  __shared__ int sTstart[kMaxGroups + 1];
  __shared__ int sOff[kMaxGroups + 1];  // expert row offsets (the shared group's start last)
  __shared__ int sSlot[2][BM];    // per table buffer: sorted slot of each routed row
  __shared__ float sRow[2][BM];   // per table buffer: routing weight (gate/up) / output row (down)
  __shared__ float sAmax[KIND == KIND_GATE_UP ? NW : 1][BM];
  __shared__ int sTile[2][5];     // per table buffer: valid, e, row0, rows, nt
  __shared__ float sSb[2][NB][kMaxKBr];  // per table buffer: weight scales per K block
                                        // (gate/up: gate blocks, then up blocks)

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, r16 = lane & 15;
  const int64_t K = args.K, N = args.N;
  const int KB = (int)(K / 128);
  const int NST = KB;
  const int n_tiles = args.n_tiles;
  const int G = args.E + (args.has_shared ? 1 : 0);
  const int64_t shared_base = args.offsets[args.E];

  for (int g = tid; g <= args.E; g += NT) sOff[g] = args.offsets[g];
  // ---- M-tile prefix over the expert groups (E routed, then the shared one)
  if (w == 0) {
    int carry = 0;
    if (lane == 0) sTstart[0] = 0;
    for (int base = 0; base < G; base += 64) {
      const int g = base + lane;
      int cnt = 0;
      if (g < args.E)
        cnt = args.offsets[g + 1] - args.offsets[g];
      else if (g < G)
        cnt = (int)args.T;
      int incl = (cnt + BM - 1) / BM;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
      }
      if (g < G) sTstart[g + 1] = carry + incl;
      carry += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
  const int total = sTstart[G] * n_tiles;
  const int xcd = blockIdx.x & 7, wslot = blockIdx.x >> 3, per_xcd = gridDim.x >> 3;
  const int per = (total + 7) >> 3;
  const int t_begin = xcd * per;
  const int t_end = min(t_begin + per, total);

  // workgroup wslot of an XCD takes its tiles wslot, wslot + per_xcd, ...
  int static_next = wslot;
  auto take_tile = [&]() -> int {
    const int l = static_next;
    static_next += per_xcd;
    return l;
  };
  struct Tile {
    int valid, e, row0, rows, nt;
  };
  auto resolve = [&](int local) -> Tile {
    Tile t = {0, 0, 0, 0, 0};
    const int L = t_begin + local;
    if (local < 0 || L >= t_end) return t;
    int lo = 0, hi = G;  // g with sTstart[g] * n_tiles <= L < sTstart[g + 1] * n_tiles
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (sTstart[mid] * n_tiles <= L) lo = mid; else hi = mid;
    }
    const int m_in_g = sTstart[lo + 1] - sTstart[lo];
    const int loc = L - sTstart[lo] * n_tiles;
    const int nt = loc / m_in_g;
    const int mt = loc - nt * m_in_g;
    // LDS only: no global load whose wait would drain the loads in flight
    const int cnt = lo < args.E ? sOff[lo + 1] - sOff[lo] : (int)args.T;
    const int base = lo < args.E ? sOff[lo] : (int)shared_base;
    t.valid = 1;
    t.e = __builtin_amdgcn_readfirstlane(lo);
    t.row0 = __builtin_amdgcn_readfirstlane(base + mt * BM);
    t.rows = __builtin_amdgcn_readfirstlane(min(BM, cnt - mt * BM));
    t.nt = __builtin_amdgcn_readfirstlane(nt);
    return t;
  };
  auto read_tile = [&](int buf) -> Tile {
    Tile t;
    t.valid = __builtin_amdgcn_readfirstlane(sTile[buf][0]);
    t.e = __builtin_amdgcn_readfirstlane(sTile[buf][1]);
    t.row0 = __builtin_amdgcn_readfirstlane(sTile[buf][2]);
    t.rows = __builtin_amdgcn_readfirstlane(sTile[buf][3]);
    t.nt = __builtin_amdgcn_readfirstlane(sTile[buf][4]);
    return t;
  };
  auto write_tile = [&](int buf, const Tile& t) {
    sTile[buf][0] = t.valid;
    sTile[buf][1] = t.e;
    sTile[buf][2] = t.row0;
    sTile[buf][3] = t.rows;
    sTile[buf][4] = t.nt;
  };
  // the epilogue value of tile row i (routed rows: of sorted slot sl): down the
  // output row t (k + shared) + j, as float bits
  auto out_row = [&](const Tile& t, int i, int sl) -> float {
    const int p = t.row0 + (i < t.rows ? i : 0);
    const int tok = t.e < args.E ? sl / args.k : p - (int)shared_base;
    const int j = t.e < args.E ? sl - tok * args.k : args.k;
    return __int_as_float(tok * args.out_k + j);
  };
  // uniform 64-bit field f of expert record e (scalar loads: the table is
  // read-only for the kernel)
  typedef __attribute__((address_space(4))) const uint64_t* cptr64;
  auto rec_field = [&](const sgl_expert_ptrs* tab, int e, int f) -> uint64_t {
    return *((cptr64)(uintptr_t)(tab + e) + f);
  };

  // ---- per-tile load sources of this wavefront
  const int ch = lane & 7;
  auto a_row = [&](int q) -> int { return RPW * w + 8 * q + (lane >> 3); };
  uint32_t lds_a[AQ];
#pragma unroll
  for (int q = 0; q < AQ; ++q) lds_a[q] = (uint32_t)(a_row(q) * 128 + ((ch ^ swz(a_row(q))) << 4));
  struct Src {
    uint32_t a[AQ];   // rows a_row(q) of the tile: byte offset of (row, 16 ch) in A
    uint32_t sa;      // waves 0, 1: offset (floats) of row 64 w + lane's row scales
    uint64_t b0, b1;  // (uniform) weight fragment blocks (n16, 0) of the wavefront's first
                      // gate / up fragment (down: b0 only); fragment j at + j K/128 WBLK
    uint64_t s0, s1;  // W4: (uniform) scale blocks (n16, 0), fragment j at + j K/512 256
  };
  // source row of tile row r (rows past the tile's last re-read its first)
  auto src_row = [&](const Tile& t, int buf, int r) -> int64_t {
    const int rc = r < t.rows ? r : 0;
    const int p = t.row0 + rc;
    if constexpr (KIND == KIND_GATE_UP) return t.e < args.E ? sSlot[buf][rc] / args.k : p - shared_base;
    else return p;
  };
  // row offsets of tile t (its slots in sSlot[buf]); T K < 2^31 and rows K < 2^31
  auto rows_of = [&](Src& s, const Tile& t, int buf) {
#pragma unroll
    for (int q = 0; q < AQ; ++q) s.a[q] = (uint32_t)(src_row(t, buf, a_row(q)) * K + ch * 16);
    s.sa = (uint32_t)((w < 2 ? src_row(t, buf, 64 * w + lane) : 0) * KB);
  };
  // a global (not flat) fp32 load: a flat load also counts in lgkmcnt and is
  // a different kind of event for the compiler's waits, which then fall back
  // to vmcnt(0)
  auto ldg_f32 = [&](uint64_t base, int64_t i) -> float {
    return ((__attribute__((address_space(1))) const float*)(uintptr_t)base)[i];
  };
  // weight bases and (loads of) the weight scales of tile t: lane kb gets
  // those of K block kb in sb0, sb1
  auto weights_of = [&](Src& s, const Tile& t, float& sb0, float& sb1) {
    const int kbl = lane < KB ? lane : KB - 1;
    if constexpr (KIND == KIND_GATE_UP) {
      const int64_t nb16 = N / 16;
      int64_t n16 = (int64_t)t.nt * (GC / 16) + NJ * w;
      if (n16 > nb16 - NJ) n16 = nb16 - NJ;  // columns past N (not stored) re-read the last blocks
      s.b0 = rec_field(args.frag, t.e, 0) + (uint64_t)(n16 * KB * WBLK);
      s.b1 = rec_field(args.frag, t.e, 1) + (uint64_t)(n16 * KB * WBLK);
      if constexpr (W4) {
        s.s0 = rec_field(args.frag, t.e, 3) + (uint64_t)(n16 * (KB / 4) * 256);
        s.s1 = rec_field(args.frag, t.e, 4) + (uint64_t)(n16 * (KB / 4) * 256);
        sb0 = sb1 = 1.0f;  // the weight scales go into the MFMA
      } else {
        const int64_t blk = n16 / 8;
        sb0 = ldg_f32(rec_field(args.experts, t.e, 3), blk * KB + kbl);
        sb1 = ldg_f32(rec_field(args.experts, t.e, 4), blk * KB + kbl);
      }
    } else {
      const int64_t nb16 = N / 16;
      int64_t n16 = (int64_t)t.nt * (TC / 16) + NF * w;
      if (n16 > nb16 - NF) n16 = nb16 - NF;  // columns past N (not stored) re-read the last blocks
      s.b0 = rec_field(args.frag, t.e, 2) + (uint64_t)(n16 * KB * WBLK);
      s.b1 = s.b0;
      if constexpr (W4) {
        s.s0 = rec_field(args.frag, t.e, 5) + (uint64_t)(n16 * (KB / 4) * 256);
        s.s1 = s.s0;
        sb0 = sb1 = 1.0f;
      } else {
        const int64_t nb = (N + 127) / 128;
        int64_t blk = ((int64_t)t.nt * TC + 16 * NF * w) / 128;
        if (blk > nb - 1) blk = nb - 1;
        sb0 = ldg_f32(rec_field(args.experts, t.e, 5), blk * KB + kbl);
        sb1 = sb0;
      }
    }
  };
  const uint32_t lane16 = (uint32_t)lane * 16;
  typedef float f4v __attribute__((ext_vector_type(4)));
  auto ld_sa = [&](uint32_t off) -> float4 {
    const f4v v = *(__attribute__((address_space(1))) const f4v*)(
        (__attribute__((address_space(1))) const float*)(uintptr_t)args.sa + off);
    return make_float4(v.x, v.y, v.z, v.w);
  };
  // global (not flat) loads: a flat load would also count in lgkmcnt, which
  // the LDS waits drain
  typedef int i4v __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(1))) const uint8_t gbyte;
  typedef __attribute__((address_space(1))) const i4v gi4v;
  gbyte* const a_g = (gbyte*)(uintptr_t)args.a;
  auto ldA = [&](uint32_t off) -> uint4 {
    const i4v v = *(gi4v*)(a_g + off);
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
  };
  // the lane's two 16-byte pieces of a weight fragment, at 16 l and
  // 1024 + 16 l of its block; with NTW by nontemporal loads (the nt cache
  // policy): a read stream on gfx950 moves 7.0 TB/s with nt loads where
  // plain loads move 6.2 (2 GiB, measured; FP4 decode T = 64 / 256 / 512
  // 0.42 / 0.65 / 0.76 -> 0.40 / 0.62 / 0.73 ms)
  auto ldB = [&](uint64_t base, uint64_t off) -> v8i {
    gbyte* p = (gbyte*)(uintptr_t)base;
    const i4v lo = NTW ? __builtin_nontemporal_load((gi4v*)(p + off + lane16)) : *(gi4v*)(p + off + lane16);
    if constexpr (W4) return v8i{lo.x, lo.y, lo.z, lo.w, 0, 0, 0, 0};  // 16 packed bytes
    const i4v hi = NTW ? __builtin_nontemporal_load((gi4v*)(p + off + (lane16 + 1024u)))
                       : *(gi4v*)(p + off + (lane16 + 1024u));
    return v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  };
  // W4: lane's scale dword of fragment f for the four stages of group g
  auto ldS = [&](const Src& s, int f, int g) -> uint32_t {
    const uint64_t base = (f < NJ || KIND == KIND_DOWN) ? s.s0 : s.s1;
    const int j = KIND == KIND_DOWN ? f : f % NJ;
    return *(__attribute__((address_space(1))) const uint32_t*)(uintptr_t)(
        base + (uint64_t)j * (KB / 4) * 256 + (uint64_t)g * 256 + (uint64_t)lane * 4);
  };
  // the 128-column weight-scale block (within the tile) of this wavefront's
  // columns, and the tile's weight scales into sSb[buf], written by the first
  // wavefront of each block
  constexpr int WPB = KIND == KIND_GATE_UP ? 8 / NJ : 4 / NJ;  // wavefronts per block
  const int bi = w / WPB;
  auto put_scales = [&](int buf, float sb0, float sb1) {
    if (lane < KB && w % WPB == 0) {
      sSb[buf][bi][lane] = sb0;
      if constexpr (KIND == KIND_GATE_UP) sSb[buf][NJ + bi][lane] = sb1;
    }
  };

  // ---- the first tile, with plain loads
  int nidx = 0;  // wave 0 lane 0: the local index of the tile after the current one
  if (w == 0) {
    int first = 0;
    if (lane == 0) {
      first = take_tile();
      nidx = take_tile();
    }
    const Tile t0 = resolve(__builtin_amdgcn_readfirstlane(__shfl(first, 0, 64)));
    if (lane == 0) write_tile(0, t0);
  }
  __syncthreads();
  Tile tc = read_tile(0);
  if (!tc.valid) return;
  if (lane < RPW) {
    const int i = RPW * w + lane;
    const int sl = (tc.e < args.E && i < tc.rows) ? args.sorted_slot[tc.row0 + i] : 0;
    sSlot[0][i] = sl;
    if constexpr (KIND == KIND_GATE_UP)
      sRow[0][i] = (tc.e < args.E && args.route_w) ? args.route_w[sl] : 1.0f;
    else
      sRow[0][i] = out_row(tc, i, sl);
  }
  __syncthreads();
  Src cs, ns;
  float nsb0, nsb1;
  rows_of(cs, tc, 0);
  weights_of(cs, tc, nsb0, nsb1);
  put_scales(0, nsb0, nsb1);
  ns = cs;

  // weight fragment f of the wavefront at stage offset off (bytes within the block row)
  auto ldBf = [&](const Src& s, int f, uint32_t off) -> v8i {
    if constexpr (KIND == KIND_GATE_UP)
      return ldB(f < NJ ? s.b0 : s.b1, (uint64_t)(f % NJ) * KB * WBLK + off);
    else
      return ldB(s.b0, (uint64_t)f * KB * WBLK + off);
  };
  uint32_t swc[NF], swn[NF];  // W4: scale dwords of the current / next group of four stages
  v8i bq[DB][NF];
  uint4 aq[2][AQ];
  float4 sq = make_float4(0.f, 0.f, 0.f, 0.f);
  {
    // stages 0 and 1 into LDS slots 0 and 1, row scales of stages 0..3
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < AQ; ++q) aq[j][q] = ldA(cs.a[q] + j * 128);
    sq = ld_sa(cs.sa);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < AQ; ++q) *reinterpret_cast<uint4*>(sA + j * A_BYTES + lds_a[q]) = aq[j][q];
    if (w < 2) *reinterpret_cast<float4*>(&sSa[0][(64 * w + lane) * 4]) = sq;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < AQ; ++q) aq[j][q] = ldA(cs.a[q] + (2 + j) * 128);
#pragma unroll
    for (int s = 0; s < DB; ++s)
#pragma unroll
      for (int f = 0; f < NF; ++f) bq[s][f] = ldBf(cs, f, s * WBLK);
#pragma unroll
    for (int f = 0; f < NF; ++f) swc[f] = swn[f] = W4 ? ldS(cs, f, 0) : 0u;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // the activation fragment's K pairing: fp8 x fp8 chunks 2 (l/16), +1; with
  // fp4 weights chunks l/16 and 4 + l/16
  const FragLane fl = W4 ? frag_lane_fp4a(r16, g4) : frag_lane(r16, g4);
  const v4f vzero = {0.0f, 0.0f, 0.0f, 0.0f};
  int tb = 0;    // table buffer of the current tile
  int gpar = 0;  // row-scale buffer of the current tile's first four stages
  float nrw = 0.0f;
  int nslot = 0;
  Tile tn = {0, 0, 0, 0, 0};

  for (;;) {
    const int nmb = (tc.rows + 15) >> 4;  // 16-row blocks holding rows
    v4f acc[8][NF];
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
      for (int f = 0; f < NF; ++f) acc[mi][f] = vzero;

    auto stage = [&](auto jc, const int st) {
      constexpr int J = decltype(jc)::value;
      // -- 1. consumers of earlier table loads, then table work of this stage
      if constexpr (J == 1) {
        if (st == 5 && w == 0) {
          const Tile t = resolve(__builtin_amdgcn_readfirstlane(__shfl(nidx, 0, 64)));
          if (lane == 0) write_tile(tb ^ 1, t);
        }
      }
      if constexpr (J == 2) {
        if (st == 10 && tn.valid && lane < RPW) {
          const int i = RPW * w + lane;
          sSlot[tb ^ 1][i] = nslot;
          if constexpr (KIND == KIND_DOWN) sRow[tb ^ 1][i] = out_row(tn, i, nslot);
        }
        if (st == 14 && tn.valid) {
          put_scales(tb ^ 1, nsb0, nsb1);
          if constexpr (KIND == KIND_GATE_UP)
            if (lane < RPW) sRow[tb ^ 1][RPW * w + lane] = (tn.e < args.E && args.route_w) ? nrw : 1.0f;
        }
      }
      if constexpr (J == 0) {
        // the slots stored at stage 10, behind the barrier that ends stage 11
        if (st == 12 && tn.valid) rows_of(ns, tn, tb ^ 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      // -- 2. activation stage st + 2 into LDS slot (J + 2) % 4 (and at J == 2
      //       the row scales of stages st + 2 .. st + 5)
      const int s2 = st + 2;
      {
        uint8_t* dst = sA + ((J + 2) & 3) * A_BYTES;
#pragma unroll
        for (int q = 0; q < AQ; ++q) *reinterpret_cast<uint4*>(dst + lds_a[q]) = aq[J & 1][q];
        if constexpr (J == 2) {
          const int grp = s2 < NST ? (s2 >> 2) : (NST >> 2);
          if (w < 2) *reinterpret_cast<float4*>(&sSa[(gpar + grp) & 1][(64 * w + lane) * 4]) = sq;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // -- 3. loads of activation stage st + 4 (at J == 0 also its row scales)
      const int s4 = st + 4;
      const bool cur4 = s4 < NST;
      {
        const uint32_t off = (uint32_t)(cur4 ? s4 : s4 - NST) * 128u;
#pragma unroll
        for (int q = 0; q < AQ; ++q) aq[J & 1][q] = ldA((cur4 ? cs.a[q] : ns.a[q]) + off);
        if constexpr (J == 0) {
          sq = ld_sa(cur4 ? cs.sa + s4 : ns.sa + (s4 - NST));
          if constexpr (W4) {
#pragma unroll
            for (int f = 0; f < NF; ++f) swn[f] = ldS(cur4 ? cs : ns, f, (cur4 ? s4 : s4 - NST) >> 2);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // -- 4. the MFMAs of stage st
      {
        const uint8_t* stg = sA + J * A_BYTES;
        const float* sS = &sSa[(gpar + (st >> 2)) & 1][0];
        const float sb0 = sSb[tb][bi][st];
        const float sb1 = KIND == KIND_GATE_UP ? sSb[tb][NJ + bi][st] : sb0;
        const int sbe0 = (int)(__float_as_uint(sb0) >> 23), sbe1 = (int)(__float_as_uint(sb1) >> 23);
        // software-pipelined over the 16-row blocks, each block a scheduling
        // region of its own (the compiler would otherwise hoist all eight
        // fragment reads and sixteen products at once and spill): block
        // mi + 1's fragment is read and block mi - 1 promoted while block
        // mi's MFMAs run.  Blocks past the tile's rows but within the body
        // are computed too (padding rows re-read the tile's first row; their
        // results are not stored).
        // NMB 16-row blocks: all eight, or the first four, two or one for a
        // tile of at most 64, 32 or 16 rows (an expert's short last tile; at
        // decode most tiles hold a few rows); the uniform branch picks one of
        // four straight-line bodies
        auto blocks = [&](auto nmb_c) {
          constexpr int NMB = decltype(nmb_c)::value;
          v8i af[2];
          v4f pr[2][NF];
          float sv[NMB];  // block mi's row scale, read one block ahead (three live at most)
          af[0] = read_frag(stg, fl);
          sv[0] = sS[r16 * 4 + J];
          __builtin_amdgcn_sched_barrier(0);
          auto promote = [&](int mi) {
            const int b = mi & 1;
            const float s0 = sv[mi] * sb0, s1 = sv[mi] * sb1;
#pragma unroll
            for (int f = 0; f < NF; ++f) {
              const float sf = f < NJ ? s0 : s1;
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[mi][f][r] = fmaf(pr[b][f][r], sf, acc[mi][f][r]);
              // keep the promotion here: left alone, the compiler sinks the
              // accumulator chains past the stage, keeps every product and spills
              asm volatile("" : "+v"(acc[mi][f]));
            }
          };
#pragma unroll
          for (int mi = 0; mi < NMB; ++mi) {
            const int b = mi & 1;
            if (mi + 1 < NMB) {
              af[b ^ 1] = read_frag(stg + (mi + 1) * 16 * 128, fl);
              sv[mi + 1] = sS[((mi + 1) * 16 + r16) * 4 + J];
            }
            if constexpr (W4) {
              // operand A = the fp4 weight fragment with its lane's e8m0
              // scale for this stage (byte J of the group's dword)
              const int sae = POW2 ? (int)(__float_as_uint(sv[mi]) >> 23) : 127;
#pragma unroll
              for (int f = 0; f < NF; ++f) {
                const int sw = (int)(swc[f] >> (8 * J));
                if constexpr (POW2)
                  acc[mi][f] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                      bq[J % DB][f], af[b], acc[mi][f], 4, 0, 0, sw, 0, sae);
                else
                  pr[b][f] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                      bq[J % DB][f], af[b], vzero, 4, 0, 0, sw, 0, sae);
              }
              if constexpr (!POW2)
                if (mi > 0) promote(mi - 1);
            } else if constexpr (POW2) {
              // operand A = the weight fragment (the block's scale), operand
              // B = the activation rows (lane r16's row scale, the same for
              // its four 32-deep K quarters)
              const int sae = (int)(__float_as_uint(sv[mi]) >> 23);
#pragma unroll
              for (int f = 0; f < NF; ++f)
                acc[mi][f] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    bq[J % DB][f], af[b], acc[mi][f], 0, 0, 0, f < NJ ? sbe0 : sbe1, 0, sae);
            } else {
#pragma unroll
              for (int f = 0; f < NF; ++f)
                pr[b][f] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bq[J % DB][f], af[b], vzero, 0,
                                                                            0, 0, 0, 0, 0);
              if (mi > 0) promote(mi - 1);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          if constexpr (!POW2) promote(NMB - 1);
        };
        if (nmb > 4) blocks(std::integral_constant<int, 8>{});
        else if (nmb > 2) blocks(std::integral_constant<int, 4>{});
        else if (nmb > 1) blocks(std::integral_constant<int, 2>{});
        else blocks(std::integral_constant<int, 1>{});
      }
      __builtin_amdgcn_sched_barrier(0);
      // -- 5. weight fragments of stage st + DB into the freed registers
      {
        const int sb_ = st + DB;
        const bool curb = sb_ < NST;
        const uint32_t off = (uint32_t)(curb ? sb_ : sb_ - NST) * WBLK;
#pragma unroll
        for (int f = 0; f < NF; ++f) bq[J % DB][f] = ldBf(curb ? cs : ns, f, off);
      }
      if constexpr (W4 && J == 3) {
        // the next group's scale dwords (loaded at this group's stage 0)
#pragma unroll
        for (int f = 0; f < NF; ++f) swc[f] = swn[f];
      }
      __builtin_amdgcn_sched_barrier(0);
      // -- 6. table loads for the next tile (consumed four stages later; the
      //       stage-10 block precedes the stage-6 one, so no path runs from
      //       the slot loads to their use without passing four stages)
      if constexpr (J == 2) {
        if (st == 10 && tn.valid) {
          weights_of(ns, tn, nsb0, nsb1);
          if constexpr (KIND == KIND_GATE_UP)
            if (lane < RPW && tn.e < args.E && args.route_w) nrw = args.route_w[nslot];
        }
        if (st == 6) {
          tn = read_tile(tb ^ 1);
          if (tn.valid && lane < RPW) {
            const int i = RPW * w + lane;
            nslot = (tn.e < args.E && i < tn.rows) ? args.sorted_slot[tn.row0 + i] : 0;
          }
        }
      }
      // a barrier every second stage suffices: slot (J + 2) & 3, written in
      // this stage, was last read two stages ago, and is read two stages
      // from now; a barrier at the end of every odd stage lies between each
      // such pair of accesses.  The table stages read what an earlier stage
      // stored across such a barrier: 6 reads 5's tile, 12 reads 10's slots,
      // the next tile reads 14's scales and routing weights.
      if constexpr (J & 1) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    for (int st0 = 0; st0 < NST; st0 += 4) {
      stage(std::integral_constant<int, 0>{}, st0);
      stage(std::integral_constant<int, 1>{}, st0 + 1);
      stage(std::integral_constant<int, 2>{}, st0 + 2);
      stage(std::integral_constant<int, 3>{}, st0 + 3);
    }

    // ---- epilogue from registers
    const int rows = tc.rows;
    if constexpr (KIND == KIND_DOWN) {
      const int64_t n0 = (int64_t)tc.nt * TC + 16 * NF * w;
#pragma unroll
      for (int mi = 0; mi < 8; ++mi) {
        const int row = mi * 16 + r16;
        if (row < rows) {
          const int64_t drow = __float_as_int(sRow[tb][row]);
#pragma unroll
          for (int f = 0; f < NF; ++f) {
            const int64_t col = n0 + 16 * f + 4 * g4;
            if (col < N) {
              const v4f v = acc[mi][f];
              store_b64(reinterpret_cast<uint16_t*>(args.c) + drow * N + col,
                        make_uint2(pk2_bf16_exact(v[0], v[1]), pk2_bf16_exact(v[2], v[3])));
            }
          }
        }
      }
    } else {
      // SwiGLU + 1x128 requant (as gemm_pipe_kernel): h kept as packed bf16
      // pairs across the barrier that publishes the row maxima
      const float lim = args.swiglu_limit;
      uint32_t h2[8][2 * NJ];
      auto swiglu = [&](auto clamp_c) {
        constexpr bool CLAMP = decltype(clamp_c)::value;
#pragma unroll
        for (int mi = 0; mi < 8; ++mi) {
          const int row = mi * 16 + r16;
          const float wr = sRow[tb][row];
          float am = 0.0f;
#pragma unroll
          for (int q = 0; q < 4 * NJ; ++q) {
            const int j = q >> 2, r = q & 3;
            float gt = bf16_round(acc[mi][j][r]);
            float up = bf16_round(acc[mi][NJ + j][r]);
            if constexpr (CLAMP) {
              up = clampf_(up, -lim, lim);
              gt = gt > lim ? lim : gt;
            }
            const float ex = __builtin_amdgcn_exp2f(gt * -1.4426950408889634f);
            const float silu = gt * __builtin_amdgcn_rcpf(1.0f + ex);
            const uint32_t hb = bf16_bits_exact(wr * (silu * up));
            if (q & 1)
              h2[mi][q >> 1] |= hb << 16;
            else
              h2[mi][q >> 1] = hb;
            am = __builtin_elementwise_maximum(am, fabsf(bits_f32(hb << 16)));
          }
          am = __builtin_elementwise_maximum(am, __shfl_xor(am, 16, 64));
          am = __builtin_elementwise_maximum(am, __shfl_xor(am, 32, 64));
          if (g4 == 0) sAmax[w][row] = am;
          // one row block at a time: a spill here would be a scratch access,
          // whose wait drains the next tile's loads in flight
#pragma unroll
          for (int q = 0; q < 2 * NJ; ++q) asm volatile("" : "+v"(h2[mi][q]));
        }
      };
      if (lim > 0.0f) swiglu(std::true_type{});
      else swiglu(std::false_type{});
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const int64_t NBK = N / 128;
      const int64_t n0 = (int64_t)tc.nt * GC;
      const bool in_n = n0 + 16 * NJ * w < N;  // the wavefront's columns exist
      auto requant = [&](auto mode_c) {
        constexpr int MODE = decltype(mode_c)::value;
#pragma unroll
        for (int mi = 0; mi < 8; ++mi) {
          const int row = mi * 16 + r16;
          if (row < rows && in_n) {
            // the row's maximum over the 128 columns of this wavefront's block
            float am = sAmax[bi * WPB][row];
#pragma unroll
            for (int q = 1; q < WPB; ++q) am = __builtin_elementwise_maximum(am, sAmax[bi * WPB + q][row]);
            const float sf = group_scale(MODE, am);
            const int64_t p = tc.row0 + row;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              float hf[4];
#pragma unroll
              for (int q = 0; q < 2; ++q) {
                hf[2 * q] = bits_f32(h2[mi][2 * j + q] << 16);
                hf[2 * q + 1] = bits_f32(h2[mi][2 * j + q] & 0xFFFF0000u);
              }
              store_b32(args.hq + p * N + n0 + 16 * (NJ * w + j) + 4 * g4, quant4_e4m3(MODE, hf, sf));
            }
            if (w % WPB == 0 && g4 == 0)
              store_b32(args.hs + p * NBK + tc.nt * NJ + bi, __float_as_uint(sf));
          }
        }
      };
      switch (args.scale_mode) {
        case SCALE_TORCH_FP32: requant(std::integral_constant<int, SCALE_TORCH_FP32>{}); break;
        case SCALE_TORCH_UE8M0: requant(std::integral_constant<int, SCALE_TORCH_UE8M0>{}); break;
        case SCALE_TILELANG_FP32: requant(std::integral_constant<int, SCALE_TILELANG_FP32>{}); break;
        default: requant(std::integral_constant<int, SCALE_TILELANG_UE8M0>{}); break;
      }
    }
    if (!tn.valid) break;
    if (w == 0 && lane == 0) nidx = take_tile();  // the tile after the next one
    tc = tn;
    cs = ns;
    tb ^= 1;
    gpar = (gpar + (NST >> 2)) & 1;
  }
}

#ifndef SGL_RB_NJ
#define SGL_RB_NJ 1
#endif
// CUs a grouped launch fills, rounded up to a multiple of 8 so every XCD
// gets the same number
int64_t cu_budget(const GemmArgs&) {
  const int64_t n = device_cu_count();
  return std::max<int64_t>(8, (n + 7) / 8 * 8);
}

template <int KIND, bool W4 = false>
int launch_rb(GemmArgs& a, int64_t rows_hint, hipStream_t stream) {
  using namespace rb;
  a.n_tiles = (int)ceil_div(a.N, (KIND == KIND_GATE_UP ? 128 : 256) * SGL_RB_NJ);
  const int64_t P = a.E > 0 ? a.T * a.k : 0;
  const int64_t mt_bound = P / BM + (P < a.E ? P : a.E) + (a.has_shared ? ceil_div(a.T, BM) : 0);
  const int64_t tiles = mt_bound * a.n_tiles;
  if (tiles == 0) return SGL_OK;
  int64_t wgs = cu_budget(a);
  const int64_t need = (tiles + 7) / 8 * 8;
  if (need < wgs) wgs = need;
  a.m_tiles = (int)mt_bound;
  // nontemporal weight loads at decode sizes (fewer than 64 rows per expert
  // on average); prefill tiles of one expert share its weights through L2
  const bool nt = SGL_NT_WEIGHTS && rows_hint < 64;
#define SGL_RB_LAUNCH(POW2_, W4_)                                                             \
  do {                                                                                        \
    if (nt)                                                                                   \
      gemm_rb_kernel<KIND, W4_ ? 1 : SGL_RB_NJ, POW2_, W4_, true><<<(unsigned)wgs, 512, 0,   \
                                                                    stream>>>(a);            \
    else                                                                                      \
      gemm_rb_kernel<KIND, W4_ ? 1 : SGL_RB_NJ, POW2_, W4_, false><<<(unsigned)wgs, 512, 0,  \
                                                                     stream>>>(a);           \
  } while (0)
  if constexpr (W4) {
    // fp4 weights: their scales always in the MFMA; the row scales too when
    // they are powers of two
    if (a.sa_pow2)
      SGL_RB_LAUNCH(true, true);
    else
      SGL_RB_LAUNCH(false, true);
  } else if (a.sa_pow2 && a.sb_pow2) {
    SGL_RB_LAUNCH(true, false);
  } else {
    SGL_RB_LAUNCH(false, false);
  }
#undef SGL_RB_LAUNCH
  return check_launch("gemm_rb");
}

// Packed e2m1 [N, K/2] with e8m0 scales [N, K/32] -> the FP4 fragment layout:
// weights 1 KB per (16-row block n16, 128-deep block kb), block index
// n16 * K/128 + kb, byte 16 l + b of a block holding packed byte
// 64 kb + 16 (l / 16) + b of row 16 n16 + l % 16 (lane l's 32 values, K
// [32 (l / 16), +32) of the block); scales 256 bytes per (n16, group q of
// four 128-deep blocks), block index n16 * K/512 + q, byte 4 l + j holding
// the scale of row 16 n16 + l % 16 for its 32-deep block 16 q + 4 j + l / 16
// (lane l's scale for stage 4 q + j).
__global__ __launch_bounds__(256) void weight_fp4_to_frag_kernel(const uint8_t* __restrict__ w,
                                                                 const uint8_t* __restrict__ s,
                                                                 int64_t N, int64_t K,
                                                                 uint8_t* __restrict__ ow,
                                                                 uint8_t* __restrict__ os) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t KB = K / 128, KR = K / 2;
  const int64_t nw = N * KR / 16;  // 16-byte weight chunks
  if (i < nw) {
    const int64_t blk = i >> 6;
    const int l = (int)(i & 63);
    const int64_t n16 = blk / KB, kb = blk - n16 * KB;
    const int64_t n = n16 * 16 + (l & 15);
    *reinterpret_cast<uint4*>(ow + i * 16) =
        *reinterpret_cast<const uint4*>(w + n * KR + kb * 64 + (l >> 4) * 16);
    return;
  }
  const int64_t d = i - nw;  // scale dword
  if (d >= N * KB) return;
  const int64_t blk = d >> 6;
  const int l = (int)(d & 63);
  const int64_t NQ = KB / 4;
  const int64_t n16 = blk / NQ, q = blk - n16 * NQ;
  const int64_t n = n16 * 16 + (l & 15);
  const uint8_t* srow = s + n * (K / 32) + 16 * q + (l >> 4);
  *reinterpret_cast<uint32_t*>(os + d * 4) =
      (uint32_t)srow[0] | ((uint32_t)srow[4] << 8) | ((uint32_t)srow[8] << 16) | ((uint32_t)srow[12] << 24);
}

// [N, K] e4m3 row-major -> the MFMA fragment layout: 2 KB per (16-row block
// n16, 128-deep block kb), block index n16 * K/128 + kb; byte
// j * 1024 + 16 l + b of a block holds row 16 n16 + l % 16, column
// 128 kb + 32 (l / 16) + 16 j + b (lane l's bytes of the operand, as
// read_frag assembles them from an LDS stage).
__global__ __launch_bounds__(256) void weight_to_frag_kernel(const uint8_t* __restrict__ w, int64_t N,
                                                             int64_t K, uint8_t* __restrict__ out) {
  const int64_t chunk = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte output chunk
  if (chunk >= N * K / 16) return;
  const int64_t KB = K / 128;
  const int64_t blk = chunk >> 7;
  const int j = (int)((chunk >> 6) & 1), l = (int)(chunk & 63);
  const int64_t n16 = blk / KB, kb = blk - n16 * KB;
  const int64_t n = n16 * 16 + (l & 15);
  const int64_t k = kb * 128 + (l >> 4) * 32 + j * 16;
  *reinterpret_cast<uint4*>(out + chunk * 16) = *reinterpret_cast<const uint4*>(w + n * K + k);
}

// ------------------------------------------------------------ wide tiles
// Dense products from M = 2048 up: 256 x 256 tiles, eight wavefronts (4 x 2,
// 64 x 128 each, two per SIMD with 256 registers) and a 2-slot ring of 64 KB
// stages.  Per 128-deep stage a CU moves 64 KB into LDS for 16.8 MFLOP (the
// 128 x 256 tile moves 48 KB for 8.4), so the operand path carries two thirds
// of the bytes per MFMA, and each stage barrier is amortized over 32 MFMAs
// per wavefront.  Wavefronts 4..7 (one per SIMD) issue the stage DMAs: stage
// st + 1 right after the barrier of stage st, into the slot stage st - 1
// used, so one stage's loads fly while the other stage is computed.  The
// promotion and its order are those of gemm_fp8_kernel, so the output is
// bit-identical to the 128 x 256 tiles (N = 4096, K = 7168, M = 4096:
// 175 -> 135 us).
namespace wide {
constexpr int BM = 256, BN = 256, WM = 4, WN = 2, TM = 4, TN = 8, NW = 8, NT = 64 * NW;
constexpr int IW = 4;                                    // DMA issuers: wavefronts 4..7
constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128, STAGE = A_BYTES + B_BYTES;
constexpr int RING = 2 * STAGE;
constexpr int SA_SLOT = BM * 4;                          // row scales of one stage
constexpr int SMEM = RING + 2 * SA_SLOT;
constexpr int ACH = BM / 8, BCH = BN / 8;                // 1 KB chunks per stage
constexpr int QA = ACH / IW, QB = BCH / IW;              // per issuer
static_assert(WM * TM * 16 == BM && WN * TN * 16 == BN && WM * WN == NW, "wavefront grid");
static_assert(IW * 64 == BM, "one row-scale DMA per issuer and stage");
static_assert(TN * 16 == 128, "a wavefront's columns are one 128-column weight-scale block");
}  // namespace wide

// SAF: the scale formats, one instantiation each (their register allocations
// stay apart): 0 fp32 row scales, promoted; 1 e8m0 row scales (bytes),
// promoted; 2 e8m0 row and weight scales, both applied inside the MFMA
template <int SAF>
__global__ __launch_bounds__(wide::NT) void gemm_wide_kernel(const GemmArgs args) {
  constexpr bool POW2 = SAF == 2;
  using namespace wide;
  __shared__ __align__(16) uint8_t smem[SMEM];
  __shared__ float sSb[2][kMaxKB];  // the tile's weight scales: column block j, K block kb

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const bool issuer = wave >= NW - IW;
  const int iw = issuer ? wave - (NW - IW) : 0;
  const int g4 = lane >> 4, r16 = lane & 15;
  const FragLane fl = frag_lane(r16, g4);
  const int64_t K = args.K, N = args.N, M = args.M;
  const int KB = (int)(K / 128);
  const int NST = KB;
  const int total_mt = (int)((M + BM - 1) / BM);
  const int total = total_mt * args.n_tiles;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per_xcd = gridDim.x >> 3;
  const int per = (total + 7) >> 3;
  const int t_begin = xcd * per;
  const int t_end = min(t_begin + per, total);

  const uint8_t* baseA = uniform_ptr(args.a);
  const uint8_t* baseB = uniform_ptr(args.b);
  const uint8_t* sa_base = uniform_ptr(args.sa);
  const uint32_t smem_lds = __builtin_amdgcn_readfirstlane(lds_u32(smem));
  // issuer iw moves chunks iw + IW q of A (rows 8 c ..) and of B; with IW
  // even every chunk of an issuer has the swizzle parity of iw, so one lane
  // offset (row rr of the chunk, the lane's swizzled 16-byte piece) serves
  // all of them; the chunk's first row is a wave-uniform base
  const int rr = lane >> 3, pc = lane & 7;
  const uint32_t chunk = (uint32_t)((pc ^ ((rr & 6) | (iw & 1))) << 4);
  const uint32_t lane_off = (uint32_t)(rr * K) + chunk;
  const v4f vzero = {0.0f, 0.0f, 0.0f, 0.0f};
  int gst = 0;  // stages issued before this tile: stage st of the tile uses ring slot (gst + st) & 1

  for (int iter = 0;; ++iter) {
    const int L = t_begin + slot + iter * per_xcd;
    if (L >= t_end) break;
    // N-slice major, the M tiles of a slice adjacent (one XCD's L2 holds the slice)
    const int nt = L / total_mt;
    const int mt = L - nt * total_mt;
    const int row0 = mt * BM;
    const int rows = (int)min((int64_t)BM, M - row0);
    const int64_t n0 = (int64_t)nt * BN;

    __syncthreads();  // the previous tile's readers of sSb are done
    for (int i = tid; i < 2 * KB; i += NT) {
      const int j = i / KB, kb = i - j * KB;
      const int64_t nb = (N + 127) / 128;
      int64_t blk = n0 / 128 + j;
      if (blk > nb - 1) blk = nb - 1;
      sSb[j][kb] = load_scale(args.sb, blk * KB + kb, args.sb_e8m0);
    }
    // A chunks wholly past the tile's last row and B chunks past N (N % 16
    // == 0: chunks are wholly in or out) are not loaded: those rows only
    // feed outputs that are never stored
    const int sa_r = iw * 64 + lane;
    constexpr bool sa_e8 = SAF != 0;  // e8m0 row scales: the aligned dwords that hold them
    const uint32_t sa_off = (uint32_t)((int64_t)(row0 + (sa_r < rows ? sa_r : rows - 1)) * KB * (sa_e8 ? 1 : 4));
    auto issue = [&](int st) {
      if (!issuer) return;
      const int s = (gst + st) & 1;
      const uint32_t sl = smem_lds + (uint32_t)(s * STAGE);
#pragma unroll
      for (int q = 0; q < QA; ++q) {
        const int c = iw + q * IW;
        if (c * 8 < rows) {
          const uint32_t vo = c * 8 + 8 <= rows ? lane_off
                                                : (uint32_t)(min(rr, rows - 1 - c * 8) * K) + chunk;
          dma16(baseA + ((int64_t)(row0 + c * 8) * K + st * 128), vo, sl + (uint32_t)c * 1024u);
        }
      }
#pragma unroll
      for (int q = 0; q < QB; ++q) {
        const int b = iw + q * IW;
        const int64_t nrow = n0 + b * 8;
        if (nrow < N) dma16(baseB + (nrow * K + st * 128), lane_off, sl + (uint32_t)(A_BYTES + b * 1024));
      }
      if (sa_e8)  // the aligned dword holding the byte
        dma4(sa_base, (sa_off + (uint32_t)st) & ~3u, smem_lds + (uint32_t)(RING + s * SA_SLOT + iw * 256));
      else
        dma4(sa_base, sa_off + (uint32_t)st * 4u, smem_lds + (uint32_t)(RING + s * SA_SLOT + iw * 256));
    };
    __syncthreads();  // sSb published
    issue(0);

    // wavefront (wm, wn): rows (wm TM + mi) 16 .., columns wn 128 + 16 nj ..
    v4f acc[TM][TN];
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
      for (int nj = 0; nj < TN; ++nj) acc[mi][nj] = vzero;
    const bool active = (wm * TM) * 16 < rows;

    for (int st = 0; st < NST; ++st) {
      // the issuers' stage-st loads are the only ones in flight
      wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      if (st + 1 < NST) issue(st + 1);
      const int s = (gst + st) & 1;
      const uint8_t* stg = smem + s * STAGE;
      const uint8_t* tB = stg + A_BYTES + (wn * TN * 16) * 128;
      const float* tS = reinterpret_cast<const float*>(smem + RING + s * SA_SLOT);
      if (active) {
        // fragments in MFMA order (A0, B0 and the scales, then A1..A3);
        // the weight fragment of block nj + 1 is read while the MFMAs of
        // block nj run.  Transposed product (weight fragment = MFMA A
        // operand): lane (g4, r16) accumulates row r16 of each 16-row block
        // and columns 4 g4 .. + 3 of each 16-column block, so one row scale
        // per lane and block and one weight scale per wavefront
        v8i af[TM];
        v8i bf[2];
        float sa1[TM];
        af[0] = read_frag(stg + (wm * TM) * 16 * 128, fl);
        bf[0] = read_frag(tB, fl);
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) sa1[mi] = tS[(wm * TM + mi) * 16 + r16];
        const float sb = sSb[wn][st];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mi = 1; mi < TM; ++mi) af[mi] = read_frag(stg + (wm * TM + mi) * 16 * 128, fl);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (sa_e8) {
          // e8m0 row scales: the byte (source row) KB + st of the scale
          // tensor, from the aligned dword the DMA staged, is the exponent
          // the MFMA takes (activation rows = operand B, lane r16's row).
          // SAF 2: the weight scale's too (operand A, one per wavefront),
          // accumulating in place; SAF 1: C += P' sb, which is the
          // promotion's C += P (sa sb) to the bit
          int sae[TM];
#pragma unroll
          for (int mi = 0; mi < TM; ++mi) {
            const int row = (wm * TM + mi) * 16 + r16;
            const int src = row0 + (row < rows ? row : rows - 1);
            sae[mi] = (int)((__float_as_uint(sa1[mi]) >> (((uint32_t)(src * KB + st) & 3u) * 8u)) & 0xFFu);
          }
          const int sbe = POW2 ? (int)(__float_as_uint(sb) >> 23) : 127;
#pragma unroll
          for (int nj = 0; nj < TN; ++nj) {
            if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + (nj + 1) * 16 * 128, fl);
            if constexpr (POW2) {
#pragma unroll
              for (int mi = 0; mi < TM; ++mi)
                acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[nj & 1], af[mi], acc[mi][nj],
                                                                               0, 0, 0, sbe, 0, sae[mi]);
            } else {
              v4f pr[TM];
#pragma unroll
              for (int mi = 0; mi < TM; ++mi)
                pr[mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[nj & 1], af[mi], vzero, 0, 0, 0,
                                                                          sbe, 0, sae[mi]);
#pragma unroll
              for (int mi = 0; mi < TM; ++mi)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[mi][nj][r] = fmaf(pr[mi][r], sb, acc[mi][nj][r]);
            }
          }
          continue;
        }
        float ss[TM];
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) ss[mi] = sa1[mi] * sb;
#pragma unroll
        for (int nj = 0; nj < TN; ++nj) {
          if (nj + 1 < TN) bf[(nj + 1) & 1] = read_frag(tB + (nj + 1) * 16 * 128, fl);
          v4f pr[TM];
#pragma unroll
          for (int mi = 0; mi < TM; ++mi)
            pr[mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[nj & 1], af[mi], vzero, 0, 0, 0,
                                                                      0, 0, 0);
          // C += P (sa sb), one FMA per output per K block
#pragma unroll
          for (int mi = 0; mi < TM; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mi][nj][r] = fmaf(pr[mi][r], ss[mi], acc[mi][nj][r]);
        }
      }
    }
    gst += NST;

    // lane (g4, r16): row (wm TM + mi) 16 + r16, columns wn 128 + 16 nj + 4 g4 .. + 3
    const bool f32out = args.out_f32;
    if (active) {
#pragma unroll
      for (int mi = 0; mi < TM; ++mi) {
        const int row = (wm * TM + mi) * 16 + r16;
        if (row < rows) {
          const int64_t drow = row0 + row;
#pragma unroll
          for (int nj = 0; nj < TN; ++nj) {
            const int64_t col = n0 + (wn * TN + nj) * 16 + 4 * g4;
            if (col < N) {
              const v4f v = acc[mi][nj];
              if (f32out)
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(args.c) + drow * N + col) =
                    make_float4(v[0], v[1], v[2], v[3]);
              else
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(args.c) + drow * N + col) =
                    make_uint2(pk2_bf16_exact(v[0], v[1]), pk2_bf16_exact(v[2], v[3]));
            }
          }
        }
      }
    }
  }
}

int launch_wide(GemmArgs& a, hipStream_t stream) {
  using namespace wide;
  a.n_tiles = (int)ceil_div(a.N, BN);
  const int64_t mt = ceil_div(a.M, BM);
  const int64_t tiles = mt * a.n_tiles;
  if (tiles == 0) return SGL_OK;
  constexpr int kLds = SMEM + 2 * kMaxKB * 4;
  static_assert(kLds <= 160 * 1024, "wide tile exceeds the LDS of a CU");
  int64_t wgs = (int64_t)device_cu_count();
  wgs = (wgs + 7) / 8 * 8;
  const int64_t need = (tiles + 7) / 8 * 8;
  if (need < wgs) wgs = need;
  a.m_tiles = (int)mt;
  if (a.sa_e8m0 && a.sb_e8m0)
    gemm_wide_kernel<2><<<(unsigned)wgs, NT, 0, stream>>>(a);
  else if (a.sa_e8m0)
    gemm_wide_kernel<1><<<(unsigned)wgs, NT, 0, stream>>>(a);
  else
    gemm_wide_kernel<0><<<(unsigned)wgs, NT, 0, stream>>>(a);
  return check_launch("gemm_wide");
}

template <int KIND, int BM, int BN, int WM, int WN, int NSTAGE, int WF = WF_FP8, bool SAHW = false,
          int LW = 0>
int launch_cfg(GemmArgs& a, hipStream_t stream) {
  const int64_t half = KIND == KIND_GATE_UP ? BN / 2 : BN;
  a.n_tiles = (int)ceil_div(a.N, half);
  int64_t mt_bound;
  if constexpr (KIND == KIND_DENSE) {
    mt_bound = ceil_div(a.M, BM);
  } else {
    const int64_t P = a.E > 0 ? a.T * a.k : 0;
    mt_bound = P / BM + (P < a.E ? P : a.E) + (a.has_shared ? ceil_div(a.T, BM) : 0);
  }
  const int64_t tiles = mt_bound * a.n_tiles;
  if (tiles == 0) return SGL_OK;
  // persistent: as many workgroups per CU as their LDS allows (the 160 KB
  // of a CU), a multiple of 8 so every XCD gets the same number
  using C = Cfg<KIND, BM, BN, WM, WN, NSTAGE, WF, SAHW, LW>;
  constexpr int kLdsPerCU = 160 * 1024;
  constexpr int kExtra = (KIND == KIND_DENSE ? 4 : 4 * (kMaxGroups + 1)) + BM * 12 +
                         2 * (WF == WF_FP4 ? 1 : kMaxKB) * 4 +
                         (KIND == KIND_GATE_UP && LW > 0 ? WN * BM * 4 : 4);
  static_assert(C::SMEM + kExtra <= kLdsPerCU, "tile configuration exceeds the LDS of a CU");
  constexpr int per_cu = kLdsPerCU / (C::SMEM + kExtra) >= 2 ? 2 : 1;
  int64_t wgs = cu_budget(a) * per_cu;
  const int64_t need = (tiles + 7) / 8 * 8;
  if (need < wgs) wgs = need;
  a.m_tiles = (int)mt_bound;
  gemm_fp8_kernel<KIND, BM, BN, WM, WN, NSTAGE, WF, SAHW, LW><<<(unsigned)wgs, C::NT, 0, stream>>>(a);
  return check_launch("gemm_fp8");
}

// ---------------------------------------------------------------- skinny
// Dense GEMM for small M (M <= 256): one workgroup per 16-column slab of B
// and (16 TM)-row tile of A, split over K inside the workgroup.  Wavefront w
// of the W (16, or 8 for the 64-row tile) takes K blocks w, w + W, ...; every lane loads its MFMA
// operands straight from global memory (row l % 16, bytes [32 (l/16), +32) of
// the block: two 16-byte loads per operand) one block ahead, promotes each
// block partial with the row and weight scales staged in LDS, and the 16
// partial tiles are summed through LDS at the end.  B, the weight stream, is
// read once (per row tile); the grid holds N/16 x ceil(M / 16 TM) workgroups,
// enough to keep every CU streaming where the 128 x 256 tiles leave most idle.
#ifndef SGL_LW
#define SGL_LW 4
#endif
#ifndef SGL_RB
#define SGL_RB 1
#endif
#ifndef SGL_PIPE
#define SGL_PIPE 1
#endif
#ifndef SGL_LWN
#define SGL_LWN 4
#endif
#ifndef SGL_SPLITK
#define SGL_SPLITK 1
#endif
#ifndef SGL_SKINNY_MAX_M
#define SGL_SKINNY_MAX_M 64
#endif
// dense GEMMs up to this M take the skinny kernel (measured crossover with
// the 64 x 128 tiles)
constexpr int64_t kSkinnyMaxM = SGL_SKINNY_MAX_M;
template <int TM>
struct Skinny {
  static constexpr int WAVES = TM >= 4 ? 8 : 16;  // 64-row tiles need the 256-VGPR budget
};

__device__ __forceinline__ v8i load_frag_global(const uint8_t* p) {
  const uint4 lo = *reinterpret_cast<const uint4*>(p);
  const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
  return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

template <int TM, int WF, bool SAHW>
__global__ __launch_bounds__(64 * Skinny<TM>::WAVES) void gemm_skinny_kernel(const GemmArgs args) {
  constexpr int ROWS = 16 * TM;
  constexpr int kSkinnyWaves = Skinny<TM>::WAVES;
  constexpr bool FP4 = WF == WF_FP4;
  __shared__ float sSa[ROWS][kMaxKB];
  __shared__ float sSk[FP4 ? 1 : kMaxKB];             // fp8: the slab's weight scale per K block
  __shared__ uint32_t sSb4[FP4 ? 16 : 1][kMaxKB];     // fp4: 4 e8m0 scales per column and K block
  __shared__ float sRed[kSkinnyWaves][ROWS * 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, r16 = lane & 15;
  const int64_t M = args.M, N = args.N, K = args.K;
  const int KB = (int)(K / 128);
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t m0 = (int64_t)blockIdx.y * ROWS;

  // operand rows of this lane (rows past M re-read row M-1; their outputs are
  // dropped).  fp8: A and B bytes [32 g4, +32) of each K block; fp4: A bytes
  // [16 g4, +16) and [64 + 16 g4, +16), B packed bytes [16 g4, +16).
  const uint8_t* arow[TM];
#pragma unroll
  for (int mi = 0; mi < TM; ++mi) {
    int64_t row = m0 + 16 * mi + r16;
    if (row > M - 1) row = M - 1;
    arow[mi] = args.a + row * K + (FP4 ? 16 : 32) * g4;
  }
  const int64_t KROW = FP4 ? K / 2 : K;
  const uint8_t* brow = args.b + (n0 + r16) * KROW + (FP4 ? 16 : 32) * g4;

  // Scale loads are issued first and the first NB operand blocks right
  // after, so waiting for the scales (to stage them in LDS) leaves the
  // operand loads in flight: loads retire in issue order.
  constexpr int SPT = (ROWS * kMaxKB + 64 * kSkinnyWaves - 1) / (64 * kSkinnyWaves);
  float sv[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    const int i = tid + j * 64 * kSkinnyWaves;
    const int r = i / KB, kb = i - r * KB;
    const int64_t row = m0 + r;
    sv[j] = (i < ROWS * KB && row < M) ? load_scale(args.sa, row * KB + kb, args.sa_e8m0) : 0.0f;
  }
  float skv = 0.0f;
  constexpr int BPT = FP4 ? (16 * kMaxKB + 64 * kSkinnyWaves - 1) / (64 * kSkinnyWaves) : 1;
  uint32_t sbw[BPT];
  if constexpr (FP4) {
    // dword kb of column c holds the e8m0 scales of its four 32-deep blocks
    const uint32_t* sb = reinterpret_cast<const uint32_t*>(args.sb);
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int i = tid + j * 64 * kSkinnyWaves;
      const int c = i / KB, kb = i - c * KB;
      sbw[j] = i < 16 * KB ? sb[(n0 + c) * KB + kb] : 0u;
    }
  } else {
    if (tid < KB) skv = load_scale(args.sb, (n0 / 128) * KB + tid, args.sb_e8m0);
  }

  // K blocks per wavefront whose loads are in flight together (the 128-row
  // tile holds 8 A fragments per block, so two blocks fit the VGPR budget)
  constexpr int NB = TM >= 8 ? 2 : 4;
  v8i af[NB][TM], bf[NB];
  auto load_chunk = [&](int base) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int kb = base + j * kSkinnyWaves;
      if (kb < KB) {
        if constexpr (FP4) {
#pragma unroll
          for (int mi = 0; mi < TM; ++mi) {
            const uint4 lo = *reinterpret_cast<const uint4*>(arow[mi] + (int64_t)kb * 128);
            const uint4 hi = *reinterpret_cast<const uint4*>(arow[mi] + (int64_t)kb * 128 + 64);
            af[j][mi] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
          }
          const uint4 v = *reinterpret_cast<const uint4*>(brow + (int64_t)kb * 64);
          bf[j] = v8i{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
        } else {
#pragma unroll
          for (int mi = 0; mi < TM; ++mi) af[j][mi] = load_frag_global(arow[mi] + (int64_t)kb * 128);
          bf[j] = load_frag_global(brow + (int64_t)kb * 128);
        }
      }
    }
  };
  load_chunk(wave);

#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    const int i = tid + j * 64 * kSkinnyWaves;
    if (i < ROWS * KB) sSa[i / KB][i - (i / KB) * KB] = sv[j];
  }
  if constexpr (FP4) {
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int i = tid + j * 64 * kSkinnyWaves;
      if (i < 16 * KB) sSb4[i / KB][i - (i / KB) * KB] = sbw[j];
    }
  } else {
    if (tid < KB) sSk[tid] = skv;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();

  v4f acc[TM];
#pragma unroll
  for (int mi = 0; mi < TM; ++mi) acc[mi] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const v4f vzero = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int base = wave; base < KB; base += NB * kSkinnyWaves) {
    if (base != wave) load_chunk(base);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int kb = base + j * kSkinnyWaves;
      if (kb < KB) {
        if constexpr (FP4) {
          const int sbb = (int)(sSb4[r16][kb] >> (8 * g4));
#pragma unroll
          for (int mi = 0; mi < TM; ++mi) {
            if constexpr (SAHW) {
              const int sae = (int)(__float_as_uint(sSa[16 * mi + r16][kb]) >> 23);
              acc[mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[j][mi], bf[j], acc[mi], 0, 4,
                                                                        0, sae, 0, sbb);
            } else {
              const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[j][mi], bf[j], vzero, 0,
                                                                             4, 0, 127, 0, sbb);
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[mi][r] = fmaf(p[r], sSa[16 * mi + 4 * g4 + r][kb], acc[mi][r]);
            }
          }
        } else {
          const float sk = sSk[kb];
#pragma unroll
          for (int mi = 0; mi < TM; ++mi) {
            const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[j][mi], bf[j], vzero, 0,
                                                                           0, 0, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[mi][r] = fmaf(p[r], sSa[16 * mi + 4 * g4 + r][kb] * sk, acc[mi][r]);
          }
        }
      }
    }
  }

  // sum the partial tiles; lane (g4, r16) holds rows 4 g4 + r, column r16
#pragma unroll
  for (int mi = 0; mi < TM; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) sRed[wave][(16 * mi + 4 * g4 + r) * 16 + r16] = acc[mi][r];
  __syncthreads();
  for (int i = tid; i < ROWS * 16; i += 64 * kSkinnyWaves) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w) v += sRed[w][i];
    const int64_t row = m0 + i / 16;
    const int64_t col = n0 + (i & 15);
    if (row < M) {
      if (args.out_f32)
        reinterpret_cast<float*>(args.c)[row * N + col] = v;
      else
        reinterpret_cast<uint16_t*>(args.c)[row * N + col] = bf16_bits_exact(v);
    }
  }
}

template <int TM, int WF = WF_FP8, bool SAHW = false>
int launch_skinny(GemmArgs& a, hipStream_t stream) {
  dim3 grid((unsigned)(a.N / 16), (unsigned)ceil_div(a.M, (int64_t)(16 * TM)));
  gemm_skinny_kernel<TM, WF, SAHW><<<grid, 64 * Skinny<TM>::WAVES, 0, stream>>>(a);
  return check_launch(WF == WF_FP4 ? "gemm_fp4_skinny" : "gemm_fp8_skinny");
}

// ---- small-M dense GEMM, split over K
//
// 16 < M <= 64 rows against an N x K weight: the work is streaming B (N K
// bytes from HBM).  A workgroup that spans all of K also reads all of A (M K
// bytes, twice its B strip at M = 64) from L2, so the grid is N/128 column
// tiles x S K ranges of KS blocks, about one workgroup per CU, each reading
// only its M x KS x 128 slice of A.  The slice and the scales go to LDS by LDS
// DMA (the ring kernels' fragment layout; the DMAs are invisible to the
// compiler, which would otherwise drain every load in flight before its first
// LDS write); each of the 8 wavefronts owns 16 columns and loads their B
// fragments from HBM straight into registers, all KS blocks in flight, then
// runs the K blocks in order as they land (per block: the MFMA partial
// promoted with sa sb in fp32, as everywhere).  The fp32 tile partials go to
// a workspace and splitk_reduce_kernel, over the whole GPU, sums them in split
// order: C is the same bytes on every run.  (N = 4096, K = 7168 at M = 64: 12
// us + 4 us, against 22.6 us for the unsplit kernel.  At M <= 32 the unsplit
// kernel reads less A and already runs near a read-only stream of B, and the
// reduction does not pay: a last-workgroup sum costs three dependent trips to
// device-coherent memory, about 3 us.)
namespace splitk {
constexpr int NW = 8, NT = 64 * NW, BN = 16 * NW, KSMAX = 8, SMAX = 16, TMMAX = 4;
}  // namespace splitk

struct SplitKArgs {
  float* part;  // [S][M][N] fp32 partials
  int S;
};

template <int KS, int TM>
__global__ __launch_bounds__(splitk::NT) void gemm_splitk_kernel(const GemmArgs args, const SplitKArgs sk) {
  using namespace splitk;
  constexpr int ROWS = 16 * TM;
  static_assert(KS >= 1 && KS <= KSMAX && TM >= 1 && TM <= TMMAX, "split-K tile");
  __shared__ __align__(16) uint8_t sA[KS * TM * 2048];
  // row scales [ROWS][KS] and the weight scales of the split's blocks (fp32,
  // or e8m0 bytes at offset idx0 % 4 of the dwords that hold them)
  __shared__ __align__(16) float sSa[ROWS * KS + 64];
  __shared__ __align__(16) uint32_t sSk[64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, r16 = lane & 15;
  const int64_t M = args.M, N = args.N, K = args.K;
  const int KB = (int)(K / 128);
  // workgroup -> (row tile mt, split s, column tile t): consecutive
  // workgroups (which the dispatcher spreads over the XCDs) take consecutive
  // tiles of one split
  const int n_tiles = (int)(N / BN);
  const int rest = blockIdx.x / n_tiles;
  const int t = blockIdx.x - rest * n_tiles;
  const int mt = rest / sk.S;
  const int s = rest - mt * sk.S;
  const int64_t m0 = (int64_t)mt * ROWS;
  const int kb0 = s * KS;
  const int nkb = min(KS, KB - kb0);  // >= 1: S = ceil(KB / KS)
  const int64_t n0 = (int64_t)t * BN;
  // [gate | up] of an expert record: columns past n_split are the up half
  const bool second = args.bsrc != nullptr && n0 >= args.n_split;
  const uint8_t* bmat = args.b;
  const void* sbm = args.sb;
  if (args.bsrc) {
    bmat = uniform_ptr(second ? args.bsrc->w_up : args.bsrc->w_gate);
    sbm = uniform_ptr(second ? args.bsrc->s_up : args.bsrc->s_gate);
  }
  const int64_t nl = second ? n0 - args.n_split : n0;
  const int rr = lane >> 3, pc = lane & 7;

  // the A slice: one DMA moves rows 8h..8h+7 of K block kl (lane: row
  // 8h + lane/8, 16-byte position lane%8, which holds the row's chunk
  // position ^ swz(row)); rows past M re-read row M-1 (their outputs are
  // dropped), blocks past the split's last re-read its first (their products
  // are skipped)
  const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds_u32(sA));
  constexpr int NDA = (ROWS / 8) * KS;
#pragma unroll
  for (int j = 0; j < (NDA + NW - 1) / NW; ++j) {
    const int q = wave + NW * j;
    if (q < NDA) {
      const int kl = q / (ROWS / 8), h8 = q - kl * (ROWS / 8);
      const int r = h8 * 8 + rr;
      const int64_t row = m0 + r < M ? m0 + r : M - 1;
      const int kb = kb0 + (kl < nkb ? kl : 0);
      dma16v((uint64_t)(uintptr_t)args.a + (uint64_t)(row * K + (int64_t)kb * 128) +
                 (uint32_t)((pc ^ swz(r & 15)) << 4),
             __builtin_amdgcn_readfirstlane(a_lds + (uint32_t)((kl * TM + (h8 >> 1)) * 2048 + (h8 & 1) * 1024)));
    }
  }
  // sa rows x KS, one dword per lane (row M-1 past M, the split's first
  // block past its last), and the weight scales of blocks kb0 .. kb0 + nkb - 1
  // of column block n0 / 128 -- fp32, or the dwords holding those e8m0 bytes
  // (never past the last one's dword, so no read leaves the scales' last page)
  constexpr int NDS = (ROWS * KS + 63) / 64;
  const uint32_t sa_lds = __builtin_amdgcn_readfirstlane(lds_u32(sSa));
#pragma unroll
  for (int j = 0; j < (NDS + NW - 1) / NW; ++j) {
    const int q = wave + NW * j;
    if (q < NDS) {
      const int i = q * 64 + lane;
      const int r = i / KS, kl = i - r * KS;
      const int64_t row = m0 + r < M ? m0 + r : M - 1;
      const int kb = kb0 + (kl < nkb ? kl : 0);
      if (args.sa_e8m0)  // e8m0 scales: the aligned dword holding the byte
        dma4v((uint64_t)(uintptr_t)args.sa + (uint64_t)((row * KB + kb) & ~(int64_t)3),
              __builtin_amdgcn_readfirstlane(sa_lds + (uint32_t)(q * 256)));
      else
        dma4v((uint64_t)(uintptr_t)args.sa + (uint64_t)(row * KB + kb) * 4u,
              __builtin_amdgcn_readfirstlane(sa_lds + (uint32_t)(q * 256)));
    }
  }
  const int64_t idx0 = (nl / 128) * KB + kb0;
  if (wave == NW - 1) {
    const uint32_t sk_lds = __builtin_amdgcn_readfirstlane(lds_u32(sSk));
    if (args.sb_e8m0) {
      const int nd = (int)((idx0 & 3) + nkb + 3) / 4;
      if (lane < nd)
        dma4v((uint64_t)(uintptr_t)sbm + (uint64_t)((idx0 & ~(int64_t)3) + 4 * lane), sk_lds);
    } else if (lane < nkb) {
      dma4v((uint64_t)(uintptr_t)sbm + (uint64_t)(idx0 + lane) * 4u, sk_lds);
    }
  }
  // B: column n0 + 16 wave + r16, K bytes [32 g4, +32) of each block
  const uint8_t* brow = bmat + (nl + 16 * wave + r16) * K + 32 * g4;
  v8i bf[KS];
#pragma unroll
  for (int kl = 0; kl < KS; ++kl) bf[kl] = load_frag_global(brow + (int64_t)(kb0 + (kl < nkb ? kl : 0)) * 128);
  // the DMAs were issued before the 2 KS B loads: wait for those alone
  // (vmcnt counts in issue order)
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * KS) : "memory");
  __syncthreads();

  const FragLane fl = frag_lane(r16, g4);
  const v4f vzero = {0.0f, 0.0f, 0.0f, 0.0f};
  v4f acc[TM];
#pragma unroll
  for (int mi = 0; mi < TM; ++mi) acc[mi] = vzero;
#pragma unroll
  for (int kl = 0; kl < KS; ++kl) {
    if (kl < nkb) {
      const float skb = args.sb_e8m0 ? e8m0_value(reinterpret_cast<const uint8_t*>(sSk)[(idx0 & 3) + kl])
                                     : __uint_as_float(sSk[kl]);
      v8i af[TM];
#pragma unroll
      for (int mi = 0; mi < TM; ++mi) af[mi] = read_frag(sA + (kl * TM + mi) * 2048, fl);
      if (args.sa_e8m0) {
        // e8m0 row scales: the byte (source row) KB + kb of the scale tensor,
        // from the aligned dword the DMA staged, is the exponent the MFMA
        // takes (activation rows = operand A, lane r16's row; rows past M
        // read row M - 1, dropped); C += P' sb is the promotion's
        // C += P (sa sb) to the bit
#pragma unroll
        for (int mi = 0; mi < TM; ++mi) {
          const int row = 16 * mi + r16;
          const int64_t src = m0 + row < M ? m0 + row : M - 1;
          const int sae = (int)((__float_as_uint(sSa[row * KS + kl]) >>
                                 (((uint32_t)(src * KB + kb0 + kl) & 3u) * 8u)) & 0xFFu);
          const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[mi], bf[kl], vzero, 0, 0, 0, sae, 0,
                                                                         127);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[mi][r] = fmaf(p[r], skb, acc[mi][r]);
        }
        continue;
      }
#pragma unroll
      for (int mi = 0; mi < TM; ++mi) {
        const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[mi], bf[kl], vzero, 0, 0, 0, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mi][r] = fmaf(p[r], sSa[(16 * mi + 4 * g4 + r) * KS + kl] * skb, acc[mi][r]);
      }
    }
  }

  // lane (g4, r16) holds rows 16 mi + 4 g4 + r of column col
  const int64_t col = n0 + 16 * wave + r16;
  float* part = sk.part + (int64_t)s * M * N;
#pragma unroll
  for (int mi = 0; mi < TM; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = m0 + 16 * mi + 4 * g4 + r;
      if (row < M) part[row * N + col] = acc[mi][r];
    }
}

// C = sum over the S split partials in split order (4 consecutive elements
// of [M, N] per thread; M N % 4 == 0 as N % 128 == 0)
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int S,
                                                            int64_t MN, void* c, int out_f32) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= MN) return;
  float4 v[splitk::SMAX];
#pragma unroll
  for (int s = 0; s < splitk::SMAX; ++s)
    if (s < S) v[s] = *reinterpret_cast<const float4*>(part + (int64_t)s * MN + i);
  float4 a = v[0];
#pragma unroll
  for (int s = 1; s < splitk::SMAX; ++s)
    if (s < S) {
      a.x += v[s].x;
      a.y += v[s].y;
      a.z += v[s].z;
      a.w += v[s].w;
    }
  if (out_f32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(c) + i) = a;
  } else {
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(c) + i) =
        make_uint2((uint32_t)bf16_bits_exact(a.x) | ((uint32_t)bf16_bits_exact(a.y) << 16),
                   (uint32_t)bf16_bits_exact(a.z) | ((uint32_t)bf16_bits_exact(a.w) << 16));
  }
}

template <int KS, int TM>
int launch_splitk_gemm(GemmArgs& a, int S, float* part, hipStream_t stream) {
  const SplitKArgs sk{part, S};
  const int n_tiles = (int)(a.N / splitk::BN);
  const int m_tiles = (int)ceil_div(a.M, (int64_t)(16 * TM));
  gemm_splitk_kernel<KS, TM><<<(unsigned)(n_tiles * S * m_tiles), splitk::NT, 0, stream>>>(a, sk);
  return check_launch("gemm_fp8_splitk");
}

template <int KS, int TM>
int launch_splitk_ks(GemmArgs& a, int S, float* part, hipStream_t stream) {
  const SplitKArgs sk{part, S};
  const int n_tiles = (int)(a.N / splitk::BN);
  const int m_tiles = (int)ceil_div(a.M, (int64_t)(16 * TM));
  gemm_splitk_kernel<KS, TM><<<(unsigned)(n_tiles * S * m_tiles), splitk::NT, 0, stream>>>(a, sk);
  int rc = check_launch("gemm_fp8_splitk");
  if (rc) return rc;
  const int64_t MN = a.M * a.N;
  splitk_reduce_kernel<<<(unsigned)ceil_div(MN / 4, (int64_t)256), 256, 0, stream>>>(part, S, MN, a.c,
                                                                                    a.out_f32);
  return check_launch("gemm_fp8_splitk_reduce");
}

// The split-K path for a dense FP8 GEMM when it applies (16 < M <= 64, N %
// 128 == 0, at least two splits that fit, a workspace at hand); returns -1
// when the caller should take the unsplit kernels.
template <int TM>
int launch_splitk_tm(GemmArgs& a, int KS, int S, float* part, hipStream_t stream) {
  switch (KS) {
    case 1: return launch_splitk_ks<1, TM>(a, S, part, stream);
    case 2: return launch_splitk_ks<2, TM>(a, S, part, stream);
    case 3: return launch_splitk_ks<3, TM>(a, S, part, stream);
    case 4: return launch_splitk_ks<4, TM>(a, S, part, stream);
    case 5: return launch_splitk_ks<5, TM>(a, S, part, stream);
    case 6: return launch_splitk_ks<6, TM>(a, S, part, stream);
    case 7: return launch_splitk_ks<7, TM>(a, S, part, stream);
    default: return launch_splitk_ks<8, TM>(a, S, part, stream);
  }
}

// The split of a dense FP8 GEMM over K, a function of the shape alone (so an
// eager call and a captured one sum in the same order): 16 < M <= 64
// (N = 4096, K = 7168, graph-replayed over cold weights: M = 32 12.1 us where
// the skinny kernel takes 14.3; M = 16 10.9 vs 10.5, M = 128 with 128-row
// tiles 23.0 vs 22.0 with 32 x 64 tiles), N % 128 == 0, about one workgroup
// per CU: S <= 16 splits of KS <= 8 K blocks.  Returns false when the shape
// does not split.
bool splitk_plan(int64_t M, int64_t N, int64_t K, int* ks_out, int* s_out) {
  using namespace splitk;
  if (M <= 16 || M > 16 * TMMAX || N % BN != 0 || K % 128 != 0) return false;
  const int KB = (int)(K / 128);
  const int n_tiles = (int)(N / BN);
  const int s_target = n_tiles >= 256 ? 1 : 256 / n_tiles;
  int KS = (int)ceil_div((int64_t)KB, (int64_t)s_target);
  KS = (int)std::max<int64_t>(KS, ceil_div((int64_t)KB, (int64_t)SMAX));
  if (KS > KSMAX) return false;
  const int S = (int)ceil_div((int64_t)KB, (int64_t)KS);
  if (S < 2) return false;
  *ks_out = KS;
  *s_out = S;
  return true;
}

// The split-K path when the shape splits: the fp32 partials go to the
// caller's workspace (too small: an error, never a different summation
// order); returns kNoSplit when the caller should take the unsplit kernels,
// else the launch status.
constexpr int kNoSplit = 1;
int try_splitk(GemmArgs& a, hipStream_t stream) {
  int KS = 0, S = 0;
  if (a.wfmt != WF_FP8 || !splitk_plan(a.M, a.N, a.K, &KS, &S)) return kNoSplit;
  if (a.sb_e8m0 && !aligned(a.sb, 4)) return kNoSplit;  // e8m0 scales are read as whole dwords
  const size_t need = (size_t)S * (size_t)a.M * (size_t)a.N * 4;
  if (!a.ws || a.ws_bytes < need || !aligned(a.ws, 16)) {
    set_error("fp8_gemm: M=%lld N=%lld K=%lld splits K %d ways and needs a 16-byte aligned "
              "workspace of %zu bytes (sgl_fp8_gemm_workspace_size), got %zu",
              (long long)a.M, (long long)a.N, (long long)a.K, S, need, a.ws ? a.ws_bytes : (size_t)0);
    return SGL_ERR_WORKSPACE;
  }
  float* part = reinterpret_cast<float*>(a.ws);
  if (a.M <= 32) return launch_splitk_tm<2>(a, KS, S, part, stream);
  return launch_splitk_tm<4>(a, KS, S, part, stream);
}

}  // namespace

namespace {

// The shared expert's [gate | up] partials summed in split order (as
// splitk_reduce_kernel sums them), then the gate/up epilogue of the grouped
// kernel on each 128-column group: gate and up rounded to bf16, the SwiGLU
// clamp, h = bf16(silu(gate) * up) (routing weight 1), and the 1x128 requant
// of h.  16 lanes per (row, group), 8 columns each; 16 groups per workgroup.
template <int MODE>
__global__ __launch_bounds__(256) void shared_swiglu_kernel(const float* __restrict__ part, int S,
                                                            int64_t T, int64_t I,
                                                            const int32_t* __restrict__ shared_base,
                                                            float lim, uint8_t* __restrict__ hq,
                                                            float* __restrict__ hs) {
  const int64_t NB = I / 128;
  const int64_t task = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // (row, group)
  const int j = threadIdx.x & 15;
  const bool live = task < T * NB;  // the tail's 16-lane groups stay for the shuffles
  const int64_t t = live ? task / NB : 0, g = live ? task - (task / NB) * NB : 0;
  const int64_t N = 2 * I, MN = T * N;
  const float* pg = part + t * N + g * 128 + 8 * j;
  float gs[8], us[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) gs[i] = us[i] = 0.0f;
  for (int sp = 0; sp < S; ++sp) {
    const float4 g0 = *reinterpret_cast<const float4*>(pg + sp * MN);
    const float4 g1 = *reinterpret_cast<const float4*>(pg + sp * MN + 4);
    const float4 u0 = *reinterpret_cast<const float4*>(pg + sp * MN + I);
    const float4 u1 = *reinterpret_cast<const float4*>(pg + sp * MN + I + 4);
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      gs[i] = sp ? gs[i] + gv[i] : gv[i];
      us[i] = sp ? us[i] + uv[i] : uv[i];
    }
  }
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float gt = bf16_round(gs[i]);
    float up = bf16_round(us[i]);
    if (lim > 0.0f) {
      up = clampf_(up, -lim, lim);
      gt = gt > lim ? lim : gt;
    }
    const float ex = __builtin_amdgcn_exp2f(gt * -1.4426950408889634f);
    const float silu = gt * __builtin_amdgcn_rcpf(1.0f + ex);
    f[i] = bits_f32((uint32_t)bf16_bits_exact(silu * up) << 16);
  }
  float amax = 0.0f;  // IEEE maximum: a NaN makes the group's scale NaN
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = __builtin_elementwise_maximum(amax, fabsf(f[i]));
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) amax = __builtin_elementwise_maximum(amax, __shfl_xor(amax, o, 64));
  if (!live) return;
  const float sf = group_scale(MODE, amax);
  const int64_t p = (int64_t)*shared_base + t;
  *reinterpret_cast<uint2*>(hq + p * I + g * 128 + 8 * j) = quant8_e4m3(MODE, f, sf);
  if (j == 0) hs[p * NB + g] = sf;
}

// Split plan of the shared gate/up ([gate | up] = N = 2I columns, K = H):
// 32-row tiles up to T = 32, else 64; about 256 workgroups; at most as many
// splits as `room` bytes of partials hold.  T <= 128: at T = 256 (128 tiles
// of the grouped kernel) four splits measured no faster (H = 4096, I = 2048:
// the partials' traffic takes what the extra workgroups gain), at T = 64 the
// FP4 decode layer is 14-16 us faster.
bool shared_split_plan(int64_t T, int64_t H, int64_t I, size_t room, int* tm, int* ks, int* sp) {
  using namespace splitk;
  if (T < 1 || T > 128 || (2 * I) % BN != 0 || H % 128 != 0) return false;
  const int TM = T <= 32 ? 2 : 4;
  const int64_t m_tiles = ceil_div(T, (int64_t)(16 * TM));
  const int KB = (int)(H / 128);
  const int64_t tiles = (2 * I / BN) * m_tiles;
  const int64_t s_target = tiles >= 256 ? 1 : 256 / tiles;
  const int64_t s_room = (int64_t)(room / ((size_t)T * (size_t)(2 * I) * 4));
  int KS = (int)ceil_div((int64_t)KB, std::min<int64_t>(s_target, s_room > 0 ? s_room : 1));
  KS = (int)std::max<int64_t>(KS, ceil_div((int64_t)KB, (int64_t)SMAX));
  if (KS > KSMAX) return false;
  const int S = (int)ceil_div((int64_t)KB, (int64_t)KS);
  if (S < 2 || (int64_t)S > s_room) return false;
  *tm = TM;
  *ks = KS;
  *sp = S;
  return true;
}

template <int TM>
int launch_shared_splitk(GemmArgs& a, int KS, int S, float* part, hipStream_t stream) {
  switch (KS) {
    case 1: return launch_splitk_gemm<1, TM>(a, S, part, stream);
    case 2: return launch_splitk_gemm<2, TM>(a, S, part, stream);
    case 3: return launch_splitk_gemm<3, TM>(a, S, part, stream);
    case 4: return launch_splitk_gemm<4, TM>(a, S, part, stream);
    case 5: return launch_splitk_gemm<5, TM>(a, S, part, stream);
    case 6: return launch_splitk_gemm<6, TM>(a, S, part, stream);
    case 7: return launch_splitk_gemm<7, TM>(a, S, part, stream);
    default: return launch_splitk_gemm<8, TM>(a, S, part, stream);
  }
}

}  // namespace

int launch_shared_gate_up_split(const GemmArgs& sh, void* part, size_t part_bytes,
                                const int32_t* shared_base, hipStream_t stream) {
  int TM = 0, KS = 0, S = 0;
  if (!part || !aligned(part, 16) || sh.wfmt != WF_FP8 ||
      !shared_split_plan(sh.T, sh.K, sh.N, part_bytes, &TM, &KS, &S))
    return kSharedNoSplit;
  GemmArgs a = {};
  a.a = sh.a;
  a.sa = sh.sa;
  a.wfmt = WF_FP8;
  a.M = sh.T;
  a.N = 2 * sh.N;
  a.K = sh.K;
  a.bsrc = sh.experts;  // the shared expert's record: the kernel reads its pointers
  a.n_split = sh.N;
  float* p = reinterpret_cast<float*>(part);
  const int rc = TM == 2 ? launch_shared_splitk<2>(a, KS, S, p, stream)
                         : launch_shared_splitk<4>(a, KS, S, p, stream);
  if (rc) return rc;
  const int64_t tasks = sh.T * (sh.N / 128);
  const unsigned g = (unsigned)ceil_div(tasks, (int64_t)16);
  switch (sh.scale_mode) {
    case SCALE_TORCH_FP32:
      shared_swiglu_kernel<SCALE_TORCH_FP32><<<g, 256, 0, stream>>>(p, S, sh.T, sh.N, shared_base,
                                                                    sh.swiglu_limit, sh.hq, sh.hs);
      break;
    case SCALE_TORCH_UE8M0:
      shared_swiglu_kernel<SCALE_TORCH_UE8M0><<<g, 256, 0, stream>>>(p, S, sh.T, sh.N, shared_base,
                                                                     sh.swiglu_limit, sh.hq, sh.hs);
      break;
    case SCALE_TILELANG_FP32:
      shared_swiglu_kernel<SCALE_TILELANG_FP32><<<g, 256, 0, stream>>>(p, S, sh.T, sh.N, shared_base,
                                                                       sh.swiglu_limit, sh.hq, sh.hs);
      break;
    default:
      shared_swiglu_kernel<SCALE_TILELANG_UE8M0><<<g, 256, 0, stream>>>(p, S, sh.T, sh.N, shared_base,
                                                                        sh.swiglu_limit, sh.hq, sh.hs);
  }
  return check_launch("moe_shared_gate_up_split");
}

size_t dense_fp8_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  int KS = 0, S = 0;
  if (!SGL_SPLITK || !splitk_plan(M, N, K, &KS, &S)) return 0;
  return (size_t)S * (size_t)M * (size_t)N * 4;
}

// FP4 weights: a stage is 256 deep, so two stages fill what three fp8
// stages of the same tile would (the 128 x 256 tiles run one workgroup per
// CU with one stage in flight while the other is computed)
// fp4 experts with fragment-layout copies: the register-fed kernel (K a
// multiple of 512, 16 to 64 stages, 16-byte aligned row scales)
inline bool rb_fp4_ok(const GemmArgs& a) {
  const int64_t kb = a.K / 128;
  return SGL_RB && a.frag && kb >= rb::kMinKB && kb <= rb::kMaxKBr && kb % 4 == 0 &&
         aligned(a.sa, 16);
}

template <bool SAHW>
int launch_fp4(int kind, GemmArgs& a, int64_t rows_hint, hipStream_t stream) {
  const bool big = rows_hint >= 64;
  switch (kind) {
    case KIND_DENSE:
      if (a.M <= kSkinnyMaxM) {
        if (a.M <= 16) return launch_skinny<1, WF_FP4, SAHW>(a, stream);
        if (a.M <= 32) return launch_skinny<2, WF_FP4, SAHW>(a, stream);
        return launch_skinny<4, WF_FP4, SAHW>(a, stream);
      }
      if (a.M <= 256) return launch_cfg<KIND_DENSE, 32, 128, 1, 4, 3, WF_FP4, SAHW>(a, stream);
      if (a.M <= 512) return launch_cfg<KIND_DENSE, 64, 128, 2, 2, 2, WF_FP4, SAHW>(a, stream);
      if (a.M <= 2048) return launch_cfg<KIND_DENSE, 128, 128, 2, 4, 2, WF_FP4, SAHW>(a, stream);
      return launch_cfg<KIND_DENSE, 128, 256, 2, 4, 2, WF_FP4, SAHW>(a, stream);
    case KIND_GATE_UP:
      if (rb_fp4_ok(a)) return launch_rb<KIND_GATE_UP, true>(a, rows_hint, stream);
      return big ? launch_cfg<KIND_GATE_UP, 128, 256, 2, 4, 2, WF_FP4, SAHW>(a, stream)
                 : launch_cfg<KIND_GATE_UP, 32, 256, 1, 4, 3, WF_FP4, SAHW>(a, stream);
    default:
      if (rb_fp4_ok(a)) return launch_rb<KIND_DOWN, true>(a, rows_hint, stream);
      return big ? launch_cfg<KIND_DOWN, 128, 256, 2, 4, 2, WF_FP4, SAHW>(a, stream)
                 : launch_cfg<KIND_DOWN, 32, 256, 1, 4, 3, WF_FP4, SAHW>(a, stream);
  }
}

// The tiled dense FP8 kernels above the skinny / split-K sizes (SAHW: e8m0
// row scales; the tile choice is explained in launch_gemm).  M = 2049 with
// 256 x 256 tiles in 27 us where 128 x 256 tiles take 33; 128 x 128 with 8
// wavefronts (the issuer split) from M = 512: M = 1024 in 52 us where
// 64 x 128 tiles take 64 us.
template <bool SAHW>
int launch_dense_tiles(GemmArgs& a, hipStream_t stream) {
  if (a.M <= 128) return launch_cfg<KIND_DENSE, 32, 64, 1, 4, 4, WF_FP8, SAHW>(a, stream);
  if (a.M <= 256) return launch_cfg<KIND_DENSE, 32, 128, 1, 4, 4, WF_FP8, SAHW>(a, stream);
  if (a.M <= 512) return launch_cfg<KIND_DENSE, 64, 128, 2, 2, 3, WF_FP8, SAHW>(a, stream);
  if (a.M <= 2048) return launch_cfg<KIND_DENSE, 128, 128, 2, 4, 3, WF_FP8, SAHW>(a, stream);
  return launch_wide(a, stream);  // 256 x 256 tiles (K <= 16384 by the check in launch_gemm)
}

int launch_gemm(int kind, GemmArgs& a, int64_t rows_hint, hipStream_t stream) {
  if (a.K > 128 * kMaxKB) {
    set_error("gemm: K=%lld above the supported %d", (long long)a.K, 128 * kMaxKB);
    return SGL_ERR_UNSUPPORTED;
  }
  if (a.wfmt == WF_FP4) {
    if (a.K % 256 != 0) {
      set_error("gemm: FP4 weights need K=%lld to be a multiple of 256", (long long)a.K);
      return SGL_ERR_INVALID_ARG;
    }
    return a.sa_pow2 ? launch_fp4<true>(kind, a, rows_hint, stream)
                     : launch_fp4<false>(kind, a, rows_hint, stream);
  }
  const bool big = rows_hint >= 64;
  // the pipelined prefill kernel: K in [512, 8192] (at least four stages; the
  // tile's weight scales fit its LDS table) and fp32 weight scales
  const bool pipe_ok = SGL_PIPE && a.K >= 512 && a.K <= 128 * pipe::kMaxKBp && !a.sb_e8m0;
  // both scales powers of two: the pipelined kernel applies them in the MFMA
  // (other kernels promote in fp32, exact for such scales too)
  const bool pow2 = a.sa_pow2 && a.sb_pow2;
  // register-fed weights, at every batch size: the experts' fragment-layout
  // copies, 16 to 64 stages in multiples of four, fp32 weight scales (powers
  // of two or not), 16-byte aligned row scales for their float4 loads.  At
  // decode sizes the weight stream is the whole cost and registers fed
  // straight from memory beat the LDS-staged 32-row tiles (T = 64 / 256 /
  // 512, Zipf load: layer 676 / 1103 / 1255 -> 627 / 1024 / 1170 us)
  const int64_t kb = a.K / 128;
  // The row-major weights: the LDS-staged kernels, whose DMAs take whole
  // 128-byte row segments (8 rows per 1 KB instruction); loading them
  // straight into registers in the MFMA's lane order takes each line in two
  // halves, and measured no faster (decode T = 64 / 256 / 512: 0.66 / 1.04 /
  // 1.22 ms against 0.62 / 1.00 / 1.19 with the 32-row tiles' nontemporal
  // weight DMAs; prefill gate/up 2.08 against 1.97 ms).
  const bool rb_ok = SGL_RB && a.frag && !a.sb_e8m0 && kb >= rb::kMinKB && kb <= rb::kMaxKBr &&
                     kb % 4 == 0 && aligned(a.sa, 16);
  // the FP8 shared expert of an FP4 layer in a launch of its own at decode
  // batch sizes: 32-row tiles, so ceil(T / 32) x N / 256 workgroups share
  // its weight stream (128-row tiles give N / 256 = 16 at T <= 128); the
  // down projection, with no requant groups to keep whole, in 32 x 64 tiles
  // while 256-column tiles would leave half the CUs idle: a workgroup streams
  // its weight slice at a capped rate, so more workgroups finish sooner
  // (H = 4096, I = 2048, FP4 decode layer: T = 64 / 256 -5 / -11 us; at
  // T = 512, 256 tiles of 32 x 256 already cover the CUs and the 64-column
  // tiles' extra activation re-reads cost 15 us)
  const bool shared_small = a.E == 0 && a.has_shared && a.T <= 512;
  const bool shared_narrow = shared_small && ceil_div(a.T, 32) * ceil_div(a.N, 256) <= 128;
  switch (kind) {
    case KIND_DENSE: {
      const int rc = SGL_SPLITK ? try_splitk(a, stream) : kNoSplit;
      if (rc != kNoSplit) return rc;
      if (a.M <= kSkinnyMaxM) {
        if (a.M <= 16) return launch_skinny<1>(a, stream);
        if (a.M <= 32) return launch_skinny<2>(a, stream);
        return launch_skinny<4>(a, stream);
      }
      // 256 x 256 tiles above M = 2048, 128 x 128 from 512, 64 x 128 (two
      // workgroups per CU) from 256, so the grid still covers every CU.  A workgroup
      // streams its operands at a capped rate (about 35 GB/s measured,
      // whatever the stage depth or wavefront count), so for M <= 256 the
      // tiles shrink until there is about one per CU: N = 4096, K = 7168 at
      // M = 128 takes 23 us with 32 x 64 tiles, 39 us with 64 x 128, 36 us
      // with the skinny kernel's 128-row tiles (every workgroup re-reads all
      // of A from L2)
      // e8m0 row scales: the SAHW instantiations (bytes; with e8m0 weight
      // scales too, both in the MFMA)
      if (a.sa_e8m0) return launch_dense_tiles<true>(a, stream);
      return launch_dense_tiles<false>(a, stream);
    }
    case KIND_GATE_UP:
      if (shared_small) return launch_cfg<KIND_GATE_UP, 32, 256, 1, 4, 4>(a, stream);
      if (rb_ok) return launch_rb<KIND_GATE_UP>(a, rows_hint, stream);
      if (big && pipe_ok)
        return pow2 ? launch_pipe<KIND_GATE_UP, true>(a, stream) : launch_pipe<KIND_GATE_UP, false>(a, stream);
      return big ? launch_cfg<KIND_GATE_UP, 128, 256, 2, SGL_LWN, 3, WF_FP8, false, SGL_LW>(a, stream)
                 : launch_cfg<KIND_GATE_UP, 32, 256, 1, 4, 4>(a, stream);
    default:
      if (shared_narrow) return launch_cfg<KIND_DOWN, 32, 64, 1, 4, 4>(a, stream);
      if (shared_small) return launch_cfg<KIND_DOWN, 32, 256, 1, 4, 4>(a, stream);
      if (rb_ok) return launch_rb<KIND_DOWN>(a, rows_hint, stream);
      if (big && pipe_ok)
        return pow2 ? launch_pipe<KIND_DOWN, true>(a, stream) : launch_pipe<KIND_DOWN, false>(a, stream);
      return big ? launch_cfg<KIND_DOWN, 128, 256, 2, SGL_LWN, 3, WF_FP8, false, SGL_LW>(a, stream)
                 : launch_cfg<KIND_DOWN, 32, 256, 1, 4, 4>(a, stream);
  }
}

}  // namespace sgl

extern "C" size_t sgl_fp8_gemm_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return sgl::dense_fp8_workspace_bytes(M, N, K);
}

extern "C" int sgl_fp8_gemm(const void* a, const void* sa, int a_scale_e8m0, const void* b,
                            const void* sb, int b_scale_e8m0, void* c, int out_dtype, int64_t M,
                            int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                            sgl_stream_t stream) {
  SGL_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fp8_gemm: negative shape");
  SGL_REQUIRE(out_dtype == SGL_BF16 || out_dtype == SGL_F32, "fp8_gemm: out_dtype must be bf16/f32");
  SGL_REQUIRE(K % 128 == 0, "fp8_gemm: K=%lld must be a multiple of 128", (long long)K);
  SGL_REQUIRE(N % 16 == 0, "fp8_gemm: N=%lld must be a multiple of 16", (long long)N);
  if (M == 0 || N == 0) return SGL_OK;
  SGL_REQUIRE(a && sa && b && sb && c, "fp8_gemm: null pointer");
  SGL_REQUIRE(M * K < ((int64_t)1 << 31) && N * K < ((int64_t)1 << 31),
              "fp8_gemm: operands above 2 GiB are not supported");
  SGL_REQUIRE(sgl::aligned(a, 16) && sgl::aligned(b, 16) && sgl::aligned(c, 16),
              "fp8_gemm: A, B and C must be 16-byte aligned");
  SGL_REQUIRE(a_scale_e8m0 || sgl::aligned(sa, 4), "fp8_gemm: fp32 sa must be 4-byte aligned");
  SGL_REQUIRE(b_scale_e8m0 || sgl::aligned(sb, 4), "fp8_gemm: fp32 sb must be 4-byte aligned");
  sgl::GemmArgs g = {};
  g.a = (const uint8_t*)a;
  g.sa = sa;
  g.sa_e8m0 = a_scale_e8m0 ? 1 : 0;
  g.b = (const uint8_t*)b;
  g.sb = sb;
  g.sb_e8m0 = b_scale_e8m0;
  g.M = M;
  g.N = N;
  g.K = K;
  g.c = c;
  g.out_f32 = out_dtype == SGL_F32;
  g.ws = workspace;
  g.ws_bytes = workspace ? workspace_bytes : 0;
  return sgl::launch_gemm(sgl::KIND_DENSE, g, M, (hipStream_t)stream);
}

extern "C" int sgl_fp4_gemm(const void* a, const void* sa, int sa_format, const void* b,
                            const void* sb, void* c, int out_dtype, int64_t M, int64_t N,
                            int64_t K, sgl_stream_t stream) {
  SGL_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fp4_gemm: negative shape");
  SGL_REQUIRE(out_dtype == SGL_BF16 || out_dtype == SGL_F32, "fp4_gemm: out_dtype must be bf16/f32");
  SGL_REQUIRE(K % 256 == 0, "fp4_gemm: K=%lld must be a multiple of 256", (long long)K);
  SGL_REQUIRE(N % 16 == 0, "fp4_gemm: N=%lld must be a multiple of 16", (long long)N);
  if (M == 0 || N == 0) return SGL_OK;
  SGL_REQUIRE(a && sa && b && sb && c, "fp4_gemm: null pointer");
  SGL_REQUIRE(M * K < ((int64_t)1 << 31) && N * K / 2 < ((int64_t)1 << 31),
              "fp4_gemm: operands above 2 GiB are not supported");
  SGL_REQUIRE(sgl::aligned(a, 16) && sgl::aligned(b, 16) && sgl::aligned(c, 16),
              "fp4_gemm: A, B and C must be 16-byte aligned");
  SGL_REQUIRE(sa_format >= SGL_ASCALE_F32 && sa_format <= SGL_ASCALE_E8M0,
              "fp4_gemm: sa_format=%d is not an SGL_ASCALE_* value", sa_format);
  SGL_REQUIRE((sa_format == SGL_ASCALE_E8M0 || sgl::aligned(sa, 4)) && sgl::aligned(sb, 4),
              "fp4_gemm: fp32 sa and sb must be 4-byte aligned");
  sgl::GemmArgs g = {};
  g.a = (const uint8_t*)a;
  g.sa = sa;
  g.b = (const uint8_t*)b;
  g.sb = sb;
  g.wfmt = sgl::WF_FP4;
  // e8m0 row scales are powers of two: applied inside the MFMA
  g.sa_pow2 = sa_format != SGL_ASCALE_F32 ? 1 : 0;
  g.sa_e8m0 = sa_format == SGL_ASCALE_E8M0 ? 1 : 0;
  g.M = M;
  g.N = N;
  g.K = K;
  g.c = c;
  g.out_f32 = out_dtype == SGL_F32;
  return sgl::launch_gemm(sgl::KIND_DENSE, g, M, (hipStream_t)stream);
}

extern "C" int sgl_fp8_weight_to_frag(const void* w, int64_t N, int64_t K, void* out,
                                      sgl_stream_t stream) {
  SGL_REQUIRE(N >= 0 && K >= 0, "fp8_weight_to_frag: negative shape");
  SGL_REQUIRE(N % 16 == 0 && K % 128 == 0,
              "fp8_weight_to_frag: N=%lld must be a multiple of 16 and K=%lld of 128", (long long)N,
              (long long)K);
  if (N == 0 || K == 0) return SGL_OK;
  SGL_REQUIRE(w && out, "fp8_weight_to_frag: null pointer");
  SGL_REQUIRE(w != out, "fp8_weight_to_frag: the output must not alias the input");
  SGL_REQUIRE(sgl::aligned(w, 16) && sgl::aligned(out, 16),
              "fp8_weight_to_frag: w and out must be 16-byte aligned");
  SGL_REQUIRE(N * K < ((int64_t)1 << 36), "fp8_weight_to_frag: matrix too large");
  const int64_t chunks = N * K / 16;
  sgl::weight_to_frag_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)w, N, K, (uint8_t*)out);
  return sgl::check_launch("fp8_weight_to_frag");
}

extern "C" int sgl_fp4_weight_to_frag(const void* w, const void* s, int64_t N, int64_t K, void* out_w,
                                      void* out_s, sgl_stream_t stream) {
  SGL_REQUIRE(N >= 0 && K >= 0, "fp4_weight_to_frag: negative shape");
  SGL_REQUIRE(N % 16 == 0 && K % 512 == 0,
              "fp4_weight_to_frag: N=%lld must be a multiple of 16 and K=%lld of 512", (long long)N,
              (long long)K);
  if (N == 0 || K == 0) return SGL_OK;
  SGL_REQUIRE(w && s && out_w && out_s, "fp4_weight_to_frag: null pointer");
  SGL_REQUIRE(w != out_w && s != out_s, "fp4_weight_to_frag: the outputs must not alias the inputs");
  SGL_REQUIRE(sgl::aligned(w, 16) && sgl::aligned(out_w, 16) && sgl::aligned(out_s, 4),
              "fp4_weight_to_frag: w and out_w must be 16-byte aligned, out_s 4-byte aligned");
  SGL_REQUIRE(N * K < ((int64_t)1 << 36), "fp4_weight_to_frag: matrix too large");
  const int64_t items = N * (K / 2) / 16 + N * (K / 128);
  sgl::weight_fp4_to_frag_kernel<<<(unsigned)((items + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)w, (const uint8_t*)s, N, K, (uint8_t*)out_w, (uint8_t*)out_s);
  return sgl::check_launch("fp4_weight_to_frag");
}
