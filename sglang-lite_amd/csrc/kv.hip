// FP8 KV row pack (layouts A and B), footer paging, sparse-MLA gather-dequant
// and the SWA / compressed index split.
//
// All HBM-bound byte work: one wavefront per row, every lane moving 8 input
// values (16 B for bf16) and 8 e4m3 bytes, group maxima by xor-shuffles inside
// aligned lane groups (8 lanes = 64 values for layout A, 16 lanes = 128 values
// for layout B), the group scales gathered into one lane for a single store.
#include "sgl_common.h"
#include "sgl_numeric.h"

namespace sgl {
namespace {

constexpr int A_NOPE = 448, A_DIM = 512, A_ROW = 584, A_DATA = 576;
constexpr int B_LAT = 512, B_DIM = 576, B_ROW = 656;
#ifndef SGL_KV_ROWS
#define SGL_KV_ROWS 1
#endif
#ifndef SGL_KV_BLOCKS_PER_CU
#define SGL_KV_BLOCKS_PER_CU 32
#endif
// the layout A pack: 12 blocks per CU (65 536 rows, 64-row pages: 23.7-24.0
// against 24.6 us with 32; 8: 27.2; the gathers are 2-3 us slower at 12-16)
constexpr int kPackABlocksPerCU = 12;
constexpr int kKvRows = SGL_KV_ROWS;  // rows per wavefront step in the pack kernels
// rows per wavefront step in the gather (measured at 128 x 2048 rows of a
// 65536-row cache: layout A 87 -> 74 us with 4, layout B best with 1)
#ifndef SGL_KV_GATHER_ROWS_A
#define SGL_KV_GATHER_ROWS_A 4
#endif
#ifndef SGL_KV_GATHER_ROWS_B
#define SGL_KV_GATHER_ROWS_B 1
#endif
constexpr int kKvGatherRowsA = SGL_KV_GATHER_ROWS_A;
constexpr int kKvGatherRowsB = SGL_KV_GATHER_ROWS_B;

template <int DT>
__device__ __forceinline__ void load8(const uint8_t* row, int elem, float* f, uint4* raw) {
  if constexpr (DT == SGL_F32) {
    const float4 a = *reinterpret_cast<const float4*>(row + elem * 4);
    const float4 b = *reinterpret_cast<const float4*>(row + elem * 4 + 16);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    *raw = make_uint4(0, 0, 0, 0);
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(row + elem * 2);
    *raw = v;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == SGL_BF16) {
        f[2 * i] = bits_f32(w[i] << 16);
        f[2 * i + 1] = bits_f32(w[i] & 0xFFFF0000u);
      } else {
        f[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xFFFFu));
        f[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
      }
    }
  }
}

// Row t of a footer-paged cache sits in page t / page at slot t % page: a
// shift and a mask for power-of-two pages (the 64-row pages of the
// reference), a 64-bit division otherwise.
struct PageSplit {
  int64_t pg, l;
};
__device__ __forceinline__ int page_shift_of(int page) {
  return page > 0 && (page & (page - 1)) == 0 ? __builtin_ctz((unsigned)page) : -1;
}
__device__ __forceinline__ PageSplit page_split(int64_t t, int page, int shift) {
  if (shift >= 0) return PageSplit{t >> shift, t & (int64_t)(page - 1)};
  const int64_t pg = t / page;
  return PageSplit{pg, t - pg * page};
}

// Layout A: lanes 0..55 quantize 8 NoPE values each (7 groups of 64 = 8
// lanes), lanes 56..63 carry the 128 RoPE bytes verbatim.  paged != 0 writes
// the footer page layout of to_paged_hnd directly (data at l*576 inside the
// page, scales at page*576 + l*8) and zero-fills padding rows.  A wavefront
// takes R consecutive rows per step and issues all their loads first, so R
// rows of reads are in flight per wavefront.
// Row t of a RadixCache packed pool write (engine/kv_cache.py:340-390): token
// position start + t lands in block block_table[(start + t) / page], slot
// (start + t) % page of one layer's [num_blocks, page, 584] slab.
struct PageTable {
  const int32_t* block_table;  // null: plain / footer-paged output
  int64_t start;
  int64_t num_blocks;
};

template <int DT, int R, int MODE>
__global__ __launch_bounds__(256) void kv_pack_a_kernel(const uint8_t* __restrict__ kv, int64_t T,
                                                        int64_t ld_bytes, int paged,
                                                        int page, int64_t rows_total,
                                                        uint8_t* __restrict__ out,
                                                        const PageTable pt) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  // wave-uniform row index: the paging arithmetic and the row branches run
  // on scalar registers
  const int64_t w0 = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int shift = page_shift_of(page);
  for (int64_t tb = w0 * R; tb < rows_total; tb += nwaves * R) {
    float f[R][8];
    uint4 raw[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tb + r < T) load8<DT>(kv + (tb + r) * ld_bytes, lane * 8, f[r], &raw[r]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = tb + r;
      if (t >= rows_total) break;
      uint8_t* data;
      uint8_t* foot;
      if (pt.block_table) {
        const PageSplit ps = page_split(pt.start + t, page, shift);
        const int64_t bid = pt.block_table[ps.pg];
        if (bid < 0 || bid >= pt.num_blocks) continue;  // not a block of this pool
        data = out + (bid * page + ps.l) * A_ROW;
        foot = data + A_DATA;
      } else if (paged) {
        const PageSplit ps = page_split(t, page, shift);
        uint8_t* pbase = out + ps.pg * (int64_t)page * A_ROW;
        data = pbase + ps.l * A_DATA;
        foot = pbase + (int64_t)page * A_DATA + ps.l * 8;
      } else {
        data = out + t * A_ROW;
        foot = data + A_DATA;
      }
      if (t >= T) {  // padding row of the last page
        if (lane < 72) *reinterpret_cast<uint2*>(data + lane * 8) = make_uint2(0, 0);
        if (lane < 8) *reinterpret_cast<uint2*>(data + 512 + lane * 8) = make_uint2(0, 0);
        if (lane == 0) *reinterpret_cast<uint2*>(foot) = make_uint2(0, 0);
        continue;
      }
      // IEEE maximum (v_maximum3_f32): NaN propagates into the group's scale
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = __builtin_elementwise_maximum(amax, fabsf(f[r][i]));
      amax = lane_group_max<8>(amax);
      const float sf = group_scale(MODE, amax);
      const uint32_t sbyte = pow2_to_e8m0(sf);
      if (lane < 56) {
        *reinterpret_cast<uint2*>(data + lane * 8) = quant8_e4m3(MODE, f[r], sf);
      } else {
        // rope bytes as given (bf16 / f16), 16 per lane at 448 + 16*(lane-56)
        uint8_t* dst = data + A_NOPE + (lane - 56) * 16;
        *reinterpret_cast<uint2*>(dst) = make_uint2(raw[r].x, raw[r].y);
        *reinterpret_cast<uint2*>(dst + 8) = make_uint2(raw[r].z, raw[r].w);
      }
      // 7 scale bytes + zero pad -> one 8-byte store by lane 0 (the bytes
      // are read lane by lane into scalar registers)
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int g = 0; g < 7; ++g) {
        const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)sbyte, g * 8) & 0xFFu;
        if (g < 4)
          lo |= b << (8 * g);
        else
          hi |= b << (8 * (g - 4));
      }
      if (lane == 0) *reinterpret_cast<uint2*>(foot) = make_uint2(lo, hi);
    }
  }
}

// Layout B: 64 lanes x 8 latent values (4 groups of 128 = 16 lanes each),
// then lanes 0..7 copy the 128 RoPE bytes; 4 fp32 scales stored by lane 0.
// R consecutive rows per wavefront step, loads first.
template <int DT, int R>
__global__ __launch_bounds__(256) void kv_pack_b_kernel(const uint8_t* __restrict__ kv, int64_t T,
                                                        int64_t ld_bytes,
                                                        uint8_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const int64_t w0 = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  constexpr int ES = DT == SGL_F32 ? 4 : 2;
  for (int64_t tb = w0 * R; tb < T; tb += nwaves * R) {
    float f[R][8];
    uint4 raw[R];
    float rf[R][8];  // fp32 input: the rope values of lanes 0..7
    uint4 rope[R];   // 16-bit input: the rope bytes of lanes 0..7
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (tb + r >= T) break;
      const uint8_t* row = kv + (tb + r) * ld_bytes;
      load8<DT>(row, lane * 8, f[r], &raw[r]);
      if (lane < 8) {
        if constexpr (DT == SGL_F32) {
          uint4 unused;
          load8<DT>(row, B_LAT + lane * 8, rf[r], &unused);
        } else {
          rope[r] = *reinterpret_cast<const uint4*>(row + (B_LAT + lane * 8) * ES);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = tb + r;
      if (t >= T) break;
      uint8_t* o = out + t * B_ROW;
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf_(amax, fabsf(f[r][i]));
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) amax = fmaxf_(amax, __shfl_xor(amax, off, 64));
      const float sf = group_scale(SCALE_TORCH_FP32, amax);
      *reinterpret_cast<uint2*>(o + lane * 8) = quant8_e4m3(SCALE_TORCH_FP32, f[r], sf);
      if (lane < 8) {
        if constexpr (DT == SGL_F32) {
          // fp32 input: rope stored as bf16 (RNE) so the row stays 656 B
          uint32_t w[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) w[i] = pk2_bf16_exact(rf[r][2 * i], rf[r][2 * i + 1]);
          *reinterpret_cast<uint4*>(o + B_LAT + lane * 16) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
          *reinterpret_cast<uint4*>(o + B_LAT + lane * 16) = rope[r];
        }
      }
      const float s0 = __shfl(sf, 0, 64), s1 = __shfl(sf, 16, 64), s2 = __shfl(sf, 32, 64),
                  s3 = __shfl(sf, 48, 64);
      if (lane == 0) *reinterpret_cast<float4*>(o + 640) = make_float4(s0, s1, s2, s3);
    }
  }
}

__global__ __launch_bounds__(256) void kv_to_paged_kernel(const uint8_t* __restrict__ packed,
                                                          int64_t T, int page, int64_t rows_total,
                                                          uint8_t* __restrict__ pages) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const int shift = page_shift_of(page);
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < rows_total; t += nwaves) {
    const PageSplit ps = page_split(t, page, shift);
    const int64_t pg = ps.pg, l = ps.l;
    uint8_t* pbase = pages + pg * (int64_t)page * A_ROW;
    // 73 eight-byte words per row: 72 data words, 1 footer word
    for (int w = lane; w < 73; w += 64) {
      const uint2 v = t < T ? *reinterpret_cast<const uint2*>(packed + t * A_ROW + w * 8)
                            : make_uint2(0, 0);
      uint8_t* dst = w < 72 ? pbase + l * A_DATA + w * 8 : pbase + (int64_t)page * A_DATA + l * 8;
      *reinterpret_cast<uint2*>(dst) = v;
    }
  }
}

// One wavefront per gathered row, R rows per step.  The R indices of a step
// come in with one load, issued in the step before (ahead of that step's row
// loads, so waiting for them never waits for rows), and the row loads are
// unconditional (an index outside [0, n_rows) reads row 0, and its output
// row is written as zeros), so no branch splits them and all R rows stay in
// flight together.  Layout A: out 512 bf16 = 448 dequantized (e4m3 *
// 2^(e8m0-127), exact in bf16) + 64 rope; layout B: out 576 bf16 = 512
// bf16(e4m3 * fp32 scale) + 64 rope.
template <int LAYOUT, int R>
__global__ __launch_bounds__(256) void kv_gather_kernel(const uint8_t* __restrict__ cache,
                                                        int paged, int page, int64_t n_rows,
                                                        const int32_t* __restrict__ idx,
                                                        int64_t total, uint16_t* __restrict__ out) {
  constexpr int ODIM = LAYOUT == SGL_KV_LAYOUT_A ? A_DIM : B_DIM;
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  // wave-uniform row index: output addresses and row checks on scalar registers
  const int64_t w0 = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int shift = page_shift_of(page);
  // lane r < R: index r of the step starting at rb (clamped into the array)
  auto load_idx = [&](int64_t rb) -> int32_t {
    const int64_t i = rb + (lane < R ? lane : 0);
    return idx[i < total ? i : total - 1];
  };
  int64_t rb = w0 * R;
  int32_t my_id = rb < total ? load_idx(rb) : -1;
  for (; rb < total; rb += nwaves * R) {
    int32_t id[R];
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int32_t v = __builtin_amdgcn_readlane(my_id, r);
      ok[r] = rb + r < total && v >= 0 && v < n_rows;
      id[r] = ok[r] ? v : 0;
    }
    if (rb + nwaves * R < total) my_id = load_idx(rb + nwaves * R);
    uint2 qv[R];
    uint32_t sraw[R];  // layout A: the e8m0 byte; layout B: the fp32 scale bits
    uint4 rope[R];
    if (n_rows > 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (LAYOUT == SGL_KV_LAYOUT_A) {
          const uint8_t* data;
          const uint8_t* foot;
          if (paged) {
            const PageSplit ps = page_split(id[r], page, shift);
            const int64_t pg = ps.pg, l = ps.l;
            const uint8_t* pbase = cache + pg * (int64_t)page * A_ROW;
            data = pbase + l * A_DATA;
            foot = pbase + (int64_t)page * A_DATA + l * 8;
          } else {
            data = cache + (int64_t)id[r] * A_ROW;
            foot = data + A_DATA;
          }
          // lanes < 56: 8 e4m3 bytes + the group's scale byte; lanes 56..63:
          // 16 rope bytes (two 8-byte halves)
          const uint8_t* src = lane < 56 ? data + lane * 8 : data + A_NOPE + (lane - 56) * 16;
          const uint2 x = *reinterpret_cast<const uint2*>(src);
          const uint2 y = *reinterpret_cast<const uint2*>(lane < 56 ? foot : src + 8);
          qv[r] = x;
          sraw[r] = (y.x >> (8 * ((lane >> 3) & 3))) & 0xFFu;
          if ((lane >> 3) >= 4) sraw[r] = (y.y >> (8 * ((lane >> 3) & 3))) & 0xFFu;
          rope[r] = make_uint4(x.x, x.y, y.x, y.y);
        } else {
          const uint8_t* row = cache + (int64_t)id[r] * B_ROW;
          qv[r] = *reinterpret_cast<const uint2*>(row + lane * 8);
          sraw[r] = *reinterpret_cast<const uint32_t*>(row + 640 + (lane >> 4) * 4);
          rope[r] = *reinterpret_cast<const uint4*>(row + B_LAT + (lane & 7) * 16);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (rb + r >= total) break;
      uint16_t* o = out + (rb + r) * ODIM;
      if (!ok[r]) {
        const uint4 z = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(o + lane * 8) = z;
        if (LAYOUT == SGL_KV_LAYOUT_B && lane < 8) *reinterpret_cast<uint4*>(o + 512 + lane * 8) = z;
        continue;
      }
      const bool deq = LAYOUT == SGL_KV_LAYOUT_B || lane < 56;
      // Products are NaN only from an e4m3 NaN code (S.1111.111) or a NaN
      // scale (layout A: the 0xFF byte; layout B: NaN bits); a row with
      // neither in any lane takes the plain conversion, which equals the
      // NaN-canonicalising one for every other value (one wave-uniform test)
      const uint32_t t0 = qv[r].x & 0x7F7F7F7Fu, t1 = qv[r].y & 0x7F7F7F7Fu;
      const bool code_nan = (((t0 + 0x01010101u) | (t1 + 0x01010101u)) & 0x80808080u) != 0u;
      const bool scale_nan = LAYOUT == SGL_KV_LAYOUT_A ? sraw[r] == 0xFFu : (sraw[r] & 0x7FFFFFFFu) > 0x7F800000u;
      const bool exact = __ballot(deq && (code_nan || scale_nan)) != 0ull;
      if (deq) {
        float sc;
        if constexpr (LAYOUT == SGL_KV_LAYOUT_A) {
          // 2^(sb - 127); byte 0 is 2^-127 (0x00400000) and 0xFF the NaN
          // 0x7FC00000: both take the 0x400000 bit
          const uint32_t sb = sraw[r];
          sc = bits_f32((sb << 23) | (sb == 0u || sb == 0xFFu ? 0x00400000u : 0u));
        } else {
          sc = bits_f32(sraw[r]);
        }
        float d[8];
        unpack4_e4m3(qv[r].x, d);
        unpack4_e4m3(qv[r].y, d + 4);
        uint32_t w[4];
        if (exact) {
#pragma unroll
          for (int i = 0; i < 4; ++i) w[i] = pk2_bf16_exact(d[2 * i] * sc, d[2 * i + 1] * sc);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) w[i] = pk2_bf16(d[2 * i] * sc, d[2 * i + 1] * sc);
        }
        *reinterpret_cast<uint4*>(o + lane * 8) = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
        *reinterpret_cast<uint4*>(o + lane * 8) = rope[r];
      }
      if (LAYOUT == SGL_KV_LAYOUT_B && lane < 8) *reinterpret_cast<uint4*>(o + 512 + lane * 8) = rope[r];
    }
  }
}

template <typename IT>
__global__ __launch_bounds__(256) void split_indices_kernel(const IT* __restrict__ topk, int64_t BS,
                                                            int64_t K, int64_t window,
                                                            int32_t* __restrict__ swa,
                                                            int32_t* __restrict__ swa_lens,
                                                            int32_t* __restrict__ comp,
                                                            int32_t* __restrict__ comp_lens) {
  const int lane = threadIdx.x & 63;
  const int64_t swa_k = window < K ? window : K;
  const int64_t comp_k = K - swa_k;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); b < BS; b += nwaves) {
    int n_swa = 0, n_comp = 0;
    for (int64_t c0 = 0; c0 < K; c0 += 64) {
      const int64_t c = c0 + lane;
      const bool in = c < K;
      const int32_t v = in ? (int32_t)topk[b * K + c] : -1;
      const bool valid = in && v >= 0;
      const bool is_swa = c < swa_k;
      if (in && is_swa) swa[b * swa_k + c] = v;
      if (in && !is_swa) comp[b * comp_k + (c - swa_k)] = valid ? (int32_t)(v - window) : v;
      n_swa += __popcll(__ballot(valid && is_swa));
      n_comp += __popcll(__ballot(valid && !is_swa));
    }
    if (lane == 0) {
      swa_lens[b] = n_swa;
      comp_lens[b] = n_comp;
    }
  }
}

// 4 wavefronts per block, rows_per_wave rows per wavefront step; at most
// blocks_per_cu blocks per CU, the rest loop.
unsigned grid_for_rows(int64_t rows, int rows_per_wave = 1, int blocks_per_cu = SGL_KV_BLOCKS_PER_CU) {
  int64_t blocks = ceil_div(rows, 4 * (int64_t)rows_per_wave);
  const int64_t cap = (int64_t)device_cu_count() * blocks_per_cu;
  if (blocks > cap) blocks = cap;
  return (unsigned)(blocks < 1 ? 1 : blocks);
}

// layout A launch for the three ue8m0 scale modes (compile-time in the kernel)
template <int DT>
void launch_pack_a(unsigned g, hipStream_t st, int mode, const uint8_t* kv, int64_t T, int64_t ld_bytes,
                   int paged, int page, int64_t rows, uint8_t* out, const PageTable& pt) {
  if (mode == SGL_SCALE_KV_UE8M0)
    kv_pack_a_kernel<DT, kKvRows, SGL_SCALE_KV_UE8M0><<<g, 256, 0, st>>>(kv, T, ld_bytes, paged, page, rows, out, pt);
  else if (mode == SGL_SCALE_TORCH_UE8M0)
    kv_pack_a_kernel<DT, kKvRows, SGL_SCALE_TORCH_UE8M0><<<g, 256, 0, st>>>(kv, T, ld_bytes, paged, page, rows,
                                                                          out, pt);
  else
    kv_pack_a_kernel<DT, kKvRows, SGL_SCALE_TILELANG_UE8M0><<<g, 256, 0, st>>>(kv, T, ld_bytes, paged, page, rows,
                                                                             out, pt);
}

bool ue8m0_mode(int m) {
  return m == SGL_SCALE_KV_UE8M0 || m == SGL_SCALE_TILELANG_UE8M0 || m == SGL_SCALE_TORCH_UE8M0;
}

}  // namespace
}  // namespace sgl

extern "C" {

int sgl_kv_pack(const void* kv, int dtype, int64_t T, int64_t ldkv, int layout, int scale_mode,
                int paged, int page_size, void* out, sgl_stream_t stream) {
  SGL_REQUIRE(T >= 0, "kv_pack: negative T");
  SGL_REQUIRE(dtype == SGL_BF16 || dtype == SGL_F16 || dtype == SGL_F32, "kv_pack: bad dtype");
  SGL_REQUIRE(layout == SGL_KV_LAYOUT_A || layout == SGL_KV_LAYOUT_B, "kv_pack: bad layout");
  hipStream_t st = (hipStream_t)stream;
  const int es = dtype == SGL_F32 ? 4 : 2;
  if (layout == SGL_KV_LAYOUT_A) {
    SGL_REQUIRE(sgl::ue8m0_mode(scale_mode), "kv_pack: layout A needs a ue8m0 scale mode (got %d)",
                scale_mode);
    SGL_REQUIRE(dtype != SGL_F32, "kv_pack: layout A stores the rope as 16-bit values; fp32 "
                                  "input is not representable in the 584-byte row");
    SGL_REQUIRE(ldkv >= 512, "kv_pack: layout A row stride %lld < 512", (long long)ldkv);
    SGL_REQUIRE(!paged || page_size > 0, "kv_pack: page_size must be positive");
    const int64_t rows = paged ? sgl::ceil_div(T, page_size) * page_size : T;
    if (rows == 0) return SGL_OK;
    SGL_REQUIRE(out && (T == 0 || kv), "kv_pack: null pointer");
    SGL_REQUIRE(sgl::aligned(out, 8) && (T == 0 || (sgl::aligned(kv, 16) && (ldkv * es) % 16 == 0)),
                "kv_pack: kv rows must be 16-byte aligned, out 8-byte aligned");
    const unsigned g = sgl::grid_for_rows(rows, sgl::kKvRows, sgl::kPackABlocksPerCU);
    if (dtype == SGL_BF16)
      sgl::launch_pack_a<SGL_BF16>(g, st, scale_mode, (const uint8_t*)kv, T, ldkv * es, paged, page_size,
                                   rows, (uint8_t*)out, sgl::PageTable{});
    else
      sgl::launch_pack_a<SGL_F16>(g, st, scale_mode, (const uint8_t*)kv, T, ldkv * es, paged, page_size,
                                  rows, (uint8_t*)out, sgl::PageTable{});
    return sgl::check_launch("kv_pack_a");
  }
  SGL_REQUIRE(!paged, "kv_pack: layout B has no paged form");
  SGL_REQUIRE(ldkv >= 576, "kv_pack: layout B row stride %lld < 576", (long long)ldkv);
  if (T == 0) return SGL_OK;
  SGL_REQUIRE(kv && out, "kv_pack: null pointer");
  SGL_REQUIRE(sgl::aligned(out, 16) && sgl::aligned(kv, 16) && (ldkv * es) % 16 == 0,
              "kv_pack: layout B rows must be 16-byte aligned");
  const unsigned g = sgl::grid_for_rows(T, sgl::kKvRows);
  if (dtype == SGL_BF16)
    sgl::kv_pack_b_kernel<SGL_BF16, sgl::kKvRows><<<g, 256, 0, st>>>((const uint8_t*)kv, T, ldkv * es,
                                                       (uint8_t*)out);
  else if (dtype == SGL_F16)
    sgl::kv_pack_b_kernel<SGL_F16, sgl::kKvRows><<<g, 256, 0, st>>>((const uint8_t*)kv, T, ldkv * es,
                                                      (uint8_t*)out);
  else
    sgl::kv_pack_b_kernel<SGL_F32, sgl::kKvRows><<<g, 256, 0, st>>>((const uint8_t*)kv, T, ldkv * es,
                                                      (uint8_t*)out);
  return sgl::check_launch("kv_pack_b");
}

int sgl_kv_pack_to_pages(const void* kv, int dtype, int64_t T, int64_t ldkv, int scale_mode,
                         const int32_t* block_table, int64_t n_pages, int64_t start_pos,
                         int page_size, int64_t num_blocks, int layer_idx, int num_layers,
                         void* pool, sgl_stream_t stream) {
  SGL_REQUIRE(T >= 0 && start_pos >= 0 && page_size > 0 && num_blocks >= 0,
              "kv_pack_to_pages: bad T / start_pos / page_size / num_blocks");
  SGL_REQUIRE(dtype == SGL_BF16 || dtype == SGL_F16,
              "kv_pack_to_pages: kv must be bf16 or f16 (the 584-byte row stores 16-bit rope)");
  SGL_REQUIRE(sgl::ue8m0_mode(scale_mode),
              "kv_pack_to_pages: layout A needs a ue8m0 scale mode (got %d)", scale_mode);
  SGL_REQUIRE(layer_idx >= 0 && layer_idx < num_layers, "kv_pack_to_pages: layer_idx %d out of range (%d)",
              layer_idx, num_layers);
  SGL_REQUIRE(ldkv >= 512, "kv_pack_to_pages: row stride %lld < 512", (long long)ldkv);
  if (T == 0) return SGL_OK;
  const int64_t pages_needed = sgl::ceil_div(start_pos + T, (int64_t)page_size);
  if (pages_needed > n_pages) {
    sgl::set_error("kv_pack_to_pages: block_table too short for packed pos=%lld: pages=%lld",
                   (long long)(start_pos + T - 1), (long long)n_pages);
    return SGL_ERR_INVALID_ARG;
  }
  SGL_REQUIRE(kv && block_table && pool, "kv_pack_to_pages: null pointer");
  const int es = 2;
  SGL_REQUIRE(sgl::aligned(pool, 8) && sgl::aligned(kv, 16) && (ldkv * es) % 16 == 0,
              "kv_pack_to_pages: kv rows must be 16-byte aligned, pool 8-byte aligned");
  uint8_t* slab = (uint8_t*)pool + (int64_t)layer_idx * num_blocks * page_size * sgl::A_ROW;
  const sgl::PageTable pt{block_table, start_pos, num_blocks};
  const unsigned g = sgl::grid_for_rows(T, sgl::kKvRows, sgl::kPackABlocksPerCU);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == SGL_BF16)
    sgl::launch_pack_a<SGL_BF16>(g, st, scale_mode, (const uint8_t*)kv, T, ldkv * es, 0, page_size, T, slab, pt);
  else
    sgl::launch_pack_a<SGL_F16>(g, st, scale_mode, (const uint8_t*)kv, T, ldkv * es, 0, page_size, T, slab, pt);
  return sgl::check_launch("kv_pack_to_pages");
}

int sgl_kv_to_paged(const void* packed, int64_t T, int page_size, void* pages,
                    sgl_stream_t stream) {
  SGL_REQUIRE(T >= 0 && page_size > 0, "kv_to_paged: bad T / page_size");
  const int64_t rows = sgl::ceil_div(T, page_size) * page_size;
  if (rows == 0) return SGL_OK;
  SGL_REQUIRE(pages && (T == 0 || packed), "kv_to_paged: null pointer");
  SGL_REQUIRE(sgl::aligned(pages, 8) && sgl::aligned(packed, 8), "kv_to_paged: misaligned");
  sgl::kv_to_paged_kernel<<<sgl::grid_for_rows(rows), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)packed, T, page_size, rows, (uint8_t*)pages);
  return sgl::check_launch("kv_to_paged");
}

int sgl_kv_gather_dequant(const void* cache, int layout, int paged, int page_size, int64_t n_rows,
                          const int32_t* idx, int64_t nq, int64_t nsel, void* out,
                          sgl_stream_t stream) {
  SGL_REQUIRE(layout == SGL_KV_LAYOUT_A || layout == SGL_KV_LAYOUT_B, "kv_gather: bad layout");
  SGL_REQUIRE(nq >= 0 && nsel >= 0 && n_rows >= 0, "kv_gather: negative size");
  SGL_REQUIRE(!paged || (layout == SGL_KV_LAYOUT_A && page_size > 0),
              "kv_gather: paged caches are layout A with a positive page_size");
  const int64_t total = nq * nsel;
  if (total == 0) return SGL_OK;
  SGL_REQUIRE(idx && out && (n_rows == 0 || cache), "kv_gather: null pointer");
  SGL_REQUIRE(sgl::aligned(out, 16) && sgl::aligned(cache, layout == SGL_KV_LAYOUT_B ? 16 : 8),
              "kv_gather: misaligned cache/out");
  hipStream_t st = (hipStream_t)stream;
  if (layout == SGL_KV_LAYOUT_A)
    sgl::kv_gather_kernel<SGL_KV_LAYOUT_A, sgl::kKvGatherRowsA>
        <<<sgl::grid_for_rows(total, sgl::kKvGatherRowsA), 256, 0, st>>>(
        (const uint8_t*)cache, paged, page_size, n_rows, idx, total, (uint16_t*)out);
  else
    sgl::kv_gather_kernel<SGL_KV_LAYOUT_B, sgl::kKvGatherRowsB>
        <<<sgl::grid_for_rows(total, sgl::kKvGatherRowsB), 256, 0, st>>>(
        (const uint8_t*)cache, 0, 1, n_rows, idx, total, (uint16_t*)out);
  return sgl::check_launch("kv_gather_dequant");
}

int sgl_split_swa_compress_indices(const void* topk, int idx_int64, int64_t BS, int64_t K,
                                   int64_t window, int32_t* swa, int32_t* swa_lens,
                                   int32_t* comp, int32_t* comp_lens, sgl_stream_t stream) {
  SGL_REQUIRE(BS >= 0 && K >= 0 && window >= 0, "split_indices: negative size");
  if (BS == 0) return SGL_OK;
  SGL_REQUIRE(swa_lens && comp_lens && (K == 0 || topk), "split_indices: null pointer");
  const int64_t swa_k = window < K ? window : K;
  SGL_REQUIRE((swa_k == 0 || swa) && (K - swa_k == 0 || comp), "split_indices: null pointer");
  const unsigned g = sgl::grid_for_rows(BS);
  hipStream_t st = (hipStream_t)stream;
  if (idx_int64)
    sgl::split_indices_kernel<int64_t><<<g, 256, 0, st>>>((const int64_t*)topk, BS, K, window, swa,
                                                          swa_lens, comp, comp_lens);
  else
    sgl::split_indices_kernel<int32_t><<<g, 256, 0, st>>>((const int32_t*)topk, BS, K, window, swa,
                                                          swa_lens, comp, comp_lens);
  return sgl::check_launch("split_swa_compress_indices");
}

}  // extern "C"
