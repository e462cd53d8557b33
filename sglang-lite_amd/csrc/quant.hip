// Activation (1 x G) and weight (128 x 128) FP8 quantization kernels.
//
// Both are HBM-bound: act_quant moves 2 B in + 1 B out per element plus one
// scale per group.  One group of G bf16 values is owned by G/8 consecutive
// lanes, each holding 8 values (one 16-byte load), so a 64-lane wavefront
// covers 8 (G = 64) or 4 (G = 128) groups per iteration and the group's |x|
// maximum needs log2(G/8) cross-lane steps.
#include <type_traits>

#include "sgl_common.h"
#include "sgl_numeric.h"

#ifndef SGL_AQ_ROWS
#define SGL_AQ_ROWS 1
#endif
#ifndef SGL_AQ_BLOCKS_PER_CU
#define SGL_AQ_BLOCKS_PER_CU 32
#endif

namespace sgl {
namespace {

__device__ __forceinline__ void unpack_bf16x8(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bits_f32(w[i] << 16);
    f[2 * i + 1] = bits_f32(w[i] & 0xFFFF0000u);
  }
}

// IEEE maximum (v_maximum_f32) over the group's lanes, by DPP: a NaN element
// makes the group's amax NaN, as the reference's amax does
template <int LPG>
__device__ __forceinline__ float group_max(float v) {
  return lane_group_max<LPG>(v);
}

// R groups per thread and step (group g, g + sweep, ...), loads first, so R
// 16-byte reads per lane are in flight.
// The scale mode is a template parameter (one straight-line kernel per mode);
// IDX32: group indices fit 32 bits, so row = g / gpr is a 32-bit division.
template <int GROUP, bool INPLACE, int R, int MODE, bool IDX32>
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                        int64_t K, int64_t ldx, void* __restrict__ y,
                                                        int64_t ldy, void* __restrict__ s,
                                                        int64_t lds, int scale_e8m0) {
  constexpr int LPG = GROUP / 8;
  const int64_t gpr = K / GROUP;
  const int64_t total = M * gpr;
  auto row_of = [&](int64_t g) -> int64_t {
    if constexpr (IDX32) return (int64_t)((uint32_t)g / (uint32_t)gpr);
    return g / gpr;
  };
  const int sub = threadIdx.x % LPG;
  const int64_t sweep = (int64_t)gridDim.x * blockDim.x / LPG;
  for (int64_t gb = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / LPG; gb < total;
       gb += sweep * R) {
    uint4 v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t g = gb + r * sweep;
      if (g < total) {
        const int64_t row = row_of(g);
        const int64_t col = (g - row * gpr) * GROUP + sub * 8;
        v[r] = *reinterpret_cast<const uint4*>(x + row * ldx + col);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t g = gb + r * sweep;
      if (g >= total) break;
      const int64_t row = row_of(g);
      const int64_t col = (g - row * gpr) * GROUP + sub * 8;
      float f[8];
      unpack_bf16x8(v[r], f);
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = __builtin_elementwise_maximum(amax, fabsf(f[i]));
      amax = group_max<LPG>(amax);
      const float sf = group_scale(MODE, amax);
      const uint2 qv = quant8_e4m3(MODE, f, sf);
      if (INPLACE) {
        // quant-dequant back to bf16: bf16(fp32(e4m3) * s)
        float d[8];
        unpack4_e4m3(qv.x, d);
        unpack4_e4m3(qv.y, d + 4);
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pk2_bf16_exact(d[2 * i] * sf, d[2 * i + 1] * sf);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(y) + row * ldy + col) =
            make_uint4(o[0], o[1], o[2], o[3]);
      } else {
        *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(y) + row * ldy + col) = qv;
      }
      if (sub == 0) {
        const int64_t si = row * lds + col / GROUP;
        if (scale_e8m0)
          reinterpret_cast<uint8_t*>(s)[si] = pow2_to_e8m0(sf);
        else
          reinterpret_cast<float*>(s)[si] = sf;
      }
    }
  }
}

// One 256-thread block per 128 x 128 weight block.  Thread t owns the 8
// columns [8*(t%16), +8) of rows t/16 + 16*i, i < 8.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float* f);
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* f) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float* f) {
  unpack_bf16x8(*reinterpret_cast<const uint4*>(p), f);
}

template <typename T>
__global__ __launch_bounds__(256) void weight_quant_kernel(const T* __restrict__ w, int64_t N,
                                                           int64_t K, int64_t ldw,
                                                           uint8_t* __restrict__ q, int64_t ldq,
                                                           float* __restrict__ s, int64_t lds,
                                                           int use_ue8m0) {
  __shared__ float red[4];
  const int64_t bn = blockIdx.y, bk = blockIdx.x;
  const int t = threadIdx.x;
  const int64_t col = bk * 128 + (t % 16) * 8;
  const bool col_ok = col < K;  // K % 8 == 0: a chunk is all in or all out
  float v[8][8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t row = bn * 128 + t / 16 + 16 * i;
    if (col_ok && row < N) {
      load8<T>(w + row * ldw + col, v[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf_(amax, fabsf(v[i][j]));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf_(amax, __shfl_xor(amax, o, 64));
  if ((t & 63) == 0) red[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf_(fmaxf_(red[0], red[1]), fmaxf_(red[2], red[3]));
  float sf = fmaxf_(amax, 1e-4f) / 448.0f;
  if (use_ue8m0) sf = ceil_to_ue8m0(sf);
  const float inv = 1.0f / sf;
  if (t == 0) s[bn * lds + bk] = sf;
  if (!col_ok) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t row = bn * 128 + t / 16 + 16 * i;
    if (row >= N) continue;
    const uint32_t lo = pk4_e4m3_exact(v[i][0] * inv, v[i][1] * inv, v[i][2] * inv, v[i][3] * inv);
    const uint32_t hi = pk4_e4m3_exact(v[i][4] * inv, v[i][5] * inv, v[i][6] * inv, v[i][7] * inv);
    *reinterpret_cast<uint2*>(q + row * ldq + col) = make_uint2(lo, hi);
  }
}

__global__ void e8m0_to_f32_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                   int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t b = src[i];
    // 0xFF is the e8m0 NaN code; 0 is 2^-127 (an fp32 subnormal)
    dst[i] = b == 0xFFu ? bits_f32(0x7FC00000u) : (b == 0 ? bits_f32(0x00400000u) : bits_f32(b << 23));
  }
}

// e2m1 code -> fp32: sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0
// (0, 0.5, 1, 1.5, 2, 3, 4, 6 and their negatives).  Code 8 (the format's -0)
// decodes to +0.0 as the checkpoint converter's table has it
// (deepseek_infer/convert.py:11-14, FP4_TABLE[8] = 0.0), so the repack writes
// e4m3 0x00 there, not 0x80.
__device__ __forceinline__ float e2m1_value(uint32_t c) {
  const uint32_t e = (c >> 1) & 3u, m = c & 1u;
  const float mag = e == 0 ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, (int)e - 1);
  return ((c & 8u) && (c & 7u)) ? -mag : mag;
}

// Lossless FP4 -> FP8 weight repack (deepseek_infer/convert.py:17-52), one
// workgroup per 128 x 128 block.  Thread t covers row t/2 of the block and
// its 64 elements [64 (t%2), +64): 32 packed bytes under two e8m0 scales.
__global__ __launch_bounds__(256) void fp4_to_fp8_weight_kernel(
    const uint8_t* __restrict__ b, const uint8_t* __restrict__ sb, int64_t K,
    uint8_t* __restrict__ q, uint8_t* __restrict__ s_out) {
  __shared__ uint32_t sMax[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t kb = blockIdx.x, nb = blockIdx.y;
  const int r = tid >> 1, hf = tid & 1;
  const int64_t n = nb * 128 + r;
  const uint8_t* sp = sb + n * (K / 32) + kb * 4 + hf * 2;
  const uint32_t s0 = sp[0], s1 = sp[1];
  // the block's largest scale; 0xFF (NaN) is also the largest byte, and a
  // NaN scale makes the whole block NaN as torch's amax does
  uint32_t m = s0 > s1 ? s0 : s1;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t v = (uint32_t)__shfl_xor((int)m, o, 64);
    m = v > m ? v : m;
  }
  if (lane == 0) sMax[wave] = m;
  __syncthreads();
  uint32_t smax = sMax[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) smax = sMax[w] > smax ? sMax[w] : smax;
  const bool nan = smax == 0xFFu;
  // s = smax / 2^6 (clamped at the smallest e8m0, 2^-127)
  const int sbyte = smax >= 6 ? (int)smax - 6 : 0;
  if (tid == 0) s_out[nb * (K / 128) + kb] = nan ? 0xFF : (uint8_t)sbyte;

  const uint8_t* bp = b + n * (K / 2) + kb * 64 + hf * 32;
  uint8_t* qp = q + n * K + kb * 128 + hf * 64;
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // packed bytes [16 h, 16 h + 16): elements under scale s_h
    const uint4 v = *reinterpret_cast<const uint4*>(bp + 16 * h);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    const int off = (int)(h ? s1 : s0) - sbyte;  // scale / s = 2^off, off <= 6
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float f[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t byte = (w[i] >> (8 * j)) & 0xFFu;
        f[2 * j] = ldexpf(e2m1_value(byte & 0xFu), off);
        f[2 * j + 1] = ldexpf(e2m1_value(byte >> 4), off);
      }
      o[2 * i] = nan ? 0x7F7F7F7Fu : pk4_e4m3_exact(f[0], f[1], f[2], f[3]);
      o[2 * i + 1] = nan ? 0x7F7F7F7Fu : pk4_e4m3_exact(f[4], f[5], f[6], f[7]);
    }
    *reinterpret_cast<uint4*>(qp + 32 * h) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4*>(qp + 32 * h + 16) = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

// Self-check of the hardware conversions over every fp32 bit pattern: thread
// t of a launch covers inputs start + 4t .. start + 4t + 3.
//   counts[0]: pk4_e4m3_exact != f32_to_e4m3   (all inputs)
//   counts[1]: pk2_bf16_exact != f32_to_bf16   (all inputs)
//   counts[2]: pk4_e4m3 != f32_to_e4m3         (non-NaN inputs)
//   counts[3]: pk2_bf16 != f32_to_bf16         (non-NaN inputs)
//   counts[4]: unpack4_e4m3 != e4m3_to_f32      (256 codes; NaN code -> any NaN)
__global__ void check_conversions_kernel(uint64_t start, unsigned long long* counts) {
  const uint64_t u0 = start + ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  float x[4];
  uint32_t sw8 = 0;
  unsigned c[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = bits_f32((uint32_t)(u0 + i));
    sw8 |= (uint32_t)f32_to_e4m3(x[i]) << (8 * i);
  }
  const uint32_t hx = pk4_e4m3_exact(x[0], x[1], x[2], x[3]);
  const uint32_t hr = pk4_e4m3(x[0], x[1], x[2], x[3]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t s8 = (sw8 >> (8 * i)) & 0xFFu;
    c[0] += ((hx >> (8 * i)) & 0xFFu) != s8;
    c[2] += (x[i] == x[i]) && ((hr >> (8 * i)) & 0xFFu) != s8;
  }
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    const uint32_t sw = (uint32_t)f32_to_bf16(x[i]) | ((uint32_t)f32_to_bf16(x[i + 1]) << 16);
    const uint32_t ex = pk2_bf16_exact(x[i], x[i + 1]);
    const uint32_t raw = pk2_bf16(x[i], x[i + 1]);
    c[1] += (ex & 0xFFFFu) != (sw & 0xFFFFu);
    c[1] += (ex >> 16) != (sw >> 16);
    c[3] += (x[i] == x[i]) && (raw & 0xFFFFu) != (sw & 0xFFFFu);
    c[3] += (x[i + 1] == x[i + 1]) && (raw >> 16) != (sw >> 16);
  }
  unsigned c4 = 0;
  if (u0 < 1024) {  // the 256 e4m3 codes, one per thread of the first launch
    const uint32_t code = (uint32_t)(u0 >> 2);
    float hw[4];
    unpack4_e4m3(code, hw);
    const float ref = e4m3_to_f32((uint8_t)code);
    c4 = ref != ref ? (hw[0] == hw[0]) : (f32_bits(hw[0]) != f32_bits(ref));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (c[i]) atomicAdd(&counts[i], (unsigned long long)c[i]);
  if (c4) atomicAdd(&counts[4], (unsigned long long)c4);
}

template <int GROUP>
int launch_act_quant(const void* x, int64_t M, int64_t K, int64_t ldx, void* y, int64_t ldy,
                     void* s, int64_t lds, int mode, int scale_e8m0, int inplace,
                     hipStream_t stream) {
  constexpr int R = SGL_AQ_ROWS;
  const int64_t total_threads = M * (K / GROUP) * (GROUP / 8);
  const int64_t max_blocks = (int64_t)device_cu_count() * SGL_AQ_BLOCKS_PER_CU;
  int64_t blocks = ceil_div(total_threads, 256 * R);
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  const bool idx32 = M * (K / GROUP) + (int64_t)blocks * 256 * R < ((int64_t)1 << 31);
  auto go = [&](auto inplace_c, auto mode_c, auto idx_c) {
    act_quant_kernel<GROUP, decltype(inplace_c)::value, R, decltype(mode_c)::value, decltype(idx_c)::value>
        <<<(unsigned)blocks, 256, 0, stream>>>((const uint16_t*)x, M, K, ldx, y, ldy, s, lds, scale_e8m0);
  };
  auto with_mode = [&](auto inplace_c, auto idx_c) {
    switch (mode) {
      case SCALE_TORCH_FP32: go(inplace_c, std::integral_constant<int, SCALE_TORCH_FP32>{}, idx_c); break;
      case SCALE_TORCH_UE8M0: go(inplace_c, std::integral_constant<int, SCALE_TORCH_UE8M0>{}, idx_c); break;
      case SCALE_TILELANG_FP32: go(inplace_c, std::integral_constant<int, SCALE_TILELANG_FP32>{}, idx_c); break;
      case SCALE_TILELANG_UE8M0:
        go(inplace_c, std::integral_constant<int, SCALE_TILELANG_UE8M0>{}, idx_c);
        break;
      default: go(inplace_c, std::integral_constant<int, SCALE_KV_UE8M0>{}, idx_c); break;
    }
  };
  if (inplace) {
    if (idx32) with_mode(std::true_type{}, std::true_type{});
    else with_mode(std::true_type{}, std::false_type{});
  } else {
    if (idx32) with_mode(std::false_type{}, std::true_type{});
    else with_mode(std::false_type{}, std::false_type{});
  }
  return check_launch("act_quant");
}

}  // namespace
}  // namespace sgl

extern "C" {

int sgl_act_quant(const void* x, int64_t M, int64_t K, int64_t ldx, void* y, int64_t ldy, void* s,
                  int64_t lds, int group, int scale_mode, int scale_e8m0, int inplace,
                  sgl_stream_t stream) {
  SGL_REQUIRE(M >= 0 && K >= 0, "act_quant: negative shape M=%lld K=%lld", (long long)M,
              (long long)K);
  SGL_REQUIRE(group == 32 || group == 64 || group == 128, "act_quant: group %d not in {32,64,128}",
              group);
  SGL_REQUIRE(K % group == 0, "act_quant: K=%lld not divisible by group %d", (long long)K, group);
  SGL_REQUIRE(scale_mode >= 0 && scale_mode <= 4, "act_quant: bad scale_mode %d", scale_mode);
  SGL_REQUIRE(!scale_e8m0 || scale_mode == SGL_SCALE_TORCH_UE8M0 ||
                  scale_mode == SGL_SCALE_TILELANG_UE8M0 || scale_mode == SGL_SCALE_KV_UE8M0,
              "act_quant: e8m0 scale storage needs a power-of-two scale mode (got %d)", scale_mode);
  if (M == 0 || K == 0) return SGL_OK;
  SGL_REQUIRE(x && y && s, "act_quant: null pointer");
  SGL_REQUIRE(ldx >= K && ldy >= K && lds >= K / group, "act_quant: row stride smaller than row");
  SGL_REQUIRE(sgl::aligned(x, 16) && ldx % 8 == 0, "act_quant: x must be 16-byte aligned rows");
  SGL_REQUIRE(sgl::aligned(y, inplace ? 16 : 8) && ldy % 8 == 0,
              "act_quant: y must be aligned (16 B bf16 / 8 B e4m3) with ldy %% 8 == 0");
  SGL_REQUIRE(scale_e8m0 || sgl::aligned(s, 4), "act_quant: fp32 scales must be 4-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  switch (group) {
    case 32:
      return sgl::launch_act_quant<32>(x, M, K, ldx, y, ldy, s, lds, scale_mode, scale_e8m0,
                                       inplace, st);
    case 64:
      return sgl::launch_act_quant<64>(x, M, K, ldx, y, ldy, s, lds, scale_mode, scale_e8m0,
                                       inplace, st);
    default:
      return sgl::launch_act_quant<128>(x, M, K, ldx, y, ldy, s, lds, scale_mode, scale_e8m0,
                                        inplace, st);
  }
}

int sgl_weight_quant_128x128(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, void* q,
                             int64_t ldq, float* s, int64_t lds, int use_ue8m0,
                             sgl_stream_t stream) {
  SGL_REQUIRE(N >= 0 && K >= 0, "weight_quant: negative shape");
  SGL_REQUIRE(dtype == SGL_F32 || dtype == SGL_BF16, "weight_quant: dtype must be f32 or bf16");
  SGL_REQUIRE(K % 8 == 0, "weight_quant: K=%lld must be a multiple of 8", (long long)K);
  if (N == 0 || K == 0) return SGL_OK;
  SGL_REQUIRE(w && q && s, "weight_quant: null pointer");
  SGL_REQUIRE(ldw >= K && ldq >= K && lds >= sgl::ceil_div(K, 128), "weight_quant: bad strides");
  SGL_REQUIRE(sgl::aligned(w, 16) && ldw % 8 == 0 && sgl::aligned(q, 8) && ldq % 8 == 0,
              "weight_quant: rows must be aligned (w 16 B, q 8 B)");
  dim3 grid((unsigned)sgl::ceil_div(K, 128), (unsigned)sgl::ceil_div(N, 128));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == SGL_F32)
    sgl::weight_quant_kernel<float><<<grid, 256, 0, st>>>((const float*)w, N, K, ldw, (uint8_t*)q,
                                                          ldq, s, lds, use_ue8m0);
  else
    sgl::weight_quant_kernel<uint16_t><<<grid, 256, 0, st>>>(
        (const uint16_t*)w, N, K, ldw, (uint8_t*)q, ldq, s, lds, use_ue8m0);
  return sgl::check_launch("weight_quant_128x128");
}

int sgl_e8m0_to_f32(const void* src, float* dst, int64_t n, sgl_stream_t stream) {
  SGL_REQUIRE(n >= 0, "e8m0_to_f32: negative n");
  if (n == 0) return SGL_OK;
  SGL_REQUIRE(src && dst, "e8m0_to_f32: null pointer");
  int64_t blocks = sgl::ceil_div(n, 256);
  if (blocks > 4096) blocks = 4096;
  sgl::e8m0_to_f32_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>((const uint8_t*)src,
                                                                             dst, n);
  return sgl::check_launch("e8m0_to_f32");
}

int sgl_fp4_to_fp8_weight(const void* b, const void* sb, int64_t N, int64_t K, void* q,
                          void* s_out, sgl_stream_t stream) {
  SGL_REQUIRE(N >= 0 && K >= 0 && N % 128 == 0 && K % 128 == 0,
              "fp4_to_fp8_weight: N=%lld and K=%lld must be multiples of 128", (long long)N,
              (long long)K);
  if (N == 0 || K == 0) return SGL_OK;
  SGL_REQUIRE(b && sb && q && s_out, "fp4_to_fp8_weight: null pointer");
  SGL_REQUIRE(sgl::aligned(b, 16) && sgl::aligned(q, 16), "fp4_to_fp8_weight: b and q must be 16-byte aligned");
  SGL_REQUIRE(N / 128 <= 65535, "fp4_to_fp8_weight: N too large");
  dim3 grid((unsigned)(K / 128), (unsigned)(N / 128));
  sgl::fp4_to_fp8_weight_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)b, (const uint8_t*)sb, K, (uint8_t*)q, (uint8_t*)s_out);
  return sgl::check_launch("fp4_to_fp8_weight");
}

int sgl_check_conversions(unsigned long long* counts, sgl_stream_t stream) {
  SGL_REQUIRE(counts, "check_conversions: null pointer");
  const uint64_t per_launch = 1ull << 28;  // inputs per launch, 4 per thread
  for (uint64_t start = 0; start < (1ull << 32); start += per_launch) {
    sgl::check_conversions_kernel<<<(unsigned)(per_launch / 4 / 256), 256, 0, (hipStream_t)stream>>>(
        start, counts);
    const int rc = sgl::check_launch("check_conversions");
    if (rc != SGL_OK) return rc;
  }
  return SGL_OK;
}

}  // extern "C"
