// Scalar number-format helpers shared by the HIP kernels and the host-side
// self-test entry points: OCP e4m3fn, bf16, e8m0 and the scale formulas of the
// DeepSeek-V4 FP8 path.  Everything here is integer/IEEE arithmetic with a
// fixed rounding rule, so the same code gives the same bits on the host and on
// gfx950.
//
// Formats (OCP FP8 spec / IEEE-754):
//   e4m3fn : 1 sign, 4 exponent (bias 7), 3 mantissa bits, no infinities,
//            S.1111.111 is NaN, max finite 448, min subnormal 2^-9.
//   bf16   : upper 16 bits of an IEEE binary32.
//   e8m0   : 8-bit biased exponent (bias 127), value 2^(byte-127).
#pragma once

#include <stdint.h>

#include <type_traits>
#if !defined(__HIPCC__)
#include <math.h>
#endif

#if defined(__HIPCC__)
#define SGL_HD __host__ __device__ __forceinline__
#else
#define SGL_HD inline
#endif

namespace sgl {

SGL_HD uint32_t f32_bits(float x) { return __builtin_bit_cast(uint32_t, x); }
SGL_HD float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// bf16 -> fp32 is exact.
SGL_HD float bf16_to_f32(uint16_t h) { return bits_f32(((uint32_t)h) << 16); }

// fp32 -> bf16, round to nearest even; NaN becomes the quiet NaN 0x7FC0
// (the convention torch uses for its bfloat16 casts).
SGL_HD uint16_t f32_to_bf16(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// fp16 -> fp32 (exact), for KV inputs given as float16.
SGL_HD float f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  if (e == 0x1Fu) return bits_f32(sign | 0x7F800000u | (m << 13));
  if (e != 0) return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
  // subnormal: m * 2^-24, exact in fp32
  float v = (float)m * 5.9604644775390625e-08f;
  return sign ? -v : v;
}

// fp32 -> e4m3fn with round-to-nearest-even on the 3-bit mantissa.
//  * |x| above 464 (the midpoint between 448 and the NaN code) and NaN/Inf
//    map to the NaN code S.1111.111; exactly 464 ties to 448 (even mantissa).
//  * normal range starts at 2^-6; below it the grid is the subnormal step
//    2^-9, rounded to nearest even.
SGL_HD uint8_t f32_to_e4m3(float x) {
  const uint32_t u = f32_bits(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x43E80000u) return (uint8_t)(sign | 0x7Fu);  // > 464, Inf, NaN
  if (a >= 0x3C800000u) {                               // >= 2^-6: normal
    // keep 3 of 23 mantissa bits: add half-ulp-minus-one plus the lsb (RNE)
    uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
    // rebias exponent 127 -> 7: subtract (127-7) << 3
    return (uint8_t)(sign | (uint8_t)(r - (120u << 3)));
  }
  // subnormal / zero: value / 2^-9 rounded to nearest even integer in [0, 8]
  // (8 is the smallest normal, code 0x08).  Scaling by 2^9 is exact here.
  float q = bits_f32(a) * 512.0f;
  // round-half-even of q in [0, 8): integer part + tie handling
  uint32_t iq = (uint32_t)q;              // truncation, q >= 0
  float frac = q - (float)iq;             // exact (q < 8 has spare bits)
  if (frac > 0.5f || (frac == 0.5f && (iq & 1u))) iq += 1u;
  return (uint8_t)(sign | (uint8_t)iq);
}

#if defined(__HIPCC__)
// gfx950 conversion instructions.  v_cvt_pk_fp8_f32 (OCP e4m3fn, round to
// nearest even, out of range -> NaN code) and v_cvt_pk_bf16_f32 (round to
// nearest even) give exactly f32_to_e4m3 / f32_to_bf16 for every non-NaN fp32
// input; sgl_check_conversions re-verifies that over all 2^32 inputs on the
// device.  For NaN inputs the hardware e4m3 code can carry the other sign bit
// and the bf16 result keeps payload bits; the *_exact forms restore the
// software convention (NaN keeps its sign as S.1111.111; bf16 NaN is 0x7FC0).
typedef float sgl_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 sgl_bf2 __attribute__((ext_vector_type(2)));

// bytes {a, b, c, d} as e4m3fn, little-endian
__device__ __forceinline__ uint32_t pk4_e4m3(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}
__device__ __forceinline__ uint32_t pk4_e4m3_exact(float a, float b, float c, float d) {
  const uint32_t signs = ((f32_bits(a) >> 24) & 0x80u) | ((f32_bits(b) >> 16) & 0x8000u) |
                         ((f32_bits(c) >> 8) & 0x800000u) | (f32_bits(d) & 0x80000000u);
  return (pk4_e4m3(a, b, c, d) & 0x7F7F7F7Fu) | signs;
}
// {lo, hi} as bf16, lo in the low half-word
__device__ __forceinline__ uint32_t pk2_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(sgl_f2{lo, hi}, sgl_bf2));
}
__device__ __forceinline__ uint16_t bf16_bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
__device__ __forceinline__ uint16_t bf16_bits_exact(float x) {
  return x != x ? (uint16_t)0x7FC0 : bf16_bits(x);
}
__device__ __forceinline__ uint32_t pk2_bf16_exact(float lo, float hi) {
  return (uint32_t)bf16_bits_exact(lo) | ((uint32_t)bf16_bits_exact(hi) << 16);
}
// four e4m3 bytes (little-endian) -> fp32, exact (v_cvt_pk_f32_fp8); the NaN
// code gives a NaN
__device__ __forceinline__ void unpack4_e4m3(uint32_t w, float* f) {
  const sgl_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const sgl_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  f[0] = lo.x; f[1] = lo.y; f[2] = hi.x; f[3] = hi.y;
}
// fp32 value of the bf16 rounding of x (NaN stays NaN)
__device__ __forceinline__ float bf16_round(float x) { return bits_f32((uint32_t)bf16_bits(x) << 16); }
#endif

// e4m3fn -> fp32 (exact).
SGL_HD float e4m3_to_f32(uint8_t v) {
  const uint32_t sign = ((uint32_t)v & 0x80u) << 24;
  const uint32_t e = (v >> 3) & 0xFu;
  const uint32_t m = v & 0x7u;
  if (e == 0xFu && m == 0x7u) return bits_f32(sign | 0x7FC00000u);
  if (e == 0) {
    float s = (float)m * 0.001953125f;  // m * 2^-9
    return sign ? -s : s;
  }
  return bits_f32(sign | ((e + 120u) << 23) | (m << 20));
}

// ceil(log2(x)) for positive finite normal x from its bits:
// exponent, plus one when any mantissa bit is set.
SGL_HD int ceil_log2_bits(float x) {
  uint32_t u = f32_bits(x);
  int e = (int)((u >> 23) & 0xFFu) - 127;
  return e + ((u & 0x7FFFFFu) != 0u ? 1 : 0);
}

// 2^k as fp32 for k in the normal range [-126, 127].
SGL_HD float pow2_f32(int k) { return bits_f32((uint32_t)(k + 127) << 23); }

// DeepGEMM-style ceil_to_ue8m0: the next power of two >= |x| with the biased
// exponent clamped to [1, 254].
SGL_HD float ceil_to_ue8m0(float x) {
  uint32_t u = f32_bits(x) & 0x7FFFFFFFu;
  int e = (int)((u >> 23) & 0xFFu) + ((u & 0x7FFFFFu) != 0u ? 1 : 0);
  e = e < 1 ? 1 : (e > 254 ? 254 : e);
  return bits_f32((uint32_t)e << 23);
}

// e8m0 byte of an exact power of two (or 0 / NaN code 0xFF by convention).
SGL_HD uint8_t pow2_to_e8m0(float p) { return (uint8_t)((f32_bits(p) >> 23) & 0xFFu); }

// max / clamp that propagate NaN the way torch's amax and clamp do.
SGL_HD float fmaxf_(float a, float b) { return (a > b || a != a) ? a : b; }
SGL_HD float clampf_(float x, float lo, float hi) {
  if (x != x) return x;
  return x < lo ? lo : (x > hi ? hi : x);
}

// Activation-quant scale modes (see the mode table in sglang_lite_amd.h).
enum ScaleMode : int {
  SCALE_TORCH_FP32 = 0,     // sf = max(amax,1e-4)/448 ; q = e4m3(x * (1/sf))
  SCALE_TORCH_UE8M0 = 1,    // sf = ceil_to_ue8m0(max(amax,1e-4)/448) ; q = e4m3(x * (1/sf))
  SCALE_TILELANG_FP32 = 2,  // s = max(amax,1e-4) * (1/448) ; q = e4m3(clamp(x / s, +-448))
  SCALE_TILELANG_UE8M0 = 3, // s = 2^ceil_log2(max(amax,1e-4) * (1/448)) ; q = e4m3(clamp(x / s))
  SCALE_KV_UE8M0 = 4,       // s = 2^ceil(log2(max(max(amax,1e-12)*(1/448), 2^-30))) ; clamp
};

// 1/448 rounded to fp32, the constant the reference multiplies by.
#define SGL_INV448_F32 (1.0f / 448.0f)

// Per-group scale from the group's |x| maximum: the value the reference stores.
SGL_HD float group_scale(int mode, float amax) {
  switch (mode) {
    case SCALE_TORCH_FP32: {
      float a = fmaxf_(amax, 1e-4f);
      return a / 448.0f;
    }
    case SCALE_TORCH_UE8M0: {
      float a = fmaxf_(amax, 1e-4f);
      return ceil_to_ue8m0(a / 448.0f);
    }
    case SCALE_TILELANG_FP32: {
      float a = fmaxf_(amax, 1e-4f);
      return a * SGL_INV448_F32;
    }
    case SCALE_TILELANG_UE8M0: {
      float a = fmaxf_(amax, 1e-4f);
      return pow2_f32(ceil_log2_bits(a * SGL_INV448_F32));
    }
    default: {  // SCALE_KV_UE8M0
      float a = fmaxf_(amax, 1e-12f);
      float raw = fmaxf_(a * SGL_INV448_F32, 9.313225746154785e-10f /* 2^-30 */);
      if (!(raw < 3.0e38f)) return raw;  // Inf / NaN pass through as the scale
      // ceil of the correctly rounded fp32 log2.  For fp32 inputs just above a
      // power of two this is not the exponent+1 of the bit formula: log2 of
      // 2^k(1+tiny) rounds to exactly k.  raw = 2^k (1 + M 2^-23) is normal
      // here (raw >= 2^-30); M == 0 gives k, and M > 64 gives k + 1 for every
      // |k| <= 127 (log2(1 + 65 2^-23) > 2^-17 exceeds half the fp32 spacing
      // at any such k), so only M in [1, 64] needs the double-precision log2,
      // whose rounding to fp32 is the correctly rounded value.
      const uint32_t u = f32_bits(raw);
      const int k = (int)((u >> 23) & 0xFFu) - 127;
      const uint32_t M = u & 0x7FFFFFu;
      if (M == 0u) return pow2_f32(k);
      if (M > 64u) return pow2_f32(k + 1);
      float l = (float)log2((double)raw);
      return pow2_f32((int)ceilf(l));
    }
  }
}

// Quantize one element given the group scale, per mode.
//  torch modes multiply by the correctly rounded reciprocal and do not clamp;
//  the TileLang / KV modes divide and clamp to +-448 before the cast.
SGL_HD uint8_t quant_elem(int mode, float x, float sf, float inv) {
  if (mode == SCALE_TORCH_FP32 || mode == SCALE_TORCH_UE8M0) return f32_to_e4m3(x * inv);
  return f32_to_e4m3(clampf_(x / sf, -448.0f, 448.0f));
}

#if defined(__HIPCC__)
// clampf_(x, -448, 448) in three instructions: the median of three for every
// non-NaN x (the same value, -0 included), x itself for a NaN
__device__ __forceinline__ float clamp448(float x) {
  const float c = __builtin_amdgcn_fmed3f(x, -448.0f, 448.0f);
  return x != x ? x : c;
}
// 1 / sf, equal to the IEEE division, for the ue8m0 modes' scales: a normal
// power of two +-2^k by ldexp (2^-k is exact, 2^-127 a subnormal), +-0 gives
// +-Inf (the TileLang formula makes -0 of a NaN group: 2^(129) wraps into the
// sign bit), +-Inf gives +-0 and a NaN itself (a quiet NaN divisor is the
// quotient); subnormal scales are not produced by any mode
__device__ __forceinline__ float pow2_recip(float sf) {
  const uint32_t u = f32_bits(sf);
  const uint32_t sign = u & 0x80000000u;
  const int e = (int)((u >> 23) & 0xFFu);
  const float r = bits_f32(f32_bits(__builtin_amdgcn_ldexpf(1.0f, 127 - e)) | sign);
  const float special = e == 0 ? bits_f32(sign | 0x7F800000u) : (sf != sf ? sf : bits_f32(sign));
  return (e == 0 || e == 255) ? special : r;
}
// The maximum over aligned groups of LANES (2, 4, 8 or 16) lanes by DPP
// moves, NaN-propagating: after the two quad permutations every lane holds
// its quad's maximum, the half-row mirror (lane i <-> 7 - i) joins the two
// quads of 8 lanes and the row mirror (i <-> 15 - i) the two halves of 16
template <int LANES>
__device__ __forceinline__ float lane_group_max(float v) {
  static_assert(LANES == 2 || LANES == 4 || LANES == 8 || LANES == 16, "2 to 16 lanes");
  auto dpp = [](float x, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x),
                                                              decltype(ctrl)::value, 0xF, 0xF, false));
  };
  using quad_xor1 = std::integral_constant<int, 0xB1>;  // quad_perm [1, 0, 3, 2]
  using quad_xor2 = std::integral_constant<int, 0x4E>;  // quad_perm [2, 3, 0, 1]
  using half_mirror = std::integral_constant<int, 0x141>;
  using row_mirror = std::integral_constant<int, 0x140>;
  v = __builtin_elementwise_maximum(v, dpp(v, quad_xor1{}));
  if constexpr (LANES >= 4) v = __builtin_elementwise_maximum(v, dpp(v, quad_xor2{}));
  if constexpr (LANES >= 8) v = __builtin_elementwise_maximum(v, dpp(v, half_mirror{}));
  if constexpr (LANES >= 16) v = __builtin_elementwise_maximum(v, dpp(v, row_mirror{}));
  return v;
}

// Eight consecutive elements of one group -> e4m3 bytes (little-endian in
// .x then .y), bit-identical to quant_elem for every mode.  ue8m0 scales are
// powers of two (or Inf / NaN), so TileLang-ue8m0 and KV divisions equal the
// product with the exact reciprocal; only TileLang-fp32 divides.
template <int N>
__device__ __forceinline__ void quant_scale(int mode, const float* f, float sf, float* y) {
  if (mode == SCALE_TILELANG_FP32) {
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = clamp448(f[i] / sf);
  } else {
    const bool torch_mode = mode == SCALE_TORCH_FP32 || mode == SCALE_TORCH_UE8M0;
    const float inv = mode == SCALE_TORCH_FP32 ? 1.0f / sf : pow2_recip(sf);
#pragma unroll
    for (int i = 0; i < N; ++i) y[i] = f[i] * inv;
    if (!torch_mode) {
#pragma unroll
      for (int i = 0; i < N; ++i) y[i] = clamp448(y[i]);
    }
  }
}
__device__ __forceinline__ uint2 quant8_e4m3(int mode, const float* f, float sf) {
  float y[8];
  quant_scale<8>(mode, f, sf, y);
  return make_uint2(pk4_e4m3_exact(y[0], y[1], y[2], y[3]), pk4_e4m3_exact(y[4], y[5], y[6], y[7]));
}
// The same arithmetic for four values (four consecutive e4m3 bytes).
__device__ __forceinline__ uint32_t quant4_e4m3(int mode, const float* f, float sf) {
  float y[4];
  quant_scale<4>(mode, f, sf, y);
  return pk4_e4m3_exact(y[0], y[1], y[2], y[3]);
}
#endif

}  // namespace sgl
