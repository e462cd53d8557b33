// Library-level entry points: ABI version, last error, device probe and the
// host-compiled copies of the numeric helpers used by the CPU test suite.
#include <string.h>

#include <mutex>

#include "sgl_common.h"
#include "sgl_numeric.h"

namespace sgl {

static thread_local char g_last_error[1024] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int device_cu_count() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

namespace {

// An HBM stream: each of kStreamWgs workgroups moves one contiguous slice
// with 16-byte nontemporal loads (plain stores), four in flight per lane; a
// copy (dst) or a read that leaves the XOR of its slice in sums[workgroup].
constexpr int kStreamWgs = 2048, kStreamThreads = 512;

__global__ __launch_bounds__(kStreamThreads) void hbm_stream_kernel(const uint4* __restrict__ src,
                                                                   uint4* __restrict__ dst, int64_t n16,
                                                                   uint32_t* __restrict__ sums) {
  const int64_t per = n16 / kStreamWgs;
  const uint4* p = src + (int64_t)blockIdx.x * per;
  uint32_t acc = 0;
  for (int64_t base = 0; base < per; base += 4 * kStreamThreads) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + u * kStreamThreads + threadIdx.x;
      v[u] = i < per ? ld16_stream(p + i) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + u * kStreamThreads + threadIdx.x;
      if (dst) {
        if (i < per) dst[(int64_t)blockIdx.x * per + i] = v[u];
      } else {
        acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
      }
    }
  }
  if (!dst) {
    __shared__ uint32_t red[kStreamThreads / 64];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t a = 0;
      for (int w = 0; w < kStreamThreads / 64; ++w) a ^= red[w];
      sums[blockIdx.x] = a;
    }
  }
}

// MFMA rate of the GEMMs' inner-loop instruction mix: each wavefront runs
// `iters` rounds of a 4 x 4 block of v_mfma_f32_16x16x128_f8f6f4 from
// registers (the GEMM wavefront's 64 x 64 tile), either accumulating in the
// MFMA's C operand (variant 0: the power-of-two path) or with each block
// partial promoted by 4 dependent fp32 FMAs one column block behind
// (variant 1: the fp32-scale path).  Operands come from the lane id; the
// sums go to out[thread] so nothing is optimised away.  Two 4-wavefront
// workgroups per CU: two wavefronts per SIMD, as in the GEMMs.
typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));
constexpr int kMixThreads = 256;

template <int V>
__global__ __launch_bounds__(kMixThreads) void mfma_mix_kernel(float* __restrict__ out, int iters) {
  const int lane = threadIdx.x & 63;
  v8i_t a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // e4m3 bytes of small finite values (exponent field below 15)
      a[i][j] = (int)(0x38383838u ^ (uint32_t)((lane * 29 + i * 7 + j) & 0x07070707));
      b[i][j] = (int)(0x30303030u ^ (uint32_t)((lane * 13 + i * 5 + j) & 0x07070707));
    }
  float ss[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ss[i] = 1.0f + (float)((lane + i) & 3) * 0.25f;
  const v4f_t z = {0.0f, 0.0f, 0.0f, 0.0f};
  v4f_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = z;
  for (int it = 0; it < iters; ++it) {
    if constexpr (V == 0) {
#pragma unroll
      for (int nj = 0; nj < 4; ++nj)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
          acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b[nj], a[mi], acc[mi][nj], 0, 0, 0,
                                                                         0, 0, 0);
    } else {
      v4f_t pr[2][4];
#pragma unroll
      for (int nj = 0; nj < 5; ++nj) {
        if (nj < 4) {
#pragma unroll
          for (int mi = 0; mi < 4; ++mi)
            pr[nj & 1][mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b[nj], a[mi], z, 0, 0, 0, 0, 0, 0);
        }
        if (nj >= 1) {
#pragma unroll
          for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[mi][nj - 1][r] = fmaf(pr[(nj - 1) & 1][mi][r], ss[mi], acc[mi][nj - 1][r]);
        }
      }
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += acc[i][j][r];
  out[(int64_t)blockIdx.x * kMixThreads + threadIdx.x] = sum;
}

}  // namespace

}  // namespace sgl

extern "C" {

int sgl_abi_version(void) { return SGL_ABI_VERSION; }

int sgl_hbm_stream(const void* src, void* dst, int64_t bytes, uint32_t* sums, sgl_stream_t stream) {
  SGL_REQUIRE(bytes > 0 && bytes % (16 * (int64_t)sgl::kStreamWgs) == 0,
              "hbm_stream: bytes=%lld must be a positive multiple of %d", (long long)bytes,
              16 * sgl::kStreamWgs);
  SGL_REQUIRE(src && (dst || sums), "hbm_stream: null pointer");
  SGL_REQUIRE(sgl::aligned(src, 16) && (!dst || sgl::aligned(dst, 16)), "hbm_stream: misaligned");
  sgl::hbm_stream_kernel<<<sgl::kStreamWgs, sgl::kStreamThreads, 0, (hipStream_t)stream>>>(
      (const uint4*)src, (uint4*)dst, bytes / 16, sums);
  return sgl::check_launch("hbm_stream");
}

int sgl_mfma_mix(int variant, float* out, int64_t iters, sgl_stream_t stream) {
  SGL_REQUIRE(variant == 0 || variant == 1, "mfma_mix: variant must be 0 or 1");
  SGL_REQUIRE(iters > 0 && iters < (1 << 30), "mfma_mix: iters=%lld out of range", (long long)iters);
  SGL_REQUIRE(out, "mfma_mix: null pointer");
  const unsigned wgs = (unsigned)(2 * sgl::device_cu_count());
  if (variant == 0)
    sgl::mfma_mix_kernel<0><<<wgs, sgl::kMixThreads, 0, (hipStream_t)stream>>>(out, (int)iters);
  else
    sgl::mfma_mix_kernel<1><<<wgs, sgl::kMixThreads, 0, (hipStream_t)stream>>>(out, (int)iters);
  return sgl::check_launch("mfma_mix");
}

int sgl_mfma_mix_threads(void) { return 2 * sgl::device_cu_count() * sgl::kMixThreads; }

const char* sgl_last_error(void) { return sgl::g_last_error; }

int sgl_probe(void) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    sgl::set_error("no HIP device: %s", e != hipSuccess ? hipGetErrorString(e) : "count == 0");
    return 0;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    sgl::set_error("hipGetDevice failed");
    return 0;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    sgl::set_error("hipGetDeviceProperties failed");
    return 0;
  }
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    sgl::set_error("device %d is %s; this library is built for gfx950 only", dev, prop.gcnArchName);
    return 0;
  }
  // set-up: resolve this device's static MoE workspace address now, outside
  // any stream capture
  void* scratch = nullptr;
  if (sgl::moe_scratch_ptr(&scratch) != SGL_OK) return 0;
  return 1;
}

int sgl_host_f32_to_e4m3(const float* x, uint8_t* y, int64_t n) {
  SGL_REQUIRE(x && y && n >= 0, "sgl_host_f32_to_e4m3: bad arguments");
  for (int64_t i = 0; i < n; ++i) y[i] = sgl::f32_to_e4m3(x[i]);
  return SGL_OK;
}

int sgl_host_e4m3_to_f32(const uint8_t* x, float* y, int64_t n) {
  SGL_REQUIRE(x && y && n >= 0, "sgl_host_e4m3_to_f32: bad arguments");
  for (int64_t i = 0; i < n; ++i) y[i] = sgl::e4m3_to_f32(x[i]);
  return SGL_OK;
}

int sgl_host_group_scale(int scale_mode, const float* amax, float* scale, int64_t n) {
  SGL_REQUIRE(amax && scale && n >= 0, "sgl_host_group_scale: bad arguments");
  SGL_REQUIRE(scale_mode >= 0 && scale_mode <= 4, "sgl_host_group_scale: bad scale_mode %d",
              scale_mode);
  for (int64_t i = 0; i < n; ++i) scale[i] = sgl::group_scale(scale_mode, amax[i]);
  return SGL_OK;
}

int sgl_host_quant_elem(int scale_mode, const float* x, const float* scale, uint8_t* y, int64_t n) {
  SGL_REQUIRE(x && scale && y && n >= 0, "sgl_host_quant_elem: bad arguments");
  SGL_REQUIRE(scale_mode >= 0 && scale_mode <= 4, "sgl_host_quant_elem: bad scale_mode %d",
              scale_mode);
  for (int64_t i = 0; i < n; ++i) {
    float sf = scale[i];
    y[i] = sgl::quant_elem(scale_mode, x[i], sf, 1.0f / sf);
  }
  return SGL_OK;
}

}  // extern "C"
