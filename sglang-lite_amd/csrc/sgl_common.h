// Common plumbing for the C-ABI entry points: status codes, the thread-local
// last-error message and launch checking.  Entry points never throw across
// the ABI; they return a status and leave a message for sgl_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/sglang_lite_amd.h"

namespace sgl {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return SGL_ERR_HIP;
  }
  return SGL_OK;
}

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Device address of the current device's static MoE workspace (moe.hip),
// resolved with hipGetSymbolAddress on the first call for that device.
int moe_scratch_ptr(void** out);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

#ifndef SGL_NT_STREAMS
#define SGL_NT_STREAMS 1
#endif
#if defined(__HIPCC__)
// A 16-byte load with the nontemporal cache policy (nt), for inputs a kernel
// streams through once: a read stream of 2 GiB on gfx950 moves 7.0 TB/s with
// nt loads where plain loads move 6.2.  Only for lines whose bytes one load
// takes whole or whose other pieces follow at once: an nt line is not kept
// for a later reader.
__device__ __forceinline__ uint4 ld16_stream(const void* p) {
  typedef unsigned int u4v_ __attribute__((ext_vector_type(4)));
  const u4v_* q = reinterpret_cast<const u4v_*>(p);
  const u4v_ v = SGL_NT_STREAMS ? __builtin_nontemporal_load(q) : *q;
  return make_uint4(v.x, v.y, v.z, v.w);
}

// LDS byte address of a __shared__ object (what an LDS DMA's m0 takes).
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const uint8_t*)p);
}

// LDS DMA with a per-lane 64-bit address: lane i copies 16 bytes from addr to
// LDS m0 + 16 i (global_load_lds_dwordx4; counted by vmcnt).
__device__ __forceinline__ void dma16v(uint64_t addr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(addr), "s"(lds) : "memory");
}

// Chunk swizzle of the LDS-staged operand tiles: a 128-byte stage row's
// 16-byte chunk c sits at c ^ swz(row).  A ds_read_b128 of an MFMA operand
// has 16 lanes read one chunk column of 16 consecutive rows; with this
// swizzle those reads are conflict-free on gfx950's 64-bank LDS.  swz depends
// on row bits 1-3 only, so it repeats every 16 rows.
__device__ __forceinline__ int swz(int row) { return (row & 6) | ((row >> 3) & 1); }
#endif

}  // namespace sgl

#define SGL_REQUIRE(cond, ...)          \
  do {                                  \
    if (!(cond)) {                      \
      ::sgl::set_error(__VA_ARGS__);    \
      return SGL_ERR_INVALID_ARG;       \
    }                                   \
  } while (0)

#define SGL_REQUIRE_SUPPORTED(cond, ...) \
  do {                                   \
    if (!(cond)) {                       \
      ::sgl::set_error(__VA_ARGS__);     \
      return SGL_ERR_UNSUPPORTED;        \
    }                                    \
  } while (0)

#define SGL_CHECK_HIP(expr)                                                       \
  do {                                                                            \
    hipError_t _e = (expr);                                                       \
    if (_e != hipSuccess) {                                                       \
      ::sgl::set_error("%s failed: %s", #expr, hipGetErrorString(_e));            \
      return SGL_ERR_HIP;                                                         \
    }                                                                             \
  } while (0)
