// Internal interface between the GEMM kernels (gemm.hip) and the MoE / dense
// entry points.  Not part of the C ABI.
#pragma once

#include "sgl_common.h"

namespace sgl {

enum GemmKind : int { KIND_DENSE = 0, KIND_GATE_UP = 1, KIND_DOWN = 2 };

// Weight formats: e4m3 with one scale per 128 x 128 block (fp32, or e8m0 for
// dense sb_e8m0), or packed e2m1 (low nibble = even K) with one e8m0 scale
// per row and 32-deep K block.
enum WeightFmt : int { WF_FP8 = 0, WF_FP4 = 1 };

// One launch of the block-scaled FP8 GEMM family.
//   dense   : C[M, N] = A[M, K] . B[N, K]^T                       (fp8_gemm)
//   gate_up : rows of the routed slots (+ shared rows), A gathered from the
//             token-major quantized activations, B = w_gate | w_up of the
//             row's expert, SwiGLU epilogue, 1x128 requant into hq / hs.
//   down    : rows as gate_up, A = hq rows, B = w_down, bf16 rows scattered
//             to the token-major output of sgl_moe_down.
struct GemmArgs {
  const uint8_t* a;   // dense: A [M, K]; gate_up: xq [T, K]; down: hq [rows, K]
  const void* sa;     // row scales [*, K/128]: fp32, or e8m0 bytes (dense, sa_e8m0)
  const uint8_t* b;   // dense only: B [N, K]
  const void* sb;     // dense only: fp8 [ceil(N/128), K/128]; fp4 e8m0 [N, K/32]
  int sb_e8m0;
  int sa_e8m0;        // dense only: sa holds e8m0 bytes (DMA'd as bytes, widened in LDS)
  int wfmt;           // WeightFmt of B (moe: of every expert in the launch)
  int sa_pow2;        // activation scales are powers of two: applied inside the MFMA
  int sb_pow2;        // fp8 weight scales (fp32) are powers of two: with sa_pow2, both
                      // scales go into the MFMA and no fp32 promotion runs
  const sgl_expert_ptrs* experts;  // moe: device array [E (+1)]
  const sgl_expert_ptrs* frag;     // moe (or null): the same experts with their weights (and
                                   // FP4 scales) in the MFMA fragment layout
                                   // (sgl_fp8_weight_to_frag, sgl_fp4_weight_to_frag)
  const int32_t* offsets;          // moe: [E + 1]
  const int32_t* sorted_slot;      // moe: [T * k]
  const float* route_w;            // gate_up: [T * k] slot-indexed (may be null)
  int E, k, has_shared;  // has_shared: the launch includes the shared expert's rows
  int out_k;             // down: output rows per token (k + the layer's shared expert)
  int64_t T;
  int64_t M, N, K;  // dense: M x N x K; gate_up: N = I, K = H; down: N = H, K = I (logical K)
  void* c;          // dense: [M, N]; down: [T * (k + has_shared), N]
  int out_f32;      // dense output fp32 instead of bf16
  uint8_t* hq;      // gate_up: [rows, N] e4m3
  float* hs;        // gate_up: [rows, N/128]
  float swiglu_limit;
  int scale_mode;
  int m_tiles;      // grid rows (upper bound of M tiles)
  int n_tiles;      // tiles along N
  int* tile_ctr;    // moe: 8 zeroed per-XCD tile counters -> dynamic tile order (null: static)
  void* ws;         // dense: the caller's workspace (split-K partials), or null
  size_t ws_bytes;
  // split-K over the [gate | up] weights of one expert record (device memory,
  // read by the kernel; the shared gate/up of an FP4 layer): columns [0,
  // n_split) are w_gate / s_gate, [n_split, N) w_up / s_up at column - n_split
  const sgl_expert_ptrs* bsrc;
  int64_t n_split;
};

int launch_gemm(int kind, GemmArgs& args, int64_t rows_hint, hipStream_t stream);

// Bytes of workspace the dense FP8 GEMM of this shape uses (its split-K
// partials; 0 when the shape does not split).  A function of the shape only.
size_t dense_fp8_workspace_bytes(int64_t M, int64_t N, int64_t K);

// The FP8 shared expert's gate/up in an FP4 layer at decode sizes (T <= 128),
// split over K so that about one workgroup per CU streams its weights: the
// fp32 partials of [gate | up] go to `part` (at most part_bytes), then the
// split-ordered sum, SwiGLU and 1x128 requant write hq / hs rows from
// *shared_base (offsets[E], read on the device).  `sh` is the shared launch's
// arguments (experts[E], xq / xs, scale mode, SwiGLU limit).  Returns
// kSharedNoSplit when the shape or the space does not split.
constexpr int kSharedNoSplit = 1;
int launch_shared_gate_up_split(const GemmArgs& sh, void* part, size_t part_bytes,
                                const int32_t* shared_base, hipStream_t stream);

}  // namespace sgl
