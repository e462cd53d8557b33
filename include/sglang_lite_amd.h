/*
 * sglang_lite_amd.h -- C ABI of the MI355X (gfx950) FP8 MoE expert path and
 * FP8 KV pack of DeepSeek-V4-Flash.
 *
 * Every entry point:
 *   - takes raw device pointers, int64 sizes/strides (in elements unless a
 *     name ends in _bytes) and the HIP stream to launch on as the last
 *     argument (NULL = the null stream);
 *   - never allocates, frees or keeps a pointer after it returns; outputs and
 *     workspaces are allocated by the caller;
 *   - returns SGL_OK (0) or a negative sgl_status and never throws; the
 *     message of the last failure on the calling thread is sgl_last_error();
 *   - launches asynchronously and never reads routing data on the host, so a
 *     whole MoE layer can be captured into a HIP graph.
 *
 * Each declaration names the reference (ParaTensor/sglang-lite) interface it
 * replaces as file:line.
 */
#ifndef SGLANG_LITE_AMD_H_
#define SGLANG_LITE_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGL_ABI_VERSION 3

typedef void* sgl_stream_t; /* hipStream_t */

enum sgl_status {
  SGL_OK = 0,
  SGL_ERR_INVALID_ARG = -1, /* shape / stride / alignment / dtype the caller got wrong */
  SGL_ERR_UNSUPPORTED = -2, /* valid request this build does not implement */
  SGL_ERR_HIP = -3,         /* HIP runtime or launch failure */
  SGL_ERR_WORKSPACE = -4    /* workspace too small */
};

/* Element dtypes of floating inputs / outputs. */
enum sgl_dtype { SGL_BF16 = 0, SGL_F16 = 1, SGL_F32 = 2 };

/*
 * 1xG activation scale formulas.  amax is the group's max |x| in fp32.
 *   SGL_SCALE_TORCH_FP32   sf = max(amax,1e-4) / 448;  q = e4m3(x * (1/sf))
 *       deep_gemm_sm120/utils/math.py:25-37 per_token_cast_to_fp8(use_ue8m0=False)
 *   SGL_SCALE_TORCH_UE8M0  sf = ceil_to_ue8m0(max(amax,1e-4) / 448);  q as above
 *       deep_gemm_sm120/utils/math.py:13-16,25-37 (use_ue8m0=True)
 *   SGL_SCALE_TILELANG_FP32 s = max(amax,1e-4) * fp32(1/448);  q = e4m3(clamp(x / s, +-448))
 *       deepseek_infer/kernel.py:79,83,93-96 (round_scale=False)
 *   SGL_SCALE_TILELANG_UE8M0 s = 2^ceil_log2(max(amax,1e-4) * fp32(1/448)); q as above
 *       deepseek_infer/kernel.py:22-37,79-81,93-96 (round_scale=True)
 *   SGL_SCALE_KV_UE8M0     s = 2^ceil(log2(max(max(amax,1e-12)*(1/448), 2^-30))); q as above
 *       engine/dsv4_kv_pack.py:78-101 _torch_fp8_ue8m0_quant
 * e4m3 is OCP e4m3fn with round-to-nearest-even (torch's float8_e4m3fn cast).
 */
enum sgl_scale_mode {
  SGL_SCALE_TORCH_FP32 = 0,
  SGL_SCALE_TORCH_UE8M0 = 1,
  SGL_SCALE_TILELANG_FP32 = 2,
  SGL_SCALE_TILELANG_UE8M0 = 3,
  SGL_SCALE_KV_UE8M0 = 4
};

/* Router score functions: deepseek_infer/model.py:566-571. */
enum sgl_score_func { SGL_SCORE_SOFTMAX = 0, SGL_SCORE_SIGMOID = 1, SGL_SCORE_SQRTSOFTPLUS = 2 };

/* KV row layouts.
 *   SGL_KV_LAYOUT_A  engine/dsv4_kv_pack.py:3-37: 512-dim row = 448 NoPE dims as
 *                    e4m3 in blocks of 64 + 64 RoPE dims bf16; 584 B per row:
 *                    [0:448) e4m3 | [448:576) rope bf16 | [576:583) 7 x e8m0 | [583] 0.
 *   SGL_KV_LAYOUT_B  576-dim row = 512-dim latent as e4m3 with 4 fp32 per-128
 *                    scales (SGL_SCALE_TORCH_FP32) + 64 RoPE dims bf16; 656 B per row:
 *                    [0:512) e4m3 | [512:640) rope bf16 | [640:656) 4 x fp32 LE. */
enum sgl_kv_layout { SGL_KV_LAYOUT_A = 0, SGL_KV_LAYOUT_B = 1 };

/* Weight formats of the routed experts of a MoE layer.
 *   SGL_EXPERT_FP8_BLOCK128  e4m3 row-major [out, in] with fp32 scales
 *       [ceil(out/128), ceil(in/128)] (deepseek_infer/model.py:138-142 FP8 Linear)
 *   SGL_EXPERT_FP4_E2M1      packed e2m1 [out, in/2] (byte b of a row holds
 *       element 2b in its low nibble, 2b+1 in its high nibble; torch
 *       float4_e2m1fn_x2) with e8m0 scales [out, in/32], one per 32
 *       consecutive inputs (deepseek_infer/model.py:129-137 FP4 Linear,
 *       expert_dtype "fp4", model.py:623-624)
 * The shared expert is always SGL_EXPERT_FP8_BLOCK128 (model.py:626). */
enum sgl_expert_format { SGL_EXPERT_FP8_BLOCK128 = 0, SGL_EXPERT_FP4_E2M1 = 1 };
/* Flag OR'ed into expert_format: every FP8 block scale of the layer (the FP8
 * routed experts' and the shared expert's) is a power of two, as the
 * float8_e8m0fnu scales of deepseek_infer/model.py:138-142 are once decoded by
 * sgl_e8m0_to_f32 (the cast engine/v4_deep_gemm.py:136-141 makes before its
 * GEMMs).  Their mantissa bits are then ignored.  With a power-of-two
 * scale_mode (*_UE8M0) both scales of each FP8 product are applied as e8m0
 * exponents inside the MFMA, which accumulates across K blocks in place (no
 * fp32 promotion per 128-deep block). */
#define SGL_EXPERT_POW2_SCALES 2
/* Flag OR'ed into expert_format: the experts array holds, after its E routed
 * (+ shared) records, as many records again for the same experts whose FP8
 * weight pointers (w_gate, w_up, w_down) address copies in the MFMA fragment
 * layout written by sgl_fp8_weight_to_frag (scale pointers as in the first
 * set); for FP4 routed experts the weight and the scale pointers address the
 * copies sgl_fp4_weight_to_frag writes.  The grouped GEMMs (K a multiple of
 * 512, 2048 <= K <= 8192) then load those weights straight into registers;
 * every other kernel reads the row-major first set.  No counterpart in the
 * reference: a layout of this build, costing a second copy of the expert
 * weights. */
#define SGL_EXPERT_FRAG_COPY 4

/* Per-expert weight pointers of one MoE layer, stored in DEVICE memory as an
 * array of E routed experts followed by the shared expert; weights and
 * scales in the expert's sgl_expert_format. */
typedef struct sgl_expert_ptrs {
  const void* w_gate; /* w1: [I, H] (fp4: [I, H/2]) */
  const void* w_up;   /* w3: [I, H] (fp4: [I, H/2]) */
  const void* w_down; /* w2: [H, I] (fp4: [H, I/2]) */
  const void* s_gate; /* fp32 [I/128, H/128] (fp4: e8m0 [I, H/32]) */
  const void* s_up;   /* fp32 [I/128, H/128] (fp4: e8m0 [I, H/32]) */
  const void* s_down; /* fp32 [H/128, I/128] (fp4: e8m0 [H, I/32]) */
} sgl_expert_ptrs;

/* ---------------------------------------------------------------- library */

int sgl_abi_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* sgl_last_error(void);
/* 1 when a gfx950 device is current and the kernels are loadable, else 0
 * (and sgl_last_error() says why).  Mirrors the probe of
 * engine/v4_deep_gemm.py:97-133 probe_deep_gemm_sm120. */
int sgl_probe(void);

/* ------------------------------------------------------ activation quant */

/* Per-row 1 x group quantization of bf16 x [M, K] (K % group == 0,
 * group in {32, 64, 128}).
 * Replaces deepseek_infer/kernel.py:105-125 act_quant (and its TileLang
 * kernel :40-102), deep_gemm_sm120/utils/math.py:25-37 per_token_cast_to_fp8.
 *   y : e4m3 [M, K] with row stride ldy          (inplace == 0)
 *       bf16 [M, K] quant-dequant of x, may alias x (inplace == 1; kernel.py:84-91)
 *   s : scales [M, K/group] with row stride lds; fp32, or one e8m0 byte each
 *       when scale_e8m0 != 0 (scale_dtype == torch.float8_e8m0fnu).
 * Pointers must be 16-byte aligned and ldx, ldy multiples of 8. */
int sgl_act_quant(const void* x, int64_t M, int64_t K, int64_t ldx, void* y, int64_t ldy,
                  void* s, int64_t lds, int group, int scale_mode, int scale_e8m0, int inplace,
                  sgl_stream_t stream);

/* 128 x 128 block quantization of a weight w [N, K] (fp32 or bf16, row stride
 * ldw) into e4m3 q [N, K] (row stride ldq) and fp32 scales s [ceil(N/128),
 * ceil(K/128)] (row stride lds); ragged edge blocks behave as zero-padded.
 * Replaces deep_gemm_sm120/utils/math.py:50-60 per_block_cast_to_fp8. */
int sgl_weight_quant_128x128(const void* w, int dtype, int64_t N, int64_t K, int64_t ldw, void* q,
                             int64_t ldq, float* s, int64_t lds, int use_ue8m0,
                             sgl_stream_t stream);

/* e8m0 bytes -> fp32 powers of two (n elements).  Replaces the scale cast of
 * engine/v4_deep_gemm.py:136-141 scale_to_f32. */
int sgl_e8m0_to_f32(const void* src, float* dst, int64_t n, sgl_stream_t stream);

/* Device self-test; no counterpart in the reference.  The kernels convert
 * fp32 to e4m3fn and bf16 with gfx950's v_cvt_pk_fp8_f32 / v_cvt_pk_bf16_f32
 * plus a NaN fix-up, and e4m3 to fp32 with v_cvt_pk_f32_fp8; this compares
 * those conversions with the bit-level
 * software rules (round to nearest even, |x| > 464 -> NaN code, NaN keeps its
 * sign; bf16 NaN -> 0x7FC0) for all 2^32 fp32 inputs and adds the mismatch
 * counts to counts[5] (device memory, zeroed by the caller):
 *   [0] e4m3 with fix-up, all inputs   [1] bf16 with fix-up, all inputs
 *   [2] raw e4m3, non-NaN inputs       [3] raw bf16, non-NaN inputs
 *   [4] e4m3 -> fp32 (v_cvt_pk_f32_fp8) over the 256 codes
 * All five must stay 0. */
int sgl_check_conversions(unsigned long long* counts, sgl_stream_t stream);

/* Measurement aid; no counterpart in the reference.  A plain HBM stream over
 * `bytes` (a positive multiple of 32768) from src with 16-byte accesses: a
 * copy into dst, or, with dst NULL, a read whose XOR per 1/2048 slice goes to
 * sums[2048].  The rate it reaches is the achievable bandwidth the kernels'
 * HBM fractions are read against (the 8 TB/s nominal is not reachable). */
int sgl_hbm_stream(const void* src, void* dst, int64_t bytes, uint32_t* sums, sgl_stream_t stream);

/* Measurement aid; no counterpart in the reference.  The MFMA rate of the
 * FP8 GEMMs' inner-loop instruction mix on all CUs, two wavefronts per SIMD:
 * each wavefront runs `iters` rounds of a 4 x 4 block of 16x16x128 FP8 MFMAs
 * (65536 FLOP each) from registers, accumulating in the MFMA (variant 0: the
 * power-of-two-scale path) or promoting each block partial with 4 fp32 FMAs
 * (variant 1: the fp32-scale path).  out receives one float per thread,
 * sgl_mfma_mix_threads() of them.  The rate is the ceiling the GEMMs' MFMA
 * fractions are read against beside the 5.0 PF/s nominal. */
int sgl_mfma_mix(int variant, float* out, int64_t iters, sgl_stream_t stream);
int sgl_mfma_mix_threads(void);

/* --------------------------------------------------------------- GEMMs */

/* C[M, N] = sum_kb (A[:, kb] . B[:, kb]^T) * sa[m, kb] * sb[n/128, kb], fp32
 * accumulation promoted once per 128-deep K block, output bf16 (out_dtype
 * SGL_BF16) or fp32 (SGL_F32).  A e4m3 [M, K] contiguous, sa [M, K/128] fp32,
 * or one e8m0 byte per scale when a_scale_e8m0 is set (the reference's
 * ue8m0 act_quant output, read as it is), B e4m3 [N, K] contiguous, sb
 * [ceil(N/128), K/128] fp32, or one e8m0 byte per scale when b_scale_e8m0 is
 * set.  K % 128 == 0, N % 16 == 0, M*K and N*K < 2^31.
 * Shapes for which sgl_fp8_gemm_workspace_size is non-zero (16 < M <= 64
 * with N % 128 == 0) split the K range over workgroups and keep the fp32
 * partials in the caller's workspace (16-byte aligned, at least that many
 * bytes; a smaller one is SGL_ERR_WORKSPACE).  Whether a shape splits
 * depends on the shape alone, so eager and graph-captured calls sum in the
 * same order.  Calls that overlap in time need workspaces of their own.
 * Replaces deepseek_infer/kernel.py:257-273 fp8_gemm (kernel :203-254) and the
 * call-site adapter engine/v4_deep_gemm.py:169-218 fp4_gemm_nt (whose
 * workspace-free call the reference's adapter allocates with torch at
 * :186-188, as the caller does here). */
int sgl_fp8_gemm(const void* a, const void* sa, int a_scale_e8m0, const void* b, const void* sb,
                 int b_scale_e8m0, void* c, int out_dtype, int64_t M, int64_t N, int64_t K,
                 void* workspace, size_t workspace_bytes, sgl_stream_t stream);

/* Workspace bytes sgl_fp8_gemm needs for an M x N x K product (0: none). */
size_t sgl_fp8_gemm_workspace_size(int64_t M, int64_t N, int64_t K);

/* Formats of the activation (row) scales of sgl_fp4_gemm. */
#define SGL_ASCALE_F32 0      /* fp32, any value: each 128-deep partial promoted in fp32 */
#define SGL_ASCALE_F32_POW2 1 /* fp32 powers of two (mantissa bits ignored): in the MFMA */
#define SGL_ASCALE_E8M0 2     /* one e8m0 byte per scale: in the MFMA */

/* C[M, N] = A_e4m3[M, K] . B_e2m1[N, K]^T with A scaled per (row, 128-deep K
 * block) by sa and B per (row, 32-deep K block) by sb; fp32 accumulation,
 * output bf16 (SGL_BF16) or fp32 (SGL_F32).  A e4m3 [M, K] contiguous, sa
 * [M, K/128] in the SGL_ASCALE_* format sa_format, B packed e2m1 [N, K/2]
 * (low nibble = even K), sb e8m0 [N, K/32].  The weight scales are applied
 * inside the MFMA; the row scales too unless sa_format is SGL_ASCALE_F32.
 * K % 256 == 0, N % 16 == 0, M*K and N*K/2 < 2^31.
 * Replaces deepseek_infer/kernel.py:519-536 fp4_gemm (kernel :441-516) and
 * engine/v4_deep_gemm.py:169-218 fp4_gemm_nt (DeepGEMM fp8_fp4_gemm_nt). */
int sgl_fp4_gemm(const void* a, const void* sa, int sa_format, const void* b, const void* sb,
                 void* c, int out_dtype, int64_t M, int64_t N, int64_t K, sgl_stream_t stream);

/* Lossless FP4 -> FP8 weight repack: per 128 x 128 block, s = (max of the
 * block's 512 e8m0 scales) / 2^6 and q = e4m3(e2m1 * (scale / s)).  b packed
 * e2m1 [N, K/2], sb e8m0 [N, K/32]; q e4m3 [N, K], s_out e8m0 [N/128, K/128].
 * N % 128 == 0, K % 128 == 0.  Replaces deepseek_infer/convert.py:17-52
 * cast_e2m1fn_to_e4m3fn (the convert.py --expert-dtype fp8 load step). */
int sgl_fp4_to_fp8_weight(const void* b, const void* sb, int64_t N, int64_t K, void* q,
                          void* s_out, sgl_stream_t stream);

/* e4m3 weight [N, K] row-major -> the MFMA fragment layout that
 * SGL_EXPERT_FRAG_COPY records point at: one 2 KB block per (16-row block
 * n16, 128-deep block kb), at block index n16 * (K/128) + kb; byte
 * j * 1024 + 16 l + b of a block holds w[16 n16 + l % 16][128 kb + 32 (l/16)
 * + 16 j + b] (l < 64, j < 2, b < 16).  out: N * K bytes, not aliasing w.
 * N % 16 == 0, K % 128 == 0.  No counterpart in the reference (a one-time
 * weight layout step of this build, run when the expert table is made). */
int sgl_fp8_weight_to_frag(const void* w, int64_t N, int64_t K, void* out, sgl_stream_t stream);

/* Packed e2m1 weight [N, K/2] (low nibble = even K) with e8m0 scales
 * [N, K/32] -> the FP4 fragment layout of SGL_EXPERT_FRAG_COPY records:
 * out_w (N * K/2 bytes) one 1 KB block per (16-row block n16, 128-deep
 * block kb), at n16 * (K/128) + kb, byte 16 l + b holding packed byte
 * 64 kb + 16 (l/16) + b of row 16 n16 + l % 16; out_s (N * K/32 bytes) one
 * 256-byte block per (n16, group q of four 128-deep blocks), at
 * n16 * (K/512) + q, byte 4 l + j holding the scale of row 16 n16 + l % 16
 * for its 32-deep block 16 q + 4 j + l/16.  N % 16 == 0, K % 512 == 0; the
 * outputs do not alias the inputs.  No counterpart in the reference (a
 * one-time weight layout step of this build). */
int sgl_fp4_weight_to_frag(const void* w, const void* s, int64_t N, int64_t K, void* out_w,
                           void* out_s, sgl_stream_t stream);

/* ------------------------------------------------------------ MoE layer */

/* Gate top-k from router logits [T, E] fp32 (E <= 512, k <= 16):
 * scores = score_func(logits); selection on scores + bias (bias may be NULL);
 * weights = scores gathered, renormalised unless softmax, times route_scale.
 * ids int32 [T, k] in descending selection-score order (torch.topk order),
 * weights fp32 [T, k].  Replaces deepseek_infer/model.py:565-584 Gate.forward
 * after its router projection. */
int sgl_moe_route_topk(const float* logits, int64_t T, int E, int k, int score_func,
                       const float* bias, float route_scale, int32_t* ids, float* weights,
                       sgl_stream_t stream);

/* The whole gate of a MoE layer from the hidden states: router projection
 * logits[t, e] = sum_h x[t, h] * W[e, h] (bf16 x [T, H] and bf16 W [E, H], every
 * product exact, fp32 accumulation; logits fp32 [T, E] is written, the caller's
 * buffer), then the selection of sgl_moe_route_topk, or with tid2eid non-NULL
 * the hash routing ids[t] = tid2eid[input_ids[t]] (tid2eid int32 [vocab, k],
 * input_ids int32 or int64 [T]; ids outside [0, vocab) and table entries outside
 * [0, E) are clamped, where torch would raise) with weights = the scores at
 * those experts, renormalised unless softmax, times route_scale; bias is
 * ignored for hash routing.  H % 32 == 0, E <= 512.
 * Replaces deepseek_infer/model.py:564-584 Gate.forward (projection, score
 * function, bias, top-k or tid2eid lookup, renormalisation, route_scale). */
int sgl_moe_gate(const void* x, const void* w, int64_t T, int64_t H, int E, int k, int score_func,
                 const float* bias, float route_scale, const int32_t* tid2eid, int64_t vocab,
                 const void* input_ids, int input_ids_int64, float* logits, int32_t* ids,
                 float* weights, sgl_stream_t stream);

/* Stable counting sort of the T*k routing slots (slot = t*k + j) by expert id:
 *   counts [E], offsets [E+1] (exclusive prefix sum, offsets[E] = T*k),
 *   sorted_slot [T*k] (slot at each sorted position, token-ascending inside an
 *   expert), slot_pos [T*k] (inverse permutation).
 * Ids outside [0, E) are an error reported through counts (they are skipped
 * and not placed).  Replaces the bincount / torch.where dispatch of
 * deepseek_infer/model.py:634-640 and engine/v4_moe_fast.py:89-101. */
int sgl_moe_permute(const int32_t* ids, int64_t T, int k, int E, int32_t* counts, int32_t* offsets,
                    int32_t* sorted_slot, int32_t* slot_pos, sgl_stream_t stream);

/* Grouped gate/up GEMM with the fused SwiGLU epilogue of one MoE layer.
 * Rows are the routed slots in sorted order (row p reads token
 * sorted_slot[p]/k of xq) followed, when has_shared, by T rows of the shared
 * expert (row offsets[E]+t reads token t, weight 1).  For each row:
 *   gate = bf16(A . w_gate^T), up = bf16(A . w_up^T)   (block-scaled FP8 GEMMs)
 *   if swiglu_limit > 0: up = clamp(up, +-lim), gate = min(gate, lim)
 *   h = bf16(silu(gate) * up * route_w[slot])
 *   hq, hs = 1x128 quant of h with scale_mode (fp32 scales)
 * xq e4m3 [T, H], xs fp32 [T, H/128], route_w fp32 [T*k] (slot-indexed),
 * experts: device array of E (+1) sgl_expert_ptrs, the routed ones in
 * expert_format (sgl_expert_format), hq e4m3 [rows, I], hs fp32 [rows, I/128],
 * rows = T*k (+ T).  H % 128 == 0, I % 128 == 0 (FP4: multiples of 256).
 * With FP4 routed experts and a power-of-two scale_mode (*_UE8M0) the row
 * scales xs must be powers of two (as act_quant makes them in that mode):
 * they are applied as e8m0 exponents inside the MFMA.
 * Replaces engine/v4_moe_fast.py:43-76 _expert_forward_fused up to w2's
 * act_quant (and deepseek_infer/model.py:596-606 Expert.forward). */
int sgl_moe_gate_up(const void* xq, const float* xs, int64_t T, int64_t H, int64_t I, int E, int k,
                    const int32_t* offsets, const int32_t* sorted_slot, const float* route_w,
                    const sgl_expert_ptrs* experts, int has_shared, int expert_format,
                    float swiglu_limit, int scale_mode, void* hq, float* hs, sgl_stream_t stream);

/* Grouped down GEMM: out[slot] = bf16(hq[row] . w_down[e]^T) for every row of
 * sgl_moe_gate_up's row order; routed row p is written at output row
 * sorted_slot[p] / k * (k + has_shared) + sorted_slot[p] % k and shared row t
 * at t * (k + 1) + k, so the outputs of one token are contiguous.
 * out bf16 [T * (k + has_shared), H].  expert_format and scale_mode (the
 * mode hs was made with) as for sgl_moe_gate_up.  Replaces the w2 projection
 * of engine/v4_moe_fast.py:76 / deepseek_infer/model.py:606. */
int sgl_moe_down(const void* hq, const float* hs, int64_t T, int64_t H, int64_t I, int E, int k,
                 const int32_t* offsets, const int32_t* sorted_slot,
                 const sgl_expert_ptrs* experts, int has_shared, int expert_format, int scale_mode,
                 void* out, sgl_stream_t stream);

/* Unpermute-combine: y[t] = bf16( (sum over the token's k expert outputs in
 * ascending expert-id order, fp32) + shared[t] ), matching the fp32
 * accumulation order of engine/v4_moe_fast.py:86-106 (and
 * deepseek_infer/model.py:633-644).  out as written by sgl_moe_down,
 * ids int32 [T, k], y bf16 [T, H]. */
int sgl_moe_combine(const void* out, const int32_t* ids, int64_t T, int k, int64_t H,
                    int has_shared, void* y, sgl_stream_t stream);

/* Bytes of workspace sgl_moe_forward needs (256-byte aligned sub-buffers). */
size_t sgl_moe_workspace_size(int64_t T, int64_t H, int64_t I, int E, int k, int has_shared);

/* Whole routed+shared MoE layer from bf16 x [T, H] and a precomputed top-k
 * (ids int32 [T, k], weights fp32 [T, k]): act quant -> permute -> gate/up
 * -> down -> combine, y bf16 [T, H]; routed experts in expert_format.
 * Replaces engine/v4_moe_fast.py:79-106 _moe_forward_activated_only after
 * the gate.  Every launch goes to `stream`. */
int sgl_moe_forward(const void* x, int64_t T, int64_t H, int64_t I, int E, int k,
                    const int32_t* ids, const float* weights, const sgl_expert_ptrs* experts,
                    int has_shared, int expert_format, float swiglu_limit, int scale_mode,
                    void* workspace, size_t workspace_bytes, void* y, sgl_stream_t stream);

/* One rank's share of an expert-sharded MoE layer (the expert split of
 * deepseek_infer/model.py:616-625: the rank holds the routed experts
 * [expert_begin, expert_end) and sees every token).  act quant -> permute of
 * the slots routed to a local expert -> gate/up -> down, then
 *   y_local fp32 [T, H] = sum over the token's routed experts inside the
 *   range, in ascending expert id and fp32, of their bf16 outputs (0 for a
 *   token with none), the shared expert left out.
 * Records of experts outside the range are never read (they may hold null
 * pointers).  With has_shared the shared expert's rows run in the same
 * launches and stay in the workspace for sgl_moe_add_shared.  Workspace as
 * for sgl_moe_forward.  Replaces engine/v4_moe_fast.py:79-102
 * _moe_forward_activated_only up to its all_reduce (the range test :93-97)
 * and deepseek_infer/model.py:629-640. */
int sgl_moe_forward_local(const void* x, int64_t T, int64_t H, int64_t I, int E, int k,
                          const int32_t* ids, const float* weights, const sgl_expert_ptrs* experts,
                          int expert_begin, int expert_end, int has_shared, int expert_format,
                          float swiglu_limit, int scale_mode, void* workspace,
                          size_t workspace_bytes, float* y_local, sgl_stream_t stream);

/* y bf16 [T, H] = bf16(y_local + the shared expert's row), an fp32 addition,
 * where y_local is the caller's all-reduced sum of the ranks'
 * sgl_moe_forward_local outputs and workspace the one this rank's
 * sgl_moe_forward_local call (same T, H, I, E, k, has_shared set) filled.
 * y may alias nothing the call reads.  Replaces engine/v4_moe_fast.py:103-106
 * and deepseek_infer/model.py:641-644 (y += shared_experts(x); y.type_as(x)). */
int sgl_moe_add_shared(const float* y_local, const void* workspace, size_t workspace_bytes,
                       int64_t T, int64_t H, int64_t I, int E, int k, void* y,
                       sgl_stream_t stream);

/* Size of the static device workspace of sgl_moe_forward_noalloc: 64 MiB
 * per GPU, held from library load to process end (T <= 690 tokens at hidden
 * 4096, intermediate 2048, top-8 + shared). */
#define SGL_MOE_SCRATCH_BYTES (64u << 20)

/* sgl_moe_forward without a workspace argument and without any allocation:
 * the layer's workspace is a static device array of SGL_MOE_SCRATCH_BYTES
 * per GPU (its address resolved once per device, by sgl_probe or on the
 * first call).  No counterpart in the reference: for callers that cannot
 * allocate device memory (HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Returns SGL_ERR_WORKSPACE when
 * sgl_moe_workspace_size(T, ...) exceeds SGL_MOE_SCRATCH_BYTES.  Every call
 * on one GPU shares that GPU's array, which keeps the last call's contents:
 * calls that overlap on one GPU (concurrent streams, threads) race. */
int sgl_moe_forward_noalloc(const void* x, int64_t T, int64_t H, int64_t I, int E, int k,
                            const int32_t* ids, const float* weights,
                            const sgl_expert_ptrs* experts, int has_shared, int expert_format,
                            float swiglu_limit, int scale_mode, void* y, sgl_stream_t stream);

/* ------------------------------------------------------------- KV cache */

/* Pack KV rows.  Layout A: kv [T, 512] (bf16 / f16 / f32, row stride ldkv)
 * with scale_mode SGL_SCALE_KV_UE8M0 (the torch fallback,
 * dsv4_kv_pack.py:78-101), SGL_SCALE_TILELANG_UE8M0 (the official TileLang
 * act_quant injected, dsv4_kv_pack.py:58-61) or SGL_SCALE_TORCH_UE8M0 (this
 * library's act_quant with its default torch formula injected), out [T, 584]
 * uint8; with paged != 0 the
 * output is the footer-paged [ceil(T/page)*page*584] bytes of to_paged_hnd,
 * zero-filled padding rows included.  Layout B: kv [T, 576], out [T, 656]
 * (scale_mode ignored: SGL_SCALE_TORCH_FP32), paged must be 0.
 * Replaces engine/dsv4_kv_pack.py:40-75 pack_dsv4_kv_bf16 (+ :104-146). */
int sgl_kv_pack(const void* kv, int dtype, int64_t T, int64_t ldkv, int layout, int scale_mode,
                int paged, int page_size, void* out, sgl_stream_t stream);

/* Packed-page writer: layout A rows of kv [T, 512] (bf16 / f16, row stride
 * ldkv; scale_mode as for sgl_kv_pack) written straight into a RadixCache
 * packed pool uint8 [num_layers, num_blocks, 1, page_size, 584]: token
 * position p = start_pos + t goes to block block_table[p / page_size] (device
 * int32 [n_pages]), slot p % page_size, of layer layer_idx.  A block table
 * shorter than the span is an error (as in the reference); table entries
 * outside [0, num_blocks) are skipped (the reference raises on them; the
 * kernel cannot).  Replaces engine/kv_cache.py:340-390 write_packed_kv fed by
 * engine/dsv4_kv_pack.py:40-75 (the write of engine/v4_dual_pool.py:73-128). */
int sgl_kv_pack_to_pages(const void* kv, int dtype, int64_t T, int64_t ldkv, int scale_mode,
                         const int32_t* block_table, int64_t n_pages, int64_t start_pos,
                         int page_size, int64_t num_blocks, int layer_idx, int num_layers,
                         void* pool, sgl_stream_t stream);

/* KV row formats the sparse attention reads. */
enum sgl_attn_kv_format {
  SGL_ATTN_KV_BF16 = 0,    /* bf16 rows [n, ld] (ld >= 512, ld % 8 == 0) */
  SGL_ATTN_KV_A = 1,       /* layout A 584-byte rows [n, 584] (dsv4_kv_pack.py:40-75) */
  SGL_ATTN_KV_A_PAGED = 2  /* layout A footer pages of page_size rows (dsv4_kv_pack.py:104-146) */
};

/* Sparse multi-head attention with an attention sink over gathered KV rows:
 * for query (b, m) and head h, s_j = (q[b,m,h] . kv[b, idx[b,m,j]]) * scale
 * (idx -1, or outside [0, n), masked), online softmax over blocks of 64 rows
 * with bf16 probabilities in the P.V product and fp32 ones in the normaliser,
 * o = acc / (sum + exp(attn_sink[h] - max)) as bf16.  q bf16 [B, M, Hh, 512],
 * o bf16 [B, M, Hh, 512], attn_sink fp32 [Hh], topk_idxs int32 [B, M, K]; the
 * kv rows of batch element b start kv_batch_stride bytes apart; the FP8
 * layouts are dequantized on the way in (exactly: e4m3 * 2^(e8m0-127) fits
 * bf16), so the packed cache is read directly.  A small batch (decode) splits
 * the K rows over workgroups and needs a device workspace of
 * sgl_sparse_attn_workspace_size(B, M, Hh, K) bytes (0: none), 16-byte aligned.
 * Replaces deepseek_infer/kernel.py:350-368 sparse_attn (kernel :276-347) and
 * engine/v4_sparse_torch.py:20-106 sparse_attn_torch; with the FP8 formats,
 * the gather-dequant + attention of engine/v4_sparse_mla.py:104-118. */
int sgl_sparse_attn(const void* q, int64_t B, int64_t M, int Hh, const void* kv, int kv_format,
                    int page_size, int64_t n, int64_t kv_batch_stride, int64_t ld,
                    const float* attn_sink, const int32_t* topk_idxs, int64_t K,
                    float softmax_scale, void* o, void* workspace, size_t workspace_bytes,
                    sgl_stream_t stream);

/* Workspace bytes sgl_sparse_attn needs for this shape on the current device. */
size_t sgl_sparse_attn_workspace_size(int64_t B, int64_t M, int Hh, int64_t K);

/* Logical [T, 584] rows -> footer pages [ceil(T/page), page*584] (padding rows
 * zero).  Replaces engine/dsv4_kv_pack.py:104-146 to_paged_hnd. */
int sgl_kv_to_paged(const void* packed, int64_t T, int page_size, void* pages,
                    sgl_stream_t stream);

/* Gather-dequant for sparse MLA: out[q, i] = dequant(cache row idx[q, i]) as
 * bf16, an index of -1 gives a zero row.  Layout A rows give 512 values
 * (448 e4m3 * 2^(e8m0-127), 64 rope), layout B rows 576 (512 e4m3 * fp32
 * scale rounded to bf16, 64 rope).  cache holds n_rows rows (paged: footer
 * pages of page_size rows, layout A only).  idx int32 [nq, nsel],
 * out bf16 [nq, nsel, 512 | 576].  Indices >= n_rows are an error: the row
 * is zero-filled.  Semantics of engine/v4_sparse_torch.py:77-83 and
 * deepseek_infer/kernel.py:322-325 applied to the packed cache consumed at
 * engine/v4_sparse_mla.py:104-118. */
int sgl_kv_gather_dequant(const void* cache, int layout, int paged, int page_size, int64_t n_rows,
                          const int32_t* idx, int64_t nq, int64_t nsel, void* out,
                          sgl_stream_t stream);

/* Split concatenated top-k [BS, K] (int32, or int64 when idx_int64) into SWA
 * columns [BS, min(window, K)] + lens and compressed columns [BS, K - swa]
 * (valid entries shifted by -window) + lens, all int32.  Replaces
 * engine/dsv4_kv_pack.py:149-175 split_swa_compress_indices. */
int sgl_split_swa_compress_indices(const void* topk, int idx_int64, int64_t BS, int64_t K,
                                   int64_t window, int32_t* swa, int32_t* swa_lens,
                                   int32_t* comp, int32_t* comp_lens, sgl_stream_t stream);

/* ------------------------------------------------- host-side self checks */

/* The device numeric code compiled for the host, so the CPU test suite can
 * check it without a GPU.  n elements each. */
int sgl_host_f32_to_e4m3(const float* x, uint8_t* y, int64_t n);
int sgl_host_e4m3_to_f32(const uint8_t* x, float* y, int64_t n);
int sgl_host_group_scale(int scale_mode, const float* amax, float* scale, int64_t n);
int sgl_host_quant_elem(int scale_mode, const float* x, const float* scale, uint8_t* y, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* SGLANG_LITE_AMD_H_ */
