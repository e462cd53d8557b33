"""CPU oracle for the DeepSeek-V4-Flash FP8 MoE expert path and FP8 KV pack.

TEST INFRASTRUCTURE ONLY.  This package restates the reference algorithms
(ParaTensor/sglang-lite; each function cites the reference file:line it
follows) in numpy so the HIP kernels can be checked against it.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only to check results against or as the timed
CPU baseline.
The product package (``sglang_lite_amd``) never imports it and has no CPU
fallback.

Pinning (what checks each function against something other than itself):

* ``quant.f32_to_e4m3``: torch's ``float8_e4m3fn`` cast over every bf16 value,
  all fp32 values near each e4m3 rounding boundary and random fp32
  (``tests/test_oracle_quant.py``).
* ``quant.per_token_cast_to_fp8`` / ``act_quant_tilelang`` /
  ``per_block_cast_to_fp8`` / ``kv_ue8m0_quant``: closed forms (all-zero group,
  amax element maps to +-448, scale equals the correctly rounded quotient,
  power-of-two scale bracketing), the torch cast above, and torch.log2 for the
  ceil(log2) step of the KV scale.
* ``moe.route_topk``: torch.topk / softmax as library routines.
* ``moe.permute``: brute-force torch.where loop of the reference
  (model.py:634-640) and invariants (bijection, offsets = cumsum(bincount)).
* ``moe.expert_forward`` / ``moe.moe_forward``: vectors written by the
  reference's own layer code (tests/golden/make_ref_moe.py runs the official
  Gate / Expert / MoE of deepseek_infer/model.py and engine/v4_moe_fast.py's
  activated-only dispatch with a dequantize-to-fp32 stand-in GEMM): routing
  ids and the x quant exact, h (the input of w2's act_quant) within one bf16
  ulp and its quant bytes exact where h agrees, expert and layer outputs
  within the GEMM tolerance (tests/test_golden_ref_moe.py); the full loop of
  model.py:629-644 (``moe_forward_full_loop``) equal to the activated-only
  loop bit for bit.
* ``fp4``: the e2m1 table (code 8 = +0.0) and the repack bytes against the
  reference converter's output (tests/golden/make_ref_fp4_repack.py).
* ``kv``: the reference's tests (tests/test_dsv4_kv_pack.py:16-65,
  tests/test_v4_dual_pool.py:57-75) and closed forms of the footer layout.
  Layout B has no reference producer: parity unpinned beyond its closed form.
"""
