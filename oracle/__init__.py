"""CPU oracle for the DeepSeek-V4-Flash FP8 MoE expert path and FP8 KV pack.

TEST INFRASTRUCTURE ONLY.  This package restates the reference algorithms
(ParaTensor/sglang-lite; each function cites the reference file:line it
follows) in numpy so the HIP kernels can be checked against it.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline.
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
* ``moe.moe_forward``: the reference's own toy test (tests/test_v4_moe_fast.py:
  10-43, activated-only loop == full loop) plus closed forms of the expert.
* ``kv``: the reference's tests (tests/test_dsv4_kv_pack.py:16-65,
  tests/test_v4_dual_pool.py:57-75) and closed forms of the footer layout.
  Layout B has no reference producer: parity unpinned beyond its closed form.
"""
