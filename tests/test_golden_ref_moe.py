"""The oracle's MoE composition against vectors written by the reference's own
layer code (tests/golden/make_ref_moe.py: the official Gate / Expert / MoE of
deepseek_infer/model.py:546-644 and engine/v4_moe_fast.py:43-106, with a
dequantize-to-fp32 stand-in for the FP8 / FP4 GEMMs).

Pinned exactly: the expert weight bytes (the oracle's per_block_cast_to_fp8
against the reference's), routing ids, the 1x128 quant of x.  Pinned to the
bf16 ulp: h, the input of w2's act_quant (routing weight, SwiGLU with its
asymmetric clamp, bf16 rounding); the h quant bytes wherever h agrees.
Within the GEMM tolerance: every expert's output and the layer output."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_gemm_close, ref_moe_case
from oracle import moe as OM
from oracle import quant as Q

CASES = ["tiny", "live_fp8", "live_fp4"]


def _bits_to_f32(b):
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("name", CASES)
def test_inputs_rebuild_to_the_reference_bytes(name):
    c, gold, inp, experts, shared, stored, stored_sh, digest = ref_moe_case(name)
    assert digest == bytes(gold["weights_sha256"]).decode()


@pytest.mark.parametrize("name", CASES)
def test_routing_and_activation_quant_exact(name):
    c, gold, inp, *_ = ref_moe_case(name)
    w, ids = OM.route_topk(gold["logits"], c["k"], c["score_func"], inp["bias"], c["route_scale"])
    assert OM.topk_margin(gold["logits"], c["k"], c["score_func"], inp["bias"]) > 1e-6
    np.testing.assert_array_equal(ids, gold["ids"])
    np.testing.assert_allclose(w, gold["route_w"], rtol=2e-6, atol=1e-7)
    mode = 1 if c["ue8m0"] else 0
    xq, xs = Q.scale_mode_quant(inp["x"], mode, 128)
    np.testing.assert_array_equal(xq, gold["xq"])
    np.testing.assert_array_equal(xs.view(np.uint32), gold["xs"].view(np.uint32))


@pytest.mark.parametrize("name", CASES)
def test_expert_composition_matches_reference(name):
    """Per expert (ascending id, rows in token order; the shared expert last):
    h within one bf16 ulp (and equal almost everywhere), h's quant bytes equal
    on every row whose h is equal, the output within the GEMM tolerance."""
    c, gold, inp, experts, shared, *_ = ref_moe_case(name)
    mode = 1 if c["ue8m0"] else 0
    x, ids, w = inp["x"], gold["ids"], gold["route_w"]
    h_ref = _bits_to_f32(gold["h_bits"])
    out_ref = _bits_to_f32(gold["out_bits"])
    row = 0
    same = total = 0
    for e in range(c["E"] + 1):
        if e < c["E"]:
            tok, top = np.nonzero(ids == e)
            if tok.size == 0:
                continue
            tr = {}
            out = OM.expert_forward(x[tok], experts[e], w[tok, top][:, None], c["swiglu_limit"],
                                    mode, trace=tr)
        else:
            tok = np.arange(c["T"])
            tr = {}
            out = OM.expert_forward(x, shared, None, c["swiglu_limit"], mode, trace=tr)
        n = tok.size
        hr = h_ref[row:row + n]
        h = tr["h"]
        ulp = np.abs(h.view(np.int32).astype(np.int64) - hr.view(np.int32).astype(np.int64)) >> 16
        assert int(ulp.max()) <= 1, f"expert {e}: h differs by more than one bf16 ulp"
        same += int(np.sum(ulp == 0))
        total += h.size
        eq_rows = np.all(ulp == 0, axis=1)
        np.testing.assert_array_equal(tr["hq"][eq_rows], gold["hq"][row:row + n][eq_rows])
        np.testing.assert_array_equal(tr["hs"][eq_rows].view(np.uint32),
                                      gold["hs"][row:row + n][eq_rows].view(np.uint32))
        assert_gemm_close(out, out_ref[row:row + n], f"{name} expert {e}")
        row += n
    assert row == gold["h_bits"].shape[0]
    assert same >= 0.99 * total, f"only {same}/{total} h values equal"


@pytest.mark.parametrize("name", CASES)
def test_layer_matches_reference(name):
    c, gold, inp, experts, shared, *_ = ref_moe_case(name)
    mode = 1 if c["ue8m0"] else 0
    y = OM.moe_forward(inp["x"], gold["ids"], gold["route_w"], experts, shared,
                       c["swiglu_limit"], mode)
    y_ref = _bits_to_f32(gold["y_bits"])
    assert_gemm_close(y, y_ref, f"{name} layer")
    assert np.mean(y.view(np.uint32) == y_ref.view(np.uint32)) > 0.9
    # the official full loop (model.py:629-644) is the same composition
    y_full = OM.moe_forward_full_loop(inp["x"], gold["ids"], gold["route_w"], experts, shared,
                                      c["swiglu_limit"], mode)
    np.testing.assert_array_equal(y_full.view(np.uint32), y.view(np.uint32))


def test_clamp_binds_in_the_live_cases():
    """The live cases exercise the SwiGLU clamp (swiglu_limit 10): some gate or
    up value of the reference's h exceeds the limit before clamping, so an
    unclamped or symmetrically clamped restatement would fail above."""
    for name in ("live_fp8", "live_fp4"):
        c, gold, *_ = ref_moe_case(name)
        h = np.abs(_bits_to_f32(gold["h_bits"]))
        assert h.max() > c["swiglu_limit"], name
