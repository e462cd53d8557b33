"""The HIP MoE path against the vectors the reference's own layer code wrote
(tests/golden/make_ref_moe.py): routing ids and the activation quant bytes
exact, the requantized h and the layer output within the requantization /
layer bounds of tests/helpers.py, for fp32 scales (tiny), the live ue8m0
scales with e8m0 FP8 weight scales, sqrtsoftplus + bias + route_scale 1.5 +
swiglu_limit 10 (live_fp8), and MXFP4 routed experts (live_fp4)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (assert_layer_close, assert_requant_close, f32, ref_moe_case, to_dev_bf16,
                     to_dev_f32, u8)

pytestmark = pytest.mark.gpu


def _table(stored, stored_sh, c, dev):
    from sglang_lite_amd import moe as M

    def sc(a):
        t = torch.from_numpy(np.ascontiguousarray(a))
        return (t.view(torch.float8_e8m0fnu) if a.dtype == np.uint8 else t).to(dev)

    def w8(a):
        return torch.from_numpy(np.ascontiguousarray(a)).view(torch.float8_e4m3fn).to(dev)

    def ent(e, fp4):
        wf = (lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)) if fp4 else w8
        return (wf(e["w1"]), wf(e["w3"]), wf(e["w2"]), sc(e["s1"]), sc(e["s3"]), sc(e["s2"]))

    return M.ExpertTable.build([ent(e, c["fp4"]) for e in stored], ent(stored_sh, False))


@pytest.mark.parametrize("name", ["tiny", "live_fp8", "live_fp4"])
def test_layer_against_reference_vectors(gpu, name):
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    print(f"reference golden {name}", flush=True)
    c, gold, inp, experts, shared, stored, stored_sh, digest = ref_moe_case(name)
    assert digest == bytes(gold["weights_sha256"]).decode()
    mode = 1 if c["ue8m0"] else 0
    table = _table(stored, stored_sh, c, gpu)
    bias = to_dev_f32(inp["bias"], gpu) if inp["bias"] is not None else None
    w, ids = M.route_topk(to_dev_f32(gold["logits"], gpu), c["k"], c["score_func"], bias,
                          c["route_scale"])
    np.testing.assert_array_equal(ids.cpu().numpy(), gold["ids"])
    np.testing.assert_allclose(f32(w), gold["route_w"], rtol=2e-6, atol=1e-7)
    xd = to_dev_bf16(inp["x"], gpu)
    xq, xs = K.act_quant(xd, scale_mode=mode)
    np.testing.assert_array_equal(u8(xq), gold["xq"])
    np.testing.assert_array_equal(f32(xs).view(np.uint32), gold["xs"].view(np.uint32))
    # h rows in the reference's order (experts ascending, tokens ascending, then
    # the shared expert) are the permuted row order of the grouped GEMM
    counts, offsets, sorted_slot, _ = M.permute(ids, c["E"])
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), table, c["k"],
                       swiglu_limit=c["swiglu_limit"], scale_mode=mode)
    y = M.moe_forward(xd, ids, w, table, swiglu_limit=c["swiglu_limit"], scale_mode=mode)
    torch.cuda.synchronize()
    assert_requant_close(u8(hq), f32(hs), gold["hq"], gold["hs"], f"{name} h")
    y_ref = (gold["y_bits"].astype(np.uint32) << 16).view(np.float32)
    assert_layer_close(f32(y), y_ref, f"{name} layer")
