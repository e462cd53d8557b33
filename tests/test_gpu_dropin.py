"""The drop-in on a stand-in official graph: attach, then the patched
MoE.forward / Expert.forward / kernel.act_quant / kernel.fp8_gemm against the
oracle (the calls the reference makes at engine/v4_moe_fast.py:58-106,
deepseek_infer/model.py:108-120,629-644)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fake_official
from helpers import assert_gemm_close, bf16_values, f32, to_dev_bf16, to_dev_f32, to_dev_fp8, u8
from oracle import moe as OM
from oracle import quant as Q

pytestmark = pytest.mark.gpu


@pytest.fixture
def official(gpu):
    from sglang_lite_amd import v4_deep_gemm as D
    from sglang_lite_amd import v4_moe_fast as MF

    M, K, saved = fake_official.install()
    yield M, K
    MF.detach_v4_moe_fast()
    D.detach_v4_deep_gemm()
    fake_official.uninstall(saved)


def _dev_expert(e, dev, e8m0=False):
    def sc(s):
        if e8m0:
            return torch.from_numpy(Q.e8m0_byte(s)).view(torch.float8_e8m0fnu).to(dev)
        return to_dev_f32(s, dev)

    return (to_dev_fp8(e["w1"], dev), to_dev_fp8(e["w3"], dev), to_dev_fp8(e["w2"], dev),
            sc(e["s1"]), sc(e["s3"]), sc(e["s2"]))


def test_attach_and_moe_forward(official, gpu):
    from sglang_lite_amd import v4_deep_gemm as D
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    rng = np.random.default_rng(41)
    T, H, I, E, k = 48, 512, 256, 16, 4
    x = bf16_values(rng, (T, H))
    W = (rng.standard_normal((E, H)) * H ** -0.5).astype(np.float32)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    gate = M.Gate(to_dev_f32(W, gpu), k)
    moe = M.MoE(H, gate, [M.Expert(_dev_expert(e, gpu)) for e in experts],
                M.Expert(_dev_expert(sh, gpu)))
    st = MF.attach_v4_moe_fast(moe)
    assert st["enabled"] and st["moe_class_patched"] == 1 and st["expert_modules"] == E + 1
    assert MF.attach_v4_moe_fast(moe)["moe_class_patched"] == 0  # idempotent
    st = D.attach_v4_deep_gemm(moe)
    assert st["enabled"] and st["patched"] and st["backend"] == "gfx950_hip" and D.is_armed()
    xd = to_dev_bf16(x, gpu)
    y = moe(xd.view(1, T, H), torch.zeros(1, T, dtype=torch.long, device=gpu))
    assert y.shape == (1, T, H) and y.dtype == torch.bfloat16
    # oracle on the same router logits (the projection is torch's fp32 GEMM on the device)
    logits = F.linear(xd.float(), gate.weight.float()).cpu().numpy()
    w_ref, ids_ref = OM.route_topk(logits, k)
    assert OM.topk_margin(logits, k) > 1e-6
    y_ref = OM.moe_forward(x, ids_ref, w_ref, experts, sh)
    assert_gemm_close(f32(y[0]), y_ref, "patched MoE.forward")


def test_expert_forward_and_linear_dropins(official, gpu):
    from sglang_lite_amd import v4_deep_gemm as D
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    rng = np.random.default_rng(42)
    T, H, I = 20, 512, 256
    x = bf16_values(rng, (T, H))
    e = OM.make_expert(rng, H, I)
    ex = M.Expert(_dev_expert(e, gpu, e8m0=True), swiglu_limit=10.0)
    MF.attach_v4_moe_fast(torch.nn.ModuleList([ex]))
    D.attach_v4_deep_gemm(None)
    w = rng.uniform(0.1, 1.0, (T, 1)).astype(np.float32)
    # e8m0 weight scales hold the same powers of two only for ue8m0 weights: use
    # the exact e8m0 values of the fp32 scales in the oracle
    e8 = {k_: (Q.e8m0_byte(v).astype(np.uint32) << 23).view(np.float32) if k_.startswith("s") else v
          for k_, v in e.items()}
    y = ex(to_dev_bf16(x, gpu), to_dev_f32(w, gpu))
    y_ref = OM.expert_forward(x, e8, w, swiglu_limit=10.0)
    assert_gemm_close(f32(y), y_ref, "patched Expert.forward")
    # kernel.act_quant / kernel.fp8_gemm and the copies model.py imported
    assert K.fp8_gemm is M.fp8_gemm and K.act_quant is M.act_quant
    xq, xs = M.act_quant(to_dev_bf16(x, gpu), 128, None, torch.float32)
    q_ref, s_ref = Q.per_token_cast_to_fp8(x, False, 128)
    np.testing.assert_array_equal(u8(xq), q_ref)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        c = M.fp8_gemm(xq, xs, ex.w1.weight, ex.w1.weight.scale, torch.float32)
    finally:
        torch.set_default_dtype(prev)
    ref = OM.fp8_gemm(q_ref, s_ref, e8["w1"], e8["s1"], out_bf16=False)
    assert_gemm_close(f32(c), ref, "patched kernel.fp8_gemm")
    assert getattr(ex.w1.weight, "_dg_s_f32", None) is not None  # scale cache on the Parameter
