"""Attach / probe contract of the drop-in modules on CPU (no GPU compute):
env switches, probe failure leaves the official functions untouched, error
mapping; mirrors tests/test_v4_moe_fast.py:46-52 of the reference."""

from __future__ import annotations

import pytest
import torch

import fake_official


@pytest.fixture
def official():
    M, K, saved = fake_official.install()
    yield M, K
    fake_official.uninstall(saved)


def test_moe_fast_env_default_on(monkeypatch):
    from sglang_lite_amd.v4_moe_fast import moe_fast_enabled

    monkeypatch.delenv("SGLANG_LITE_V4_MOE_FAST", raising=False)
    assert moe_fast_enabled() is True
    monkeypatch.setenv("SGLANG_LITE_V4_MOE_FAST", "0")
    assert moe_fast_enabled() is False


def test_deep_gemm_env_switch(monkeypatch, official):
    from sglang_lite_amd import v4_deep_gemm as D

    monkeypatch.setenv("SGLANG_LITE_V4_DEEP_GEMM", "off")
    st = D.attach_v4_deep_gemm(None)
    assert st["backend"] == "disabled" and not st["patched"]


@pytest.mark.skipif(torch.cuda.is_available(), reason="probe succeeds on a GPU")
def test_failed_probe_leaves_official_functions(official):
    from sglang_lite_amd import v4_deep_gemm as D
    from sglang_lite_amd import v4_moe_fast as F

    M, K = official
    orig = (K.fp8_gemm, K.act_quant, M.MoE.forward, M.Expert.forward)
    st = D.attach_v4_deep_gemm(None)
    assert st["enabled"] is False and st["probe"]["ok"] is False
    st2 = F.attach_v4_moe_fast(torch.nn.Module())
    assert st2["enabled"] is False
    assert (K.fp8_gemm, K.act_quant, M.MoE.forward, M.Expert.forward) == orig
    assert D.is_armed() is False


def test_fp4_path_refuses_cpu_tensors():
    from sglang_lite_amd import v4_deep_gemm as D

    a = torch.zeros(2, 256, dtype=torch.float8_e4m3fn)
    s = torch.ones(2, 2)
    b = torch.zeros(16, 128, dtype=torch.uint8)
    bs = torch.ones(16, 8)
    with pytest.raises(RuntimeError, match="no CPU path"):
        D.fp4_gemm_nt(a, s, b, bs)


def test_fp4_weight_detection():
    from sglang_lite_amd import v4_deep_gemm as D

    w = torch.nn.Parameter(torch.zeros(64, 128, dtype=torch.int8), requires_grad=False)
    w.scale = torch.nn.Parameter(torch.ones(64, 8), requires_grad=False)  # in = 256, 256/32 = 8
    assert D.is_fp4_weight(w)
    w.scale = torch.nn.Parameter(torch.ones(1, 2), requires_grad=False)  # 128x128 block scale
    assert not D.is_fp4_weight(w)
    w4 = torch.zeros(64, 128, dtype=torch.uint8).view(torch.float4_e2m1fn_x2)
    assert D.is_fp4_weight(w4)


def test_scale_formula_switch(monkeypatch):
    from sglang_lite_amd import _lib, kernel as K

    monkeypatch.delenv("SGLANG_LITE_AMD_ACT_QUANT", raising=False)
    assert K.scale_mode_for(None) == _lib.SCALE_TORCH_FP32
    assert K.scale_mode_for("ue8m0") == _lib.SCALE_TORCH_UE8M0
    monkeypatch.setenv("SGLANG_LITE_AMD_ACT_QUANT", "tilelang")
    assert K.scale_mode_for(None) == _lib.SCALE_TILELANG_FP32
    assert K.scale_mode_for("ue8m0") == _lib.SCALE_TILELANG_UE8M0
    monkeypatch.setenv("SGLANG_LITE_AMD_ACT_QUANT", "bogus")
    with pytest.raises(ValueError):
        K.scale_mode_for(None)


def test_kv_pack_fuses_the_attached_act_quant():
    """After attach_v4_deep_gemm, kernel.act_quant is the package's drop-in
    wrapper; the live KV pack injects that name (engine/v4_sparse_mla.py:85,91),
    so the pack must compute its formula in the fused kernel (not call it
    through the unfused path), like the package's own act_quant."""
    from sglang_lite_amd import dsv4_kv_pack as KVP
    from sglang_lite_amd import kernel as HK
    from sglang_lite_amd import v4_deep_gemm as D

    want = HK.scale_mode_for("ue8m0")
    assert KVP._fused_quant_mode(HK.act_quant) == want
    assert KVP._fused_quant_mode(D._act_quant_dropin) == want
    assert KVP._fused_quant_mode(None) == KVP._lib.SCALE_KV_UE8M0

    def other(*a, **k):
        raise AssertionError

    assert KVP._fused_quant_mode(other) is None
