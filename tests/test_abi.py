"""The C-ABI library: loads on CPU, exports every declared symbol, and its
host-compiled numeric core agrees with the oracle (no GPU compute here)."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from oracle import quant as Q

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sglang_lite_amd.h")


def _lib():
    from sglang_lite_amd import _lib

    return _lib.load()


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sgl_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from sglang_lite_amd import _lib

    assert declared_symbols() == sorted(_lib.SIGNATURES), (
        "ctypes signature table and include/sglang_lite_amd.h disagree")


def test_library_exports_every_declared_symbol():
    lib = _lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    from sglang_lite_amd import _lib as L

    assert lib.sgl_abi_version() == L.ABI_VERSION == 3


def test_probe_without_gpu_reports_why():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    lib = _lib()
    assert lib.sgl_probe() == 0
    assert lib.sgl_last_error()


def _host(fn, *arrays, n):
    lib = _lib()
    args = [a.ctypes.data_as(ctypes.c_void_p) if isinstance(a, np.ndarray) else a for a in arrays]
    assert getattr(lib, fn)(*args, n) == 0


def test_host_e4m3_conversion_matches_oracle():
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    rng = np.random.default_rng(0)
    rand = rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for x in (bits, rand):
        x = np.ascontiguousarray(x)
        y = np.zeros(x.size, np.uint8)
        _host("sgl_host_f32_to_e4m3", x, y, n=x.size)
        np.testing.assert_array_equal(y, Q.f32_to_e4m3(x))
    codes = np.arange(256, dtype=np.uint8)
    out = np.zeros(256, np.float32)
    _host("sgl_host_e4m3_to_f32", codes, out, n=256)
    ref = Q.e4m3_to_f32(codes)
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(out[ok], ref[ok])
    assert np.all(np.isnan(out[~ok]))


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_host_group_scale_and_quant_match_oracle(mode):
    rng = np.random.default_rng(10 + mode)
    group = 64 if mode == 4 else 128
    x = Q.bf16_round(rng.standard_normal((256, group * 2)).astype(np.float32) *
                     np.exp(rng.uniform(-12, 6, (256, 1))).astype(np.float32))
    x[0] = 0.0
    q_ref, s_ref = Q.scale_mode_quant(x, mode, group)
    amax = np.ascontiguousarray(np.abs(x.reshape(256, 2, group)).max(-1).ravel())
    s = np.zeros_like(amax)
    lib = _lib()
    assert lib.sgl_host_group_scale(mode, amax.ctypes.data_as(ctypes.c_void_p),
                                    s.ctypes.data_as(ctypes.c_void_p), amax.size) == 0
    np.testing.assert_array_equal(s, s_ref.ravel())
    xs = np.ascontiguousarray(x.ravel())
    ss = np.ascontiguousarray(np.repeat(s, group))
    q = np.zeros(xs.size, np.uint8)
    assert lib.sgl_host_quant_elem(mode, xs.ctypes.data_as(ctypes.c_void_p),
                                   ss.ctypes.data_as(ctypes.c_void_p),
                                   q.ctypes.data_as(ctypes.c_void_p), xs.size) == 0
    np.testing.assert_array_equal(q, q_ref.ravel())


def test_kv_scale_host_matches_torch_log2_near_powers_of_two():
    """fp32 amax values whose raw scale sits just above 2^k: the library follows
    torch.log2 (correctly rounded), not the exponent+1 bit formula."""
    ks = np.arange(-28, 10)
    js = np.arange(0, 24)
    target = (np.ldexp(1.0, ks)[:, None] * (1 + js[None, :] * 2.0**-23)).ravel()
    amax = np.ascontiguousarray((target / float(Q.INV448)).astype(np.float32))
    s = np.zeros_like(amax)
    lib = _lib()
    assert lib.sgl_host_group_scale(4, amax.ctypes.data_as(ctypes.c_void_p),
                                    s.ctypes.data_as(ctypes.c_void_p), amax.size) == 0
    raw = torch.from_numpy(amax).clamp(min=1e-12) * (1.0 / 448.0)
    ref = torch.exp2(torch.ceil(torch.log2(raw.clamp(min=2**-30)))).numpy()
    np.testing.assert_array_equal(s, ref)


def test_kv_scale_mantissa_shortcut_premise():
    """The KV ue8m0 scale skips the double log2 when the raw scale's mantissa
    field M is 0 (-> 2^k) or above 64 (-> 2^(k+1)).  Pin the premise: for every
    exponent the raw scale can have, M = 65 already rounds log2 above k (the
    smallest such M, log2 is monotone), while small M can round to exactly k."""
    ks = np.arange(-30, 128)
    for M, expect_up in ((65, True), (1, None)):
        raw = (np.ldexp(1.0, ks) * (1 + M * 2.0**-23)).astype(np.float32)
        ceil_t = torch.ceil(torch.log2(torch.from_numpy(raw))).numpy().astype(np.int64)
        ceil_d = np.ceil(np.log2(raw.astype(np.float64)).astype(np.float32)).astype(np.int64)
        np.testing.assert_array_equal(ceil_t, ceil_d)
        if expect_up:
            np.testing.assert_array_equal(ceil_t, ks + 1)
        else:
            assert (ceil_t == ks).any()  # the hazard the double path exists for
    # end to end through the library on amax values whose raw scale has
    # M in [0, 70] or near the top, over the whole exponent range
    ms = np.concatenate([np.arange(0, 71), [2**22, 2**23 - 1]])
    raw = (np.ldexp(1.0, ks)[:, None] * (1 + ms[None, :] * 2.0**-23)).ravel()
    amax = np.ascontiguousarray((raw / float(Q.INV448)).astype(np.float32))
    amax = amax[np.isfinite(amax)]
    s = np.zeros_like(amax)
    lib = _lib()
    assert lib.sgl_host_group_scale(4, amax.ctypes.data_as(ctypes.c_void_p),
                                    s.ctypes.data_as(ctypes.c_void_p), amax.size) == 0
    rawt = torch.from_numpy(amax).clamp(min=1e-12) * (1.0 / 448.0)
    ref = torch.exp2(torch.ceil(torch.log2(rawt.clamp(min=2**-30)))).numpy()
    np.testing.assert_array_equal(s, ref)


def test_invalid_arguments_map_to_value_error_without_launch():
    from sglang_lite_amd import _lib as L

    lib = _lib()
    rc = lib.sgl_act_quant(None, 4, 100, 100, None, 100, None, 1, 128, 0, 0, 0, None)
    assert rc == L.SGL_ERR_INVALID_ARG
    assert "divisible" in L.last_error()
    with pytest.raises(ValueError, match="group"):
        L.call("sgl_act_quant", None, 4, 128, 128, None, 128, None, 1, 96, 0, 0, 0, None)
    rc = lib.sgl_fp8_gemm(None, None, 0, None, None, 0, None, 0, 4, 100, 256, None, 0, None)
    assert rc == L.SGL_ERR_INVALID_ARG and "multiple of 16" in L.last_error()
    rc = lib.sgl_hbm_stream(None, None, 1000, None, None)
    assert rc == L.SGL_ERR_INVALID_ARG and "multiple of 32768" in L.last_error()
    rc = lib.sgl_mfma_mix(2, None, 10, None)
    assert rc == L.SGL_ERR_INVALID_ARG and "variant" in L.last_error()
    rc = lib.sgl_moe_permute(None, 4, 2, 5000, None, None, None, None, None)
    assert rc == L.SGL_ERR_INVALID_ARG
    assert lib.sgl_moe_workspace_size(8192, 4096, 2048, 256, 8, 1) > 8192 * 4096


def test_product_refuses_cpu_tensors():
    from sglang_lite_amd import dsv4_kv_pack as KVP
    from sglang_lite_amd import kernel as K

    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        K.act_quant(x)
    with pytest.raises(RuntimeError, match="no CPU path"):
        KVP.pack_dsv4_kv_bf16(torch.zeros(2, 512, dtype=torch.bfloat16))
    # argument errors keep the reference's exception types (dsv4_kv_pack.py:50-53)
    with pytest.raises(ValueError):
        KVP.pack_dsv4_kv_bf16(torch.zeros(2, 500, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        KVP.pack_dsv4_kv_bf16(torch.zeros(2, 512, dtype=torch.int32))
    with pytest.raises(AssertionError):
        K.act_quant(torch.zeros(2, 100, dtype=torch.bfloat16))


@pytest.mark.parametrize("name", ["sgl_moe_forward", "sgl_moe_gate_up", "sgl_moe_down"])
@pytest.mark.parametrize("T", [300_000, 600_000])
def test_moe_rejects_tokens_beyond_32_bit_operand_offsets(name, T):
    """The grouped GEMMs address A rows with 32-bit lane offsets (xq [T, H],
    hq [T (k + 1), I]): a T whose operands pass 2 GiB is refused with
    ValueError before any launch (null pointers: nothing is touched)."""
    from sglang_lite_amd import _lib as L

    H, I, E, k = 4096, 2048, 256, 8
    args = {
        "sgl_moe_forward": (None, T, H, I, E, k, None, None, None, 1, 0, 0.0, 0, None, 0, None, None),
        "sgl_moe_gate_up": (None, None, T, H, I, E, k, None, None, None, None, 1, 0, 0.0, 0, None,
                            None, None),
        "sgl_moe_down": (None, None, T, H, I, E, k, None, None, None, 1, 0, 0, None, None),
    }[name]
    with pytest.raises(ValueError, match="2 GiB operand limit"):
        L.call(name, *args)
    # a prefill-sized T passes the shape checks (then fails on the null pointers)
    small = list(args)
    small[args.index(T)] = 8192
    with pytest.raises(ValueError, match="null pointer"):
        L.call(name, *small)


def test_expert_format_pow2_flag():
    """Power-of-two weight scales are recognised (e8m0 by type, fp32 with no
    mantissa bits, positive); the C boundary accepts SGL_EXPERT_POW2_SCALES
    and SGL_EXPERT_FRAG_COPY OR'ed into either weight format and refuses any
    other bit before a launch."""
    from sglang_lite_amd import _lib as L
    from sglang_lite_amd import moe as M

    e8 = torch.tensor([1, 120, 127, 254], dtype=torch.uint8).view(torch.float8_e8m0fnu)
    assert M._pow2_scale(e8)
    assert M._pow2_scale(torch.tensor([0.25, 1.0, 2.0 ** -20, 2.0 ** 60]))
    assert not M._pow2_scale(torch.tensor([0.25, 0.3]))           # a mantissa bit
    assert not M._pow2_scale(torch.tensor([1.0, 0.0]))            # zero
    assert not M._pow2_scale(torch.tensor([-1.0, 1.0]))           # sign
    assert not M._pow2_scale(torch.tensor([2.0 ** -130]))         # subnormal
    assert L.EXPERT_POW2_SCALES == 2 and L.EXPERT_FRAG_COPY == 4
    H, I, E, k = 4096, 2048, 256, 8
    for fmt, ok in ((0, True), (1, True), (2, True), (3, True), (4, True), (7, True), (8, False),
                    (10, False), (2 | 16, False)):
        args = (None, None, 64, H, I, E, k, None, None, None, None, 1, fmt, 0.0, 0, None, None, None)
        with pytest.raises(ValueError, match="null pointer" if ok else "bad expert_format"):
            L.call("sgl_moe_gate_up", *args)


def test_fp8_gemm_split_decision_is_a_function_of_the_shape():
    """sgl_fp8_gemm_workspace_size depends on (M, N, K) only: split-K for
    16 < M <= 64 with N % 128 == 0, S splits of fp32 [M, N] partials; a call
    whose shape splits and whose workspace is missing or short is refused with
    SGL_ERR_WORKSPACE before anything is launched (the pointers below are
    never dereferenced), rather than summed in another order."""
    from sglang_lite_amd import _lib as L

    lib = _lib()
    ws = lib.sgl_fp8_gemm_workspace_size
    assert ws(40, 4096, 7168) == 8 * 40 * 4096 * 4  # 56 K blocks in 8 splits of 7
    assert ws(17, 4096, 7168) == 8 * 17 * 4096 * 4
    assert ws(64, 384, 2048) > 0
    for M, N, K in ((16, 4096, 7168), (65, 4096, 7168), (1024, 4096, 7168), (40, 4096 + 16, 7168)):
        assert ws(M, N, K) == 0, (M, N, K)
    fake = 1 << 20  # aligned, never read: the workspace check comes first
    need = ws(40, 4096, 7168)
    for buf, n in ((None, 0), (fake, need - 16)):
        rc = lib.sgl_fp8_gemm(fake, fake, 0, fake, fake, 0, fake, 0, 40, 4096, 7168, buf, n, None)
        assert rc == L.SGL_ERR_WORKSPACE, rc
        assert str(need) in L.last_error()
