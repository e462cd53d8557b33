"""Pins the oracle's quantization against library routines and closed forms (CPU)."""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import quant as Q


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(
        torch.uint8).numpy()


def _boundary_values() -> np.ndarray:
    """fp32 values at and one ulp around every e4m3 rounding midpoint and code."""
    codes = Q.e4m3_to_f32(np.arange(127, dtype=np.uint8)).astype(np.float64)
    mids = (codes[:-1] + codes[1:]) / 2
    pts = np.concatenate([codes, mids, [448.0, 456.0, 464.0, 472.0, 480.0, 2.0**-10, 2.0**-11]])
    f = pts.astype(np.float32)
    u = f.view(np.uint32).astype(np.int64)
    around = np.concatenate([u - 2, u - 1, u, u + 1, u + 2])
    around = around[(around >= 0) & (around < 0x7F800000)].astype(np.uint32)
    v = around.view(np.float32)
    return np.concatenate([v, -v])


def test_e4m3_cast_matches_torch_on_every_bf16_value():
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(Q.f32_to_e4m3(bits), _torch_e4m3(bits))


def test_e4m3_cast_matches_torch_at_rounding_boundaries():
    v = _boundary_values()
    np.testing.assert_array_equal(Q.f32_to_e4m3(v), _torch_e4m3(v))


def test_e4m3_cast_matches_torch_on_random_fp32():
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(2_000_000).astype(np.float32) * np.float32(60.0))
    v2 = rng.integers(0, 2**32, 1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for arr in (v, v2):
        np.testing.assert_array_equal(Q.f32_to_e4m3(arr), _torch_e4m3(arr))


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = Q.e4m3_to_f32(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    v = rng.integers(0, 2**32, 1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    v = v[np.isfinite(v)]
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(Q.bf16_round(v).view(np.uint32), ref.view(np.uint32))


def test_per_token_closed_forms():
    rng = np.random.default_rng(2)
    x = Q.bf16_round(rng.standard_normal((64, 512)).astype(np.float32))
    x[3, :128] = 0.0  # all-zero group
    q, sf = Q.per_token_cast_to_fp8(x, False, 128)
    # all-zero group: scale fp32(1e-4)/448, zero bytes
    assert sf[3, 0] == np.float32(np.float32(1e-4) / np.float32(448.0))
    assert not q[3, :128].any()
    g = x.reshape(64, 4, 128)
    amax = np.abs(g).max(-1)
    for r in range(64):
        for c in range(4):
            if amax[r, c] == 0:
                continue
            # scale = amax/448 correctly rounded to fp32
            exact = Fraction(float(amax[r, c])) / 448
            cand = np.float32(float(exact))
            assert sf[r, c] == cand or abs(Fraction(float(sf[r, c])) - exact) <= abs(
                Fraction(float(cand)) - exact)
            # the element holding amax quantizes to +-448 (codes 0x7E / 0xFE)
            j = int(np.argmax(np.abs(g[r, c])))
            assert q[r, c * 128 + j] & 0x7F == 0x7E
    # dequantization error within half an e4m3 step (relative 2^-4) or the subnormal step
    deq = Q.dequant_rows(q, sf, 128)
    step = np.maximum(np.abs(x) * 2.0**-4, np.repeat(sf, 128, 1) * 2.0**-10)
    assert np.all(np.abs(deq - x) <= step * 1.0001)


def test_per_token_ue8m0_scale_brackets_amax():
    rng = np.random.default_rng(3)
    x = Q.bf16_round(rng.standard_normal((32, 256)).astype(np.float32) * 7)
    _, sf = Q.per_token_cast_to_fp8(x, True, 128)
    amax = np.maximum(np.abs(x.reshape(32, 2, 128)).max(-1), np.float32(1e-4))
    m, _ = np.frexp(sf)
    assert np.all(m == 0.5)  # powers of two
    assert np.all(sf >= amax / 448) and np.all(sf < 2 * amax / 448)


def test_tilelang_formula_clamps_and_uses_division():
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 300.0
    x[0, 1] = -300.0
    q, s = Q.act_quant_tilelang(x, 128)
    assert s[0, 0] == np.float32(np.float32(300.0) * Q.INV448)
    assert q[0, 0] == 0x7E and q[0, 1] == 0xFE


def test_kv_scale_log2_step_matches_torch_log2():
    """The ceil(log2(raw)) of dsv4_kv_pack.py:94 against torch.log2 on values
    at and just above powers of two (where it differs from exponent+1)."""
    ks = np.arange(-30, 10)
    js = np.arange(0, 40)
    target = (np.ldexp(1.0, ks)[:, None] * (1 + js[None, :] * 2.0**-23)).ravel()
    # fp32 amax values whose raw = amax * fp32(1/448) lands on / just above 2^k
    groups = np.zeros((target.size, 64), np.float32)
    groups[:, 0] = (target / float(Q.INV448)).astype(np.float32)
    _, scale = Q.kv_ue8m0_quant(groups, 64)
    raw = torch.from_numpy(groups[:, 0]).clamp(min=1e-12) * (1.0 / 448.0)
    ref = torch.exp2(torch.ceil(torch.log2(raw.clamp(min=2**-30)))).numpy()
    np.testing.assert_array_equal(scale[:, 0], ref)
    # the hazard is real: for some inputs the bit formula (exponent + 1) differs
    assert np.any(scale[:, 0] != Q.pow2_ceil_log2_bits(raw.numpy()))


def test_per_block_closed_forms():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((300, 200)).astype(np.float32) * np.float32(0.02))
    q, s = Q.per_block_cast_to_fp8(w)
    assert s.shape == (3, 2)
    for bi in range(3):
        for bj in range(2):
            blk = w[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            assert s[bi, bj] == np.float32(np.float32(np.abs(blk).max()) / np.float32(448.0))
            qb = q[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            r, c = np.unravel_index(np.argmax(np.abs(blk)), blk.shape)
            assert qb[r, c] & 0x7F == 0x7E


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_scale_modes_differ_only_in_documented_ways(mode):
    rng = np.random.default_rng(5 + mode)
    x = Q.bf16_round(rng.standard_normal((16, 256)).astype(np.float32))
    q, s = Q.scale_mode_quant(x, mode, 128 if mode != 4 else 64)
    deq = Q.dequant_rows(q, s, 128 if mode != 4 else 64)
    assert np.max(np.abs(deq - x)) <= np.max(np.abs(x)) * 2.0**-3
