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


# ------------------------------------------------------------------
# TileLang act_quant (deepseek_infer/kernel.py:22-37,79-96): the scale and
# the quotient are pinned independently of the oracle's own arithmetic.


def _exact_quotient_f32(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    """fp32 round-to-nearest-even of the exact quotient x / s, decided without
    trusting a float division's rounding: the float64 quotient only picks the
    neighbourhood, and its three float32 neighbours are ranked by their
    residuals |x - c*s|, which are exact in float64 (c and s
    have 24-bit significands, so c*s has at most 48 bits, and c*s is within a
    factor of two of x, so the subtraction is exact by Sterbenz's lemma);
    equal residuals go to the even significand."""
    x = np.asarray(x, np.float32)
    s = np.asarray(s, np.float32)
    c0 = (x.astype(np.float64) / s.astype(np.float64)).astype(np.float32)
    cands = np.stack([np.nextafter(c0, np.float32(-np.inf)), c0,
                      np.nextafter(c0, np.float32(np.inf))]).astype(np.float32)
    res = np.abs(x.astype(np.float64)[None] - cands.astype(np.float64) * s.astype(np.float64)[None])
    best = res.min(axis=0)
    odd = (cands.view(np.uint32) & 1).astype(bool)
    # among the minimisers prefer the even significand
    score = np.where(res == best[None], np.where(odd, 1, 0), 2)
    pick = np.argmin(score, axis=0)
    return np.take_along_axis(cands, pick[None], axis=0)[0]


def _fraction_round_f32(num: Fraction) -> np.float32:
    """fp32 RNE of an exact rational (normal range), by brute force over the
    two float32 neighbours of the double nearest to it."""
    c = np.float32(float(num))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(cand)) - num)
        key = (d, int(np.float32(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, np.float32(cand))
    return best[1]


def _tilelang_sweep(amaxes: np.ndarray):
    """Every bf16 value x with |x| <= amax, for each amax, laid out as 1x128
    groups whose element 0 is the amax itself (so the group's amax is known).
    Returns the groups and the group amax per group."""
    allbf = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    allbf = allbf[np.isfinite(allbf)]
    groups, gam = [], []
    for a in amaxes:
        xs = allbf[np.abs(allbf) <= a]
        n = -(-xs.size // 127)
        pad = np.zeros(n * 127, np.float32)
        pad[:xs.size] = xs
        g = np.empty((n, 128), np.float32)
        g[:, 0] = a
        g[:, 1:] = pad.reshape(n, 127)
        groups.append(g)
        gam.append(np.full(n, a, np.float32))
    return np.concatenate(groups), np.concatenate(gam)


def test_tilelang_fp32_mode_is_clamped_exact_division_over_every_bf16_value():
    """Mode 2 (kernel.py:83,93-96): s = amax * fp32(1/448), q = e4m3(clamp(x / s,
    +-448)) with x / s the correctly rounded fp32 quotient.  Swept over every
    bf16 value at 300 group maxima; the expected codes come from the exact
    quotient (residual ranking above) and torch's e4m3 cast.  The sweep holds
    inputs where multiplying by fp32(1/s) instead gives another code, so a
    reciprocal-based oracle fails it."""
    rng = np.random.default_rng(11)
    allbf = (np.arange(1, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    amaxes = np.unique(np.concatenate([
        rng.choice(allbf[(allbf >= 1e-4) & (allbf <= 1e4)], 297, replace=False),
        np.float32([1.4375, 1e-4, 448.0])])).astype(np.float32)
    amaxes = np.maximum(amaxes, np.float32(1e-4))
    g, gam = _tilelang_sweep(amaxes)
    q, s = Q.act_quant_tilelang(g, 128, round_scale=False)
    s_ref = (gam * np.float32(1.0 / 448.0)).astype(np.float32)
    np.testing.assert_array_equal(s[:, 0], s_ref)
    quo = _exact_quotient_f32(g, np.repeat(s_ref, 128).reshape(g.shape))
    ref = _torch_e4m3(np.clip(quo, -448.0, 448.0))
    np.testing.assert_array_equal(q, ref)
    recip = (g * (np.float32(1.0) / s_ref)[:, None]).astype(np.float32)
    n_diff = int((_torch_e4m3(np.clip(recip, -448.0, 448.0)) != ref).sum())
    assert n_diff > 0, "the sweep must hold inputs that tell division from the reciprocal"


def test_tilelang_division_known_answer():
    """amax 1.4375, x = 2.193451e-05 (bf16): x / s lands exactly on the midpoint
    3.5 * 2^-9 of two e4m3 subnormals and ties to the even code 0x04; the
    product with fp32(1/s) is one ulp below it and rounds to 0x03."""
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 1.4375
    x[0, 1] = np.float32(2.193450927734375e-05)
    q, s = Q.act_quant_tilelang(x, 128)
    sv = Fraction(float(np.float32(1.4375) * np.float32(1.0 / 448.0)))
    quo = _fraction_round_f32(Fraction(float(x[0, 1])) / sv)
    assert float(quo) == 3.5 * 2.0**-9
    assert q[0, 1] == 0x04 and q[0, 0] == 0x7E
    assert _torch_e4m3(np.float32(x[0, 1]) * (np.float32(1.0) / s[:, 0]))[0] == 0x03


def test_exact_quotient_helper_against_fractions():
    """The residual ranking used above equals RNE of the rational quotient."""
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(3000) * 10.0).astype(np.float32)
    x = Q.bf16_round(x)
    s = (np.abs(rng.standard_normal(3000)) * 0.01 + 1e-6).astype(np.float32)
    got = _exact_quotient_f32(x, s)
    for i in range(x.size):
        if x[i] == 0:
            assert got[i] == 0
            continue
        exp = _fraction_round_f32(Fraction(float(x[i])) / Fraction(float(s[i])))
        assert got[i] == exp, (x[i], s[i], got[i], exp)


def _brute_pow2_ceil(raw: np.ndarray) -> np.ndarray:
    """Smallest power of two >= raw, by comparison against every 2^k."""
    ks = np.arange(-140, 129, dtype=np.float64)
    p = np.exp2(ks)
    r = np.asarray(raw, np.float64)[:, None]
    k = ks[np.argmax(p[None, :] >= r, axis=1)]
    return np.exp2(k).astype(np.float32)


def test_tilelang_ue8m0_scale_is_the_smallest_power_of_two_above_raw():
    """Mode 3 (kernel.py:22-37,80-81): s = 2^ceil(log2(amax * fp32(1/448))) by
    the bit rule; checked against a brute-force search over every power of two,
    on random fp32 maxima and on maxima whose raw scale is at, or a few ulp
    above or below, a power of two."""
    rng = np.random.default_rng(13)
    am = np.abs(rng.standard_normal(20000)).astype(np.float32) * np.float32(50.0)
    ks = np.arange(-13, 3)
    near = []
    for kk in ks:
        base = np.float32(2.0**float(kk))
        u = base.view(np.uint32).astype(np.int64)
        for d in (-3, -1, 0, 1, 2, 5, 40):
            raw = np.uint32(u + d).view(np.float32)
            near.append(np.float32(raw / np.float32(1.0 / 448.0)))
    am = np.maximum(np.concatenate([am, np.float32(near)]), np.float32(1e-4)).astype(np.float32)
    g = np.zeros((am.size, 128), np.float32)
    g[:, 0] = am
    _, s = Q.act_quant_tilelang(g, 128, round_scale=True)
    raw = (am * np.float32(1.0 / 448.0)).astype(np.float32)
    np.testing.assert_array_equal(s[:, 0], _brute_pow2_ceil(raw))


def test_tilelang_ue8m0_differs_from_the_kv_log2_rule_just_above_powers_of_two():
    """Mode 3 (the quantizer the live KV pack injects, engine/v4_sparse_mla.py:
    85,91) and mode 4 (the torch fallback, dsv4_kv_pack.py:92-94) disagree
    exactly where raw is a few ulp above 2^k: torch.log2 rounds to k there, so
    mode 4 keeps 2^k while mode 3 goes to 2^(k+1) (the brute-force ceiling).
    At exact powers of two and elsewhere they agree."""
    rows, kinds = [], []
    for kk in range(-14, 4):
        base = np.float32(2.0**kk)
        u = int(base.view(np.uint32))
        for d, kind in ((0, "exact"), (1, "above"), (2, "above"), (3, "above"), (-1, "below")):
            raw = np.uint32(u + d).view(np.float32)
            am = np.float32(raw / np.float32(1.0 / 448.0))
            rows.append(am)
            kinds.append(kind)
    am = np.float32(rows)
    g = np.zeros((am.size, 64), np.float32)
    g[:, 0] = am
    _, s3 = Q.act_quant_tilelang(g, 64, round_scale=True)
    _, s4 = Q.kv_ue8m0_quant(g, 64)
    raw = (np.maximum(am, np.float32(1e-4)) * np.float32(1.0 / 448.0)).astype(np.float32)
    brute = _brute_pow2_ceil(raw)
    np.testing.assert_array_equal(s3[:, 0], brute)
    t_raw = torch.from_numpy(am).clamp(min=1e-12) * (1.0 / 448.0)
    t_ref = torch.exp2(torch.ceil(torch.log2(t_raw.clamp(min=2**-30)))).numpy()
    np.testing.assert_array_equal(s4[:, 0], t_ref)
    kinds = np.array(kinds)
    differ = s3[:, 0] != s4[:, 0]
    assert differ.any()
    # they can only differ on the rows just above a power of two, by a factor 2
    assert not differ[kinds != "above"].any()
    assert np.all(s3[differ, 0] == 2 * s4[differ, 0])
