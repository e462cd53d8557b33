"""Property tests (hypothesis) of the oracle's permutation, routing, index
split and quantization formulas: invariants and closed forms that hold for
every input, drawn beyond the fixed seeds of the other tests.  The GPU
kernels are checked bit for bit against these same oracle functions, so a
property that fails here would fail there."""

from __future__ import annotations

import numpy as np
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import kv as OK
from oracle import moe as OM
from oracle import quant as Q

SETTINGS = settings(max_examples=80, deadline=None, derandomize=True,
                    suppress_health_check=[HealthCheck.too_slow])


@st.composite
def routing_ids(draw):
    E = draw(st.integers(1, 40))
    k = draw(st.integers(1, min(8, E)))
    T = draw(st.integers(0, 30))
    ids = draw(st.lists(st.lists(st.integers(0, E - 1), min_size=k, max_size=k), min_size=T, max_size=T))
    return np.asarray(ids, dtype=np.int64).reshape(T, k), E


@SETTINGS
@given(routing_ids())
def test_permute_is_the_reference_loop_and_a_stable_counting_sort(case):
    """model.py:635-640: experts ascending, slots row-major inside an expert."""
    ids, E = case
    p = OM.permute(ids, E)
    flat = ids.reshape(-1)
    n = flat.size
    np.testing.assert_array_equal(p["sorted_slot"], OM.permute_bruteforce(ids, E))
    assert p["counts"].sum() == n
    np.testing.assert_array_equal(p["counts"], np.bincount(flat, minlength=E)[:E])
    np.testing.assert_array_equal(p["offsets"][1:] - p["offsets"][:-1], p["counts"])
    assert p["offsets"][0] == 0 and p["offsets"][-1] == n
    # a permutation of the slots whose inverse is slot_pos
    np.testing.assert_array_equal(np.sort(p["sorted_slot"]), np.arange(n))
    np.testing.assert_array_equal(p["sorted_slot"][p["slot_pos"]], np.arange(n))
    for e in range(E):
        seg = p["sorted_slot"][p["offsets"][e]:p["offsets"][e + 1]]
        assert np.all(flat[seg] == e)
        assert np.all(np.diff(seg) > 0)  # stable: slot order kept inside an expert


@st.composite
def logits_rows(draw):
    E = draw(st.integers(2, 48))
    k = draw(st.integers(1, min(8, E)))
    T = draw(st.integers(1, 12))
    vals = draw(st.lists(st.floats(-8, 8, width=32), min_size=T * E, max_size=T * E))
    return np.asarray(vals, dtype=np.float32).reshape(T, E), k


@SETTINGS
@given(logits_rows(), st.sampled_from(["softmax", "sigmoid", "sqrtsoftplus"]),
       st.floats(0.5, 3.0, width=32))
def test_route_topk_selects_the_k_largest_scores_ties_to_lower_id(case, score_func, route_scale):
    lg, k = case
    w, ids = OM.route_topk(lg, k, score_func, None, route_scale)
    sc = OM.route_scores(lg, score_func)
    for t in range(lg.shape[0]):
        order = sorted(range(lg.shape[1]), key=lambda e: (-float(sc[t, e]), e))
        assert ids[t].tolist() == order[:k]
    if score_func != "softmax":
        np.testing.assert_allclose(w.sum(-1), route_scale, rtol=1e-5)
    else:
        np.testing.assert_allclose(w, np.take_along_axis(sc, ids, 1) * np.float32(route_scale), rtol=1e-6)


@SETTINGS
@given(st.integers(1, 3), st.integers(1, 4), st.integers(1, 12), st.integers(1, 16), st.data())
def test_split_swa_compress_indices_lengths_and_shift(b, s, k, window, data):
    """dsv4_kv_pack.py:149-175: the first min(window, k) columns are the
    window part, the rest are shifted down by window; -1 marks padding and
    the lengths count the non-negative entries."""
    topk = np.asarray(data.draw(st.lists(st.integers(-1, 500), min_size=b * s * k, max_size=b * s * k)),
                      dtype=np.int32).reshape(b, s, k)
    swa, swa_lens, comp, comp_lens = OK.split_swa_compress_indices(topk, window)
    flat = topk.reshape(b * s, k)
    w = min(window, k)
    np.testing.assert_array_equal(swa, flat[:, :w])
    np.testing.assert_array_equal(swa_lens, (flat[:, :w] >= 0).sum(-1))
    rest = flat[:, w:]
    np.testing.assert_array_equal(comp, np.where(rest >= 0, rest - window, rest).reshape(comp.shape))
    np.testing.assert_array_equal(comp_lens, (rest >= 0).sum(-1))


# bf16 values (the kernels' activation inputs) with a wide exponent range
_bf16 = st.floats(-3.0e4, 3.0e4, width=32).map(lambda v: float(Q.bf16_round(np.float32(v))))


@st.composite
def groups(draw, size):
    vals = draw(st.lists(_bf16, min_size=size, max_size=size))
    return np.asarray(vals, dtype=np.float32).reshape(1, size)


def _e4m3_half_ulp(v):
    """Half the e4m3 spacing at |v| (normals: 2^(e-4); subnormals: 2^-10)."""
    a = np.abs(v).astype(np.float64)
    e = np.floor(np.log2(np.maximum(a, 2.0**-6)))
    return np.where(a < 2.0**-6, 2.0**-10, 2.0 ** (e - 4))


@SETTINGS
@given(groups(128), st.booleans())
def test_per_token_cast_closed_forms(g, ue8m0):
    """utils/math.py:25-37: sf = max(amax, 1e-4)/448 (correctly rounded), or
    the next power of two up; every element dequantizes within half an e4m3
    step (of x / sf, times sf); the amax element lands on +-448 (fp32 scale,
    amax >= 1e-4)."""
    q, sf = Q.per_token_cast_to_fp8(g, ue8m0, 128)
    amax = float(np.max(np.abs(g)))
    want = np.float32(np.float64(max(np.float32(amax), np.float32(1e-4))) / 448.0)
    if ue8m0:
        s = float(sf[0, 0])
        assert s == 2.0 ** np.round(np.log2(s))  # a power of two
        assert float(want) <= s < 2.0 * float(want) or s == float(want)
    else:
        assert sf[0, 0] == want
    s = np.float64(sf[0, 0])
    y = g.astype(np.float64) / s
    deq = Q.e4m3_to_f32(q).astype(np.float64)
    err = np.abs(deq - np.clip(y, -448, 448))
    assert np.all(err <= _e4m3_half_ulp(y) * (1 + 1e-6) + 1e-12)
    if not ue8m0 and amax >= 1e-4:
        i = int(np.argmax(np.abs(g)))
        assert abs(float(Q.e4m3_to_f32(q.reshape(-1)[i:i + 1])[0])) == 448.0


@SETTINGS
@given(groups(128), st.integers(-6, 6))
def test_per_token_cast_commutes_with_powers_of_two(g, j):
    """Scaling a group by 2^j scales its fp32 scale by 2^j and keeps its codes
    (while amax stays above the 1e-4 floor and nothing leaves fp32 range)."""
    amax = float(np.max(np.abs(g)))
    if amax < 1e-4 * 2.0 ** max(0, -j) * 4 or amax * 2.0**j > 1e37:
        return
    q0, s0 = Q.per_token_cast_to_fp8(g, False, 128)
    q1, s1 = Q.per_token_cast_to_fp8((g * np.float32(2.0**j)).astype(np.float32), False, 128)
    np.testing.assert_array_equal(q1, q0)
    assert s1[0, 0] == np.float32(s0[0, 0] * np.float32(2.0**j))


@SETTINGS
@given(groups(64))
def test_kv_ue8m0_scale_is_the_power_of_two_ceiling(g):
    """dsv4_kv_pack.py:78-101: scale = 2^ceil(log2(max(amax/448, 2^-30)))
    brackets raw = max(amax * fp32(1/448), 2^-30): raw <= scale < 2 raw (up
    to the correctly rounded log2 at powers of two), and every element
    quantizes within half an e4m3 step of clamp(x / scale)."""
    q, sc = Q.kv_ue8m0_quant(g, 64)
    amax = np.float32(max(float(np.max(np.abs(g))), 1e-12))
    raw = max(float(np.float32(amax * Q.INV448)), 2.0**-30)
    s = float(sc[0, 0])
    assert s == 2.0 ** np.round(np.log2(s))
    assert raw * (1 - 2.0**-22) <= s < 2.0 * raw * (1 + 2.0**-22)
    y = np.clip(g.astype(np.float64) / s, -448, 448)
    err = np.abs(Q.e4m3_to_f32(q).astype(np.float64) - y)
    assert np.all(err <= _e4m3_half_ulp(y) * (1 + 1e-6) + 1e-12)


def test_e4m3_codes_round_trip():
    """Every finite e4m3 code decodes to a value that encodes back to it (both
    signs; -0 keeps its sign bit); the NaN codes stay NaN."""
    codes = np.arange(256, dtype=np.uint8)
    vals = Q.e4m3_to_f32(codes)
    finite = (codes & 0x7F) != 0x7F
    np.testing.assert_array_equal(Q.f32_to_e4m3(vals[finite]), codes[finite])
    assert np.all(np.isnan(vals[~finite]))
