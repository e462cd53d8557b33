"""Shared test helpers: numpy <-> device tensors and the GEMM tolerance."""

from __future__ import annotations

import numpy as np
import torch

# GEMM outputs (bf16) against the dequantize-to-fp32 reference: rel-L2 <= 1e-2
# and |out - ref| <= 2e-2 + 2^-7 * |ref| elementwise (2e-2 absolute plus one
# bf16 ulp of the reference, since a bf16 output cannot hold 2e-2 absolute
# accuracy above |C| = 8).
REL_L2 = 1e-2
ATOL = 2e-2
RTOL_BF16 = 2.0 ** -7


def to_dev_u8(a: np.ndarray, dev, dtype=torch.uint8) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.uint8))
    return t.view(dtype).to(dev) if dtype != torch.uint8 else t.to(dev)


def to_dev_fp8(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).view(torch.float8_e4m3fn).to(dev)


def to_dev_f32(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def to_dev_bf16(a: np.ndarray, dev) -> torch.Tensor:
    """float32 array holding bf16 values -> exact bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(dev)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).cpu().numpy()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def assert_gemm_close(out: np.ndarray, ref: np.ndarray, what: str = "gemm") -> float:
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    denom = max(np.linalg.norm(ref), 1e-30)
    rel = float(np.linalg.norm(out - ref) / denom)
    err = np.abs(out - ref)
    bound = ATOL + RTOL_BF16 * np.abs(ref)
    bad = int(np.sum(err > bound))
    assert rel <= REL_L2, f"{what}: rel-L2 {rel:.3e} > {REL_L2}"
    assert bad == 0, f"{what}: {bad} elements beyond 2e-2 + 2^-7|ref| (max err {err.max():.3e})"
    return rel


def bf16_values(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    from oracle.quant import bf16_round

    return bf16_round((rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32))


def ref_moe_case(name: str):
    """Inputs of a reference-generated MoE golden case (tests/golden/
    ref_moe_<name>.npz) rebuilt with the oracle: FP8 weights quantized by the
    oracle's per_block_cast_to_fp8 (the fixture's digest of the reference's
    bytes checks them), FP4 weights as drawn.  Returns (case dict, fixture
    dict, experts, shared, digest) with oracle-format expert dicts; e8m0
    scales are kept as bytes under ``s*`` and decoded under ``s*_f32``."""
    import os
    import sys

    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    if here not in sys.path:
        sys.path.insert(0, here)
    import ref_moe_cases as C
    from oracle import fp4 as F4
    from oracle import quant as Q

    c = C.CASES[name]
    gold = dict(np.load(C.path(name)))
    inp = C.draw(name)

    def fp8(e):
        out = {}
        for nm in ("1", "3", "2"):
            q, s = Q.per_block_cast_to_fp8(e["w" + nm], use_ue8m0=c["ue8m0"])
            out["w" + nm] = q
            out["s" + nm] = Q.e8m0_byte(s) if c["ue8m0"] else s
        return out

    def fp4(e):
        out = {"fmt": "fp4"}
        out.update(e)
        return out

    stored = [fp4(e) if c["fp4"] else fp8(e) for e in inp["experts"]]
    shared = fp8(inp["shared"])
    digest = C.digest(stored, shared)

    def oracle_view(e):
        if e.get("fmt") == "fp4":
            return e
        o = dict(e)
        for nm in ("1", "3", "2"):
            o["s" + nm] = F4.e8m0_to_f32(e["s" + nm]) if c["ue8m0"] else e["s" + nm]
        return o

    return (c, gold, inp, [oracle_view(e) for e in stored], oracle_view(shared), stored, shared,
            digest)


def gemm_err_stats(out: np.ndarray, ref: np.ndarray, atol_scale: float = 1.0) -> dict:
    """Error of ``out`` against ``ref`` in units of the GEMM elementwise bound
    (its absolute term times ``atol_scale``)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    r = np.abs(out - ref) / (ATOL * atol_scale + RTOL_BF16 * np.abs(ref))
    return {"rel_l2": float(np.linalg.norm(out - ref) / max(np.linalg.norm(ref), 1e-30)),
            "max_ratio": float(r.max()), "n_over": int(np.sum(r > 1)), "n": int(r.size),
            "p999_ratio": float(np.quantile(r, 0.999))}


def assert_layer_close(out: np.ndarray, ref: np.ndarray, what: str = "layer",
                       tail: float = 5e-4) -> dict:
    """A whole MoE layer against the oracle's layer.  The layer requantizes
    twice inside (x, and h between gate/up and down): where the device's bf16
    h and the oracle's differ by one ulp across an e4m3 rounding boundary, or
    move a 128-group's amax, the requantized codes move by one e4m3 step
    (2^-3 relative) and that step reaches the output through w2 -- a tail the
    single-GEMM bound does not model (each GEMM is held to that bound on its
    own inputs by the stage tests).  Bound: rel-L2 <= 1e-2; the GEMM
    elementwise bound for all but a fraction ``tail`` of the elements, and
    twice the bound for every element.  The bound's 2e-2 absolute term is
    sized for unit-scale outputs (N(0, 1) activations through N(0, 0.02)
    weights, the configurations' data); for a layer whose outputs are larger
    it is scaled by the reference output's RMS."""
    rms = float(np.sqrt(np.mean(np.square(np.asarray(ref, dtype=np.float64))))) if np.size(ref) else 0.0
    st = gemm_err_stats(out, ref, max(1.0, rms))
    st["ref_rms"] = rms
    print(f"{what}: {st}", flush=True)
    assert np.all(np.isfinite(np.asarray(out, dtype=np.float64))), f"{what}: non-finite output"
    assert st["rel_l2"] <= REL_L2, f"{what}: rel-L2 {st['rel_l2']:.3e} > {REL_L2}"
    assert st["n_over"] <= tail * st["n"], f"{what}: {st['n_over']} of {st['n']} beyond the bound"
    assert st["max_ratio"] <= 2.0, f"{what}: an element at {st['max_ratio']:.2f}x the bound"
    return st


def assert_requant_close(q_dev: np.ndarray, s_dev: np.ndarray, q_ref: np.ndarray,
                         s_ref: np.ndarray, what: str = "requant", max_diff: float = 0.01,
                         pow2: bool = False) -> dict:
    """1x128 FP8-requantized rows of a GEMM epilogue (the gate/up kernel's h)
    against the oracle's requantization of its own h.  The two h agree to
    rounding (bf16 ulps), so their quantizations agree except where a value
    straddles an e4m3 rounding boundary or a group's amax moves by an ulp:
    bytes equal for all but ``max_diff`` of the elements, scales within
    2^-6 relative, rel-L2 of the dequantized rows <= 1e-2, and every
    dequantized pair within the sum of the two quantization errors and the
    h difference: h = bf16(w silu(g) u) of bf16 g, u differs by at most two
    bf16 ulps (2^-6 |h|) between the two, and each quantization errs by at
    most half an e4m3 step (2^-4 |h|, or 2^-10 of the scale below the
    normal range), so |d| <= (2^-3 + 2^-6)(1 + 2^-4) max(|dev|, |ref|) +
    2^-9 max(scale), plus 2^-14 of the group's amax (448 scale): the MFMA
    forms each 128-deep fp8 partial to about 1e-5 of the sum of its
    |products| (not an IEEE fp32 sum), so a gate or up output near zero --
    and the h value made from it, far below its group's amax -- carries an
    absolute error that no relative bound covers.

    ``pow2``: power-of-two scales (the *_UE8M0 modes), where an amax ulp at a
    binade edge moves a group's scale by a factor of two: every scale ratio
    is then 1/2, 1 or 2, and at most ``max_diff`` of the groups move (the
    per-value bound above holds either way)."""
    from oracle.quant import dequant_rows

    q_dev, q_ref = np.asarray(q_dev, np.uint8), np.asarray(q_ref, np.uint8)
    s_dev, s_ref = np.asarray(s_dev, np.float32), np.asarray(s_ref, np.float32)
    dd = dequant_rows(q_dev, s_dev).astype(np.float64)
    dr = dequant_rows(q_ref, s_ref).astype(np.float64)
    frac = float(np.mean(q_dev != q_ref))
    ratio = s_dev.astype(np.float64) / s_ref if s_ref.size else np.ones(1)
    if pow2:
        assert np.all(np.isin(ratio, (0.5, 1.0, 2.0))), f"{what}: scale ratios {np.unique(ratio)[:8]}"
        moved = float(np.mean(ratio != 1.0))
        assert moved <= max_diff, f"{what}: {moved:.4f} of the groups changed binade"
        ratio = np.ones(1)
    srel = float(np.max(np.abs(ratio - 1.0)))
    smax = np.repeat(np.maximum(s_dev, s_ref).astype(np.float64), 128, axis=-1)
    mag = np.maximum(np.abs(dd), np.abs(dr))
    step = (2.0 ** -3 + 2.0 ** -6) * (1 + 2.0 ** -4) * mag + (2.0 ** -9 + 448.0 * 2.0 ** -14) * smax
    over = int(np.sum(np.abs(dd - dr) > step))
    rel = float(np.linalg.norm(dd - dr) / max(np.linalg.norm(dr), 1e-30))
    st = {"byte_diff": frac, "scale_rel": srel, "over_step": over, "rel_l2": rel}
    if over:
        bad = np.argwhere(np.abs(dd - dr) > step)[:4]
        sd = np.repeat(s_dev, 128, axis=-1)
        sr = np.repeat(s_ref, 128, axis=-1)
        st["worst"] = [(tuple(int(v) for v in i), float(dd[tuple(i)]), float(dr[tuple(i)]),
                        int(q_dev[tuple(i)]), int(q_ref[tuple(i)]), float(sd[tuple(i)]),
                        float(sr[tuple(i)])) for i in bad]
    assert frac <= max_diff, f"{what}: {frac:.4f} of the bytes differ ({st})"
    assert srel <= 2.0 ** -6, f"{what}: scales differ by {srel:.3e} ({st})"
    assert over == 0, f"{what}: {over} values beyond the requantization bound ({st})"
    assert rel <= REL_L2, f"{what}: rel-L2 {rel:.3e} ({st})"
    return st


def ids_with_counts(rng, counts, k):
    """[T, k] expert ids in which expert e appears exactly counts[e] times, k
    distinct experts per token (each count at most T), tokens shuffled."""
    pool = np.repeat(np.arange(len(counts)), counts)
    assert pool.size % k == 0
    T = pool.size // k
    assert max(counts) <= T
    ids = pool.reshape(k, T).T  # token t: pool[t], pool[t + T], ... (distinct: runs are <= T long)
    return np.ascontiguousarray(ids[rng.permutation(T)]).astype(np.int32)


# group sizes on both sides of every 16-row block edge of a 32-row decode
# tile, in a group's only tile and in its last one; 16 experts, k = 2: 228
# and 674 slots (14 and 42 rows per expert on average), plus the shared
# expert's T rows
EDGE_COUNTS_SHORT = [1, 15, 16, 17, 31, 32, 33, 0, 47, 2, 3, 4, 5, 6, 7, 9]
EDGE_COUNTS_LONG = [1, 15, 16, 17, 31, 32, 33, 47, 48, 49, 63, 64, 65, 0, 96, 97]


def assert_e4m3_equal_nan_signless(got: np.ndarray, ref: np.ndarray, what: str = "e4m3") -> None:
    """e4m3 bytes equal, except that two NaN codes (S.1111.111) may differ in
    sign: a NaN's sign is not fixed by the reference's arithmetic (x86 numpy's
    Inf * 0 is a negative NaN, the GPU's a positive one)."""
    got = np.asarray(got, np.uint8)
    ref = np.asarray(ref, np.uint8)
    both_nan = ((got & 0x7F) == 0x7F) & ((ref & 0x7F) == 0x7F)
    bad = (got != ref) & ~both_nan
    assert not bad.any(), f"{what}: {int(bad.sum())} bytes differ, first at {np.argwhere(bad)[:4].tolist()}"


def nan_inf_rows(rng, cols: int) -> np.ndarray:
    """Six bf16-exact rows with NaN / Inf elements: a NaN, +Inf, -Inf, NaN in
    an all-zero row, +Inf beside NaN in one group, and a plain row."""
    x = bf16_values(rng, (6, cols))
    x[0, 3] = np.nan
    x[1, 70] = np.inf
    x[2, cols - 56] = -np.inf
    x[3, :] = 0.0
    x[3, 129] = np.nan
    x[4, 10] = np.inf
    x[4, 11] = np.nan
    return x

