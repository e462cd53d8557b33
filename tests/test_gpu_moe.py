"""MoE path on the GPU vs the oracle: routing and permutation bit-exact, expert
outputs within the GEMM tolerance, combine bit-exact given the expert rows."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (EDGE_COUNTS_LONG, EDGE_COUNTS_SHORT, assert_gemm_close, bf16_values, f32,
                     ids_with_counts, to_dev_bf16, to_dev_f32, to_dev_fp8, u8)
from oracle import moe as OM
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def zipf_logits(rng, T, E, s=1.1):
    """Router logits whose top-k load follows Zipf(s) over a random expert ranking."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = rng.permutation(E)
    logp = np.log(p)[np.argsort(perm)]
    g = rng.gumbel(size=(T, E))
    return (logp[None, :] + g).astype(np.float32)


def logits_without_near_ties(rng, T, E, k, score_func="softmax", bias=None, min_gap=1e-6,
                             scale=2.0):
    """N(0, scale) router logits, redrawing every row whose k-th and (k+1)-th
    selection values are closer than ``min_gap`` (torch.topk's tie order is
    unspecified, so test data carries no ties)."""
    lg = (rng.standard_normal((T, E)) * scale).astype(np.float32)
    for _ in range(100):
        bad = [t for t in range(T) if OM.topk_margin(lg[t:t + 1], k, score_func, bias) < min_gap]
        if not bad:
            return lg
        lg[bad] = (rng.standard_normal((len(bad), E)) * scale).astype(np.float32)
    raise AssertionError("could not draw tie-free logits")


def table_from(experts, shared, dev):
    from sglang_lite_amd import moe as M

    def ent(e):
        return (to_dev_fp8(e["w1"], dev), to_dev_fp8(e["w3"], dev), to_dev_fp8(e["w2"], dev),
                to_dev_f32(e["s1"], dev), to_dev_f32(e["s3"], dev), to_dev_f32(e["s2"], dev))

    return M.ExpertTable.build([ent(e) for e in experts], ent(shared) if shared else None)


@pytest.mark.parametrize("score_func,use_bias", [("softmax", False), ("sigmoid", True),
                                                 ("sqrtsoftplus", True), ("sqrtsoftplus", False)])
@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (512, 256, 8), (300, 64, 6)])
def test_route_topk(gpu, score_func, use_bias, T, E, k):
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(T + E + k)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if use_bias else None
    logits = logits_without_near_ties(rng, T, E, k, score_func, bias)
    assert OM.topk_margin(logits, k, score_func, bias) >= 1e-6
    w_ref, ids_ref = OM.route_topk(logits, k, score_func, bias, route_scale=1.5)
    w, ids = M.route_topk(to_dev_f32(logits, gpu), k, score_func,
                          to_dev_f32(bias, gpu) if use_bias else None, route_scale=1.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("score_func,use_bias", [("softmax", False), ("sigmoid", True),
                                                 ("sqrtsoftplus", False)])
@pytest.mark.parametrize("E,k", [(256, 8), (200, 16), (8, 8), (70, 3)])
def test_route_topk_exact_ties_go_to_lower_ids(gpu, score_func, use_bias, E, k):
    """Logits on a coarse grid, so most picks tie exactly (-0.0 beside +0.0
    among them): the picks and their order are the oracle's stable descending
    sort, ties to the lower expert id; E = 200 and 70 leave lanes past E."""
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(E * 31 + k)
    T = 300
    logits = (rng.integers(-3, 3, (T, E)) * 0.5).astype(np.float32)
    zeros = logits == 0
    logits[zeros] = np.where(rng.random(int(zeros.sum())) < 0.5, np.float32(-0.0), np.float32(0.0))
    assert np.signbit(logits[zeros]).any() and (~np.signbit(logits[zeros])).any()
    bias = np.zeros(E, np.float32) if use_bias else None
    w_ref, ids_ref = OM.route_topk(logits, k, score_func, bias, route_scale=1.5)
    w, ids = M.route_topk(to_dev_f32(logits, gpu), k, score_func,
                          to_dev_f32(bias, gpu) if use_bias else None, route_scale=1.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("score_func", ["sigmoid", "softmax"])
def test_route_topk_score_ties_from_distinct_logits(gpu, score_func):
    """Distinct logits whose fp32 scores are equal (sigmoid saturates to 1.0
    above 17.5; softmax underflows to 0 far below the row max): the picks
    follow the scores, ties to the lower id, as topk on the scores does
    (model.py:574-579), not the order of the logits."""
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(77)
    T, E, k = 64, 256, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    for t in range(T):
        if score_func == "sigmoid":  # 12 saturated logits, shuffled so that id order != logit order
            cols = rng.choice(E, 12, replace=False)
            logits[t, cols] = rng.uniform(18.0, 30.0, 12).astype(np.float32)
        else:  # three dominant logits, the rest far enough below to underflow
            logits[t] = rng.uniform(-70.0, -60.0, E).astype(np.float32)
            logits[t, rng.choice(E, 3, replace=False)] = [52.0, 51.0, 50.0]
    scores = OM.route_scores(logits, score_func)
    top = -np.sort(-scores, axis=1)
    assert np.all(top[:, k - 1] == top[:, k])  # the k-th pick is tied in every row
    w_ref, ids_ref = OM.route_topk(logits, k, score_func)
    w, ids = M.route_topk(to_dev_f32(logits, gpu), k, score_func)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)


def test_route_topk_matches_torch_topk(gpu):
    """Library routine pin: torch.topk on torch.softmax scores (CPU)."""
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(3)
    logits = zipf_logits(rng, 256, 256)
    assert OM.topk_margin(logits, 8) >= 1e-7, "test data has a near-tie"
    t = torch.from_numpy(logits)
    scores = t.softmax(dim=-1)
    ref_idx = scores.topk(8, dim=-1)[1]
    ref_w = scores.gather(1, ref_idx)
    w, ids = M.route_topk(t.to(gpu), 8)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_idx.numpy())
    np.testing.assert_allclose(w.cpu().numpy(), ref_w.numpy(), rtol=2e-6)


@pytest.mark.parametrize("T,k,E,kind", [(1, 1, 1, "uniform"), (64, 8, 256, "zipf"),
                                        (512, 8, 256, "zipf"), (8192, 8, 256, "uniform"),
                                        (1000, 6, 1024, "uniform"), (333, 2, 8, "one"),
                                        (4096, 8, 256, "zipf"), (2500, 8, 1024, "uniform"),
                                        (16384, 8, 256, "one"), (2049, 8, 16, "uniform")])
def test_permute_bit_exact(gpu, T, k, E, kind):
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(T * k)
    if kind == "zipf":
        ids = np.argsort(-zipf_logits(rng, T, E), axis=1)[:, :k]
    elif kind == "one":
        ids = np.zeros((T, k), np.int64)
        ids[:, 1:] = rng.integers(1, E, (T, k - 1))
    else:
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]) if k <= E else None
    ref = OM.permute(ids, E)
    if T * k <= 4096:
        np.testing.assert_array_equal(ref["sorted_slot"], OM.permute_bruteforce(ids, E))
    counts, offsets, sorted_slot, slot_pos = M.permute(torch.from_numpy(ids).to(gpu), E)
    np.testing.assert_array_equal(counts.cpu().numpy(), ref["counts"])
    np.testing.assert_array_equal(offsets.cpu().numpy(), ref["offsets"])
    np.testing.assert_array_equal(sorted_slot.cpu().numpy(), ref["sorted_slot"])
    np.testing.assert_array_equal(slot_pos.cpu().numpy(), ref["slot_pos"])


def _moe_case(rng, T, H, I, E, k, shared=True, zipf=False):
    x = bf16_values(rng, (T, H))
    logits = zipf_logits(rng, T, E) if zipf else logits_without_near_ties(rng, T, E, k)
    w, ids = OM.route_topk(logits, k)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I) if shared else None
    return x, logits, w, ids, experts, sh


def test_moe_stages_tiny(gpu):
    """Config 1 shapes, stage by stage."""
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(1)
    T, H, I, E, k = 32, 256, 128, 8, 2
    x, logits, w, ids, experts, sh = _moe_case(rng, T, H, I, E, k)
    table = table_from(experts, sh, gpu)
    xd = to_dev_bf16(x, gpu)
    idd = torch.from_numpy(ids).to(gpu)
    wd = to_dev_f32(w, gpu)
    xq, xs = K.act_quant(xd)
    counts, offsets, sorted_slot, _ = M.permute(idd, E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, wd.reshape(-1), table, k)
    out = M.down(hq, hs, offsets, sorted_slot, table, T, k)
    y = M.combine(out, idd, True)
    torch.cuda.synchronize()
    perm = OM.permute(ids, E)
    hq_n, hs_n, out_n = u8(hq), hs.cpu().numpy(), f32(out)
    # per expert: the dequantized h rows and the expert outputs
    for e in range(E):
        rows = perm["sorted_slot"][perm["offsets"][e]:perm["offsets"][e + 1]]
        if rows.size == 0:
            continue
        tok, top = rows // k, rows % k
        tr = {}
        ref_out = OM.expert_forward(x[tok], experts[e], w[tok, top][:, None], trace=tr)
        p0, p1 = perm["offsets"][e], perm["offsets"][e + 1]
        h_dev = Q.dequant_rows(hq_n[p0:p1], hs_n[p0:p1])
        assert_gemm_close(h_dev, Q.dequant_rows(tr["hq"], tr["hs"]), f"h expert {e}")
        assert_gemm_close(out_n[tok, top], ref_out, f"out expert {e}")
    tr = {}
    ref_sh = OM.expert_forward(x, sh, None, trace=tr)
    assert_gemm_close(out_n[:, k], ref_sh, "shared")
    # combine is exact given the device's expert rows
    order = np.argsort(ids, axis=1, kind="stable")
    acc = np.zeros((T, H), np.float32)
    for jj in range(k):
        acc = (acc + np.take_along_axis(out_n[:, :k], order[:, jj][:, None, None], 1)[:, 0]).astype(np.float32)
    acc = (acc + out_n[:, k]).astype(np.float32)
    np.testing.assert_array_equal(f32(y).view(np.uint32), Q.bf16_round(acc).view(np.uint32))
    # the whole layer against the oracle
    y_ref = OM.moe_forward(x, ids, w, experts, sh)
    assert_gemm_close(f32(y), y_ref, "moe tiny")


@pytest.mark.parametrize("T,H,I,E,k,shared,lim,zipf", [
    (32, 256, 128, 8, 2, True, 0.0, False),
    (100, 512, 256, 16, 4, True, 10.0, False),
    (64, 1024, 512, 32, 8, True, 0.0, True),
    (7, 512, 384, 5, 3, False, 0.5, False),
    # >= 64 rows per expert on average: the pipelined 128 x 256 kernels, with
    # five (gate/up, K = 640) and four (down, K = 512) K stages, a partial
    # last column tile in down (N = 640) whose second scale block is clamped,
    # and skewed routing (empty and one-row experts beside full tiles)
    (300, 640, 512, 12, 3, True, 7.0, True),
])
def test_moe_forward_matches_oracle(gpu, T, H, I, E, k, shared, lim, zipf):
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(T * H + E)
    x, logits, w, ids, experts, sh = _moe_case(rng, T, H, I, E, k, shared, zipf)
    table = table_from(experts, sh, gpu)
    y = M.moe_forward(to_dev_bf16(x, gpu), torch.from_numpy(ids).to(gpu), to_dev_f32(w, gpu),
                      table, swiglu_limit=lim)
    y_ref = OM.moe_forward(x, ids, w, experts, sh, swiglu_limit=lim)
    assert_gemm_close(f32(y), y_ref, f"moe T={T} H={H} I={I} E={E} k={k}")


@pytest.mark.parametrize("counts", [EDGE_COUNTS_SHORT, EDGE_COUNTS_LONG], ids=["rows14", "rows42"])
def test_moe_forward_group_sizes_at_block_edges(gpu, counts):
    """Decode tiles compute only the 16-row blocks a group fills (one or two
    of them): every group size at a block edge against the oracle."""
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(sum(counts))
    H, I, E, k = 256, 256, len(counts), 2
    ids = ids_with_counts(rng, counts, k)
    T = ids.shape[0]
    print(f"moe block edges T={T} E={E} rows/expert={T * k // E}", flush=True)
    x = bf16_values(rng, (T, H))
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    table = table_from(experts, sh, gpu)
    y = M.moe_forward(to_dev_bf16(x, gpu), torch.from_numpy(ids).to(gpu), to_dev_f32(w, gpu), table)
    y_ref = OM.moe_forward(x, ids, w, experts, sh)
    assert_gemm_close(f32(y), y_ref, f"moe block edges T={T}")


def test_moe_forward_big_rows_tile_path(gpu):
    """Enough rows per expert (>= 64) to take the 128-row tile configuration."""
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(5)
    T, H, I, E, k = 512, 512, 256, 8, 2
    x, logits, w, ids, experts, sh = _moe_case(rng, T, H, I, E, k)
    table = table_from(experts, sh, gpu)
    y = M.moe_forward(to_dev_bf16(x, gpu), torch.from_numpy(ids).to(gpu), to_dev_f32(w, gpu), table)
    y_ref = OM.moe_forward(x, ids, w, experts, sh)
    assert_gemm_close(f32(y), y_ref, "moe big tiles")


def test_moe_forward_deterministic_and_repeatable(gpu):
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(9)
    T, H, I, E, k = 200, 512, 256, 16, 4
    x, logits, w, ids, experts, sh = _moe_case(rng, T, H, I, E, k)
    table = table_from(experts, sh, gpu)
    args = (to_dev_bf16(x, gpu), torch.from_numpy(ids).to(gpu), to_dev_f32(w, gpu), table)
    ws = M.MoEWorkspace()
    y1 = u8(M.moe_forward(*args, workspace=ws))
    y2 = u8(M.moe_forward(*args, workspace=ws))
    np.testing.assert_array_equal(y1, y2)


def test_tiny_moe_golden_fixture(gpu):
    """The committed tiny-MoE fixture (tests/golden/tiny_moe_seed1.npz):
    routing, permutation and activation quant bit-exact against the stored
    bytes; the requantized gate/up rows and the layer output within the GEMM
    tolerance."""
    import os
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import make_tiny_moe as G
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    gold = dict(np.load(G.PATH))
    inp = G.make_inputs()
    assert bytes(gold["weights_sha256"]).decode() == G.weights_digest(inp)
    table = table_from(inp["experts"], inp["shared"], gpu)
    w, ids = M.route_topk(to_dev_f32(gold["logits"], gpu), G.K_TOP)
    xd = to_dev_bf16(inp["x"], gpu)
    xq, xs = K.act_quant(xd)
    counts, offsets, sorted_slot, slot_pos = M.permute(ids, G.E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), table, G.K_TOP)
    y = M.moe_forward(xd, ids, w, table)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy().astype(np.int32), gold["ids"])
    np.testing.assert_allclose(f32(w), gold["route_w"], rtol=1e-6, atol=1e-7)
    for name, dev in (("counts", counts), ("offsets", offsets), ("sorted_slot", sorted_slot),
                      ("slot_pos", slot_pos)):
        np.testing.assert_array_equal(dev.cpu().numpy(), gold[name], err_msg=name)
    np.testing.assert_array_equal(u8(xq), gold["xq"])
    np.testing.assert_array_equal(f32(xs).view(np.uint32), gold["xs"].view(np.uint32))
    assert_gemm_close(Q.dequant_rows(u8(hq), f32(hs)), Q.dequant_rows(gold["hq"], gold["hs"]),
                      "golden h")
    y_ref = (gold["y_bf16_bits"].astype(np.uint32) << 16).view(np.float32)
    assert_gemm_close(f32(y), y_ref, "golden y")


def _gate_case(rng, T, H, E, scale=None):
    x = bf16_values(rng, (T, H))
    W = bf16_values(rng, (E, H), scale=(scale or H ** -0.5))
    return x, W


@pytest.mark.parametrize("T,H,E,k,score_func,use_bias", [
    (64, 4096, 256, 8, "sqrtsoftplus", True),
    (300, 1024, 64, 6, "softmax", False),
    (32, 256, 8, 2, "sigmoid", True),
    (1000, 512, 256, 8, "sqrtsoftplus", False),
    (7, 4096, 256, 8, "softmax", True),
    # 2 x 2 wavefronts over 64-deep stages
    (4100, 1024, 256, 8, "sqrtsoftplus", True),  # 32 x 128 tiles, a ragged last tile
    (8200, 512, 256, 8, "sqrtsoftplus", False),  # 64 x 128 tiles
    (8200, 192, 256, 8, "sigmoid", True),  # 64 x 128 tiles, H % 128 == 64
    (4100, 320, 256, 8, "sigmoid", True),  # 32 x 128 tiles, H % 128 == 64
    (2050, 320, 256, 8, "sqrtsoftplus", False),  # 32 x 64 tiles (H % 128 == 64)
    (513, 64, 72, 4, "sigmoid", True),  # 32 x 32 tiles (H % 128 == 64), one stage
    # K split over the wavefronts, 128-deep stages (also (300, 1024, ...) and (1000, 512, ...) above)
    (2050, 1024, 256, 8, "sigmoid", True),  # 32 x 64 tiles
    (600, 256, 200, 8, "sqrtsoftplus", True),  # 32 x 32 tiles, E past the last tile, 2 stages
    (400, 96, 64, 4, "softmax", False),  # H % 64 != 0: the register-loaded kernel
])
def test_gate_kernel_matches_oracle(gpu, T, H, E, k, score_func, use_bias):
    """model.py:564-584 from the hidden states: the bf16-MFMA projection within
    the fp32 summation bound of the exact logits, the routing of those logits
    exact, and equal to the oracle's routing of the exact logits where no
    near-tie lies within the projection's error or the scores' fp32 rounding."""
    from sglang_lite_amd import moe as M

    print(f"gate T={T} H={H} E={E} k={k} {score_func} bias={use_bias}", flush=True)
    rng = np.random.default_rng(T + H + E)
    x, W = _gate_case(rng, T, H, E)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if use_bias else None
    lg = torch.empty(T, E, dtype=torch.float32, device=gpu)
    w, ids = M.gate(to_dev_bf16(x, gpu), to_dev_bf16(W, gpu), k, score_func,
                    to_dev_f32(bias, gpu) if use_bias else None, 1.5, logits=lg)
    torch.cuda.synchronize()
    exact = OM.router_logits(x, W)
    mag = (np.abs(x).astype(np.float64) @ np.abs(W).astype(np.float64).T)
    got = f32(lg)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= 2.0 ** -21 * mag + 1e-30)
    w_dev, ids_dev = OM.route_topk(got, k, score_func, bias, 1.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_dev)
    np.testing.assert_allclose(f32(w), w_dev, rtol=2e-6, atol=1e-7)
    w_ex, ids_ex = OM.route_topk(exact, k, score_func, bias, 1.5)
    err = float(np.max(np.abs(got.astype(np.float64) - exact)))
    # ids hold the picks in order, so a near-tie is any adjacent pair of the
    # k + 1 largest selection values closer than the projection's error or
    # the fp32 rounding of the scores and their sum with the bias (4 ulp of
    # the largest: 2.5e-7 of it)
    sel_ex = OM.route_scores(exact, score_func).astype(np.float64)
    if bias is not None:
        sel_ex = sel_ex + bias
    top = -np.sort(-sel_ex, axis=1)[:, :min(k + 1, E)]
    floor = 2.5e-7 * np.abs(top).max(axis=1)
    ok = np.min(top[:, :-1] - top[:, 1:], axis=1) > 8 * err + floor
    assert ok.mean() > 0.9
    np.testing.assert_array_equal(ids.cpu().numpy()[ok], ids_ex[ok])


@pytest.mark.parametrize("ids64", [False, True])
def test_gate_hash_routing(gpu, ids64):
    """Hash-routed layers (model.py:576-577): ids = tid2eid[input_ids] exactly,
    weights = the sqrtsoftplus scores there, renormalised, times route_scale."""
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(55 + ids64)
    T, H, E, k, V = 100, 512, 64, 6, 1000
    x, W = _gate_case(rng, T, H, E)
    tid2eid = np.stack([rng.permutation(E)[:k] for _ in range(V)]).astype(np.int32)
    input_ids = rng.integers(0, V, T).astype(np.int64 if ids64 else np.int32)
    lg = torch.empty(T, E, dtype=torch.float32, device=gpu)
    w, ids = M.gate(to_dev_bf16(x, gpu), to_dev_bf16(W, gpu), k, "sqrtsoftplus", None, 1.5,
                    tid2eid=torch.from_numpy(tid2eid).to(gpu),
                    input_ids=torch.from_numpy(input_ids).to(gpu), logits=lg)
    np.testing.assert_array_equal(ids.cpu().numpy(), tid2eid[input_ids])
    w_ref, ids_ref = OM.route_hash(f32(lg), tid2eid, input_ids, k, "sqrtsoftplus", 1.5)
    np.testing.assert_array_equal(ids_ref, tid2eid[input_ids])
    np.testing.assert_allclose(f32(w), w_ref, rtol=2e-6, atol=1e-7)
