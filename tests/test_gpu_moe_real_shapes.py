"""The MoE layer and the dense GEMM at the benchmarked shapes, against the oracle.

Expert shapes of the decode and prefill workloads: hidden 4096, expert
intermediate 2048, 256 routed experts top-8 plus one shared expert, FP8 e4m3
weights N(0, 0.02) with fp32 128x128 block scales.  Weights are drawn on the
device from a seeded generator and quantized by the library's weight-quant
kernel (bit-exact against the oracle in test_gpu_quant.py); the oracle reads
the same bytes back.

* Decode, T = 64 and 256 with Zipf(1.1) expert load: the whole layer
  against ``oracle.moe.moe_forward`` (every touched expert).
* Decode T = 512 (Zipf) and prefill T = 8192 (uniform logits): routing,
  permutation and the combine (given the device's expert rows) bit-exact at
  full size; for the hottest and the coldest touched expert, a one-row
  expert when there is one, and the shared expert's first 256 rows: the
  gate/up rows (requantized h) against the oracle's requantized h (equal
  bytes but for one-step rounding flips), the down rows against the
  dequantize-to-fp32 product of the device's own h (the GEMM bound) and
  against ``oracle.moe.expert_forward`` (the layer bound).

Tolerances: a single GEMM on given operands is held to rel-L2 <= 1e-2 and
|d| <= 2e-2 + 2^-7 |ref| per element; results that pass through an FP8
requantization (h, and so the layer) use ``assert_requant_close`` /
``assert_layer_close`` of tests/helpers.py, which allow the one-step e4m3
flips a bf16-ulp difference produces at a rounding boundary.
* Dense FP8 GEMM M = 1024 and 4096 at N = 4096, K = 7168 against the
  dequantize-to-fp32 product.
* FP4 routed experts (the reference's live format) at decode T = 64: the
  whole layer against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (assert_gemm_close, assert_layer_close, assert_requant_close, bf16_values, f32,
                     gemm_err_stats, to_dev_bf16, to_dev_f32, u8)
from oracle import fp4 as F4
from oracle import moe as OM
from oracle import quant as Q

pytestmark = pytest.mark.gpu

H, I, E, K_TOP = 4096, 2048, 256, 8


def zipf_logits(rng, T, s=1.1):
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = rng.permutation(E)
    logp = np.log(p)[np.argsort(perm)]
    return (logp[None, :] + rng.gumbel(size=(T, E))).astype(np.float32)


class DeviceExperts:
    """257 FP8 experts on the device (256 routed + shared) and their host
    bytes on demand, in the oracle's dict format."""

    def __init__(self, dev, seed=7):
        from sglang_lite_amd import kernel as K
        from sglang_lite_amd import moe as M

        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        n = E + 1
        self.w13 = torch.empty(n, 2, I, H, dtype=torch.float8_e4m3fn, device=dev)
        self.s13 = torch.empty(n, 2, I // 128, H // 128, dtype=torch.float32, device=dev)
        self.w2 = torch.empty(n, H, I, dtype=torch.float8_e4m3fn, device=dev)
        self.s2 = torch.empty(n, H // 128, I // 128, dtype=torch.float32, device=dev)
        for e in range(n):
            for j in range(2):
                q, s = K.per_block_cast_to_fp8(torch.randn(I, H, generator=g, device=dev) * 0.02, False)
                self.w13[e, j].copy_(q)
                self.s13[e, j].copy_(s)
            q, s = K.per_block_cast_to_fp8(torch.randn(H, I, generator=g, device=dev) * 0.02, False)
            self.w2[e].copy_(q)
            self.s2[e].copy_(s)
        ent = [(self.w13[e, 0], self.w13[e, 1], self.w2[e], self.s13[e, 0], self.s13[e, 1], self.s2[e])
               for e in range(n)]
        self.table = M.ExpertTable.build(ent[:E], ent[E])
        self.cache = {}

    def host(self, e):
        if e == "shared":
            e = E
        if e not in self.cache:
            self.cache[e] = {"w1": u8(self.w13[e, 0]), "w3": u8(self.w13[e, 1]), "w2": u8(self.w2[e]),
                             "s1": f32(self.s13[e, 0]), "s3": f32(self.s13[e, 1]), "s2": f32(self.s2[e])}
        return self.cache[e]

    def __getitem__(self, e):
        return self.host(int(e))


@pytest.fixture(scope="module")
def experts(gpu):
    ex = DeviceExperts(gpu)
    torch.cuda.synchronize()
    yield ex
    ex.cache.clear()


def _untie(rng, logits, draw, min_gap=1e-6):
    """Redraw every row whose k-th and (k+1)-th softmax scores are within
    ``min_gap`` (torch.topk's order of ties is unspecified)."""
    for _ in range(50):
        sc = np.sort(OM.route_scores(logits, "softmax").astype(np.float64), axis=1)[:, ::-1]
        bad = (sc[:, K_TOP - 1] - sc[:, K_TOP]) <= min_gap
        if not bad.any():
            return logits
        logits[bad] = draw(int(bad.sum()))
    raise AssertionError("could not draw tie-free logits")


def _route(gpu, logits):
    from sglang_lite_amd import moe as M

    w, ids = M.route_topk(to_dev_f32(logits, gpu), K_TOP)
    w_ref, ids_ref = OM.route_topk(logits, K_TOP)
    assert OM.topk_margin(logits, K_TOP) > 1e-6, "test data has a near-tie"
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(f32(w), w_ref, rtol=2e-6, atol=1e-7)
    return w, ids, w_ref, ids_ref


@pytest.mark.parametrize("T", [64, 256])
def test_decode_zipf_layer_matches_oracle(gpu, experts, T):
    """The whole layer against the oracle's layer (every touched expert), and
    each touched expert's down GEMM on the device's own requantized h rows
    against the dequantize-to-fp32 product at the single-GEMM bound (decode
    batches of 64 and 256 tokens, Zipf(1.1) expert load)."""
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    print(f"decode T={T} zipf, full layer", flush=True)
    rng = np.random.default_rng(T)
    x = bf16_values(rng, (T, H))
    w, ids, w_ref, ids_ref = _route(gpu, _untie(rng, zipf_logits(rng, T), lambda n: zipf_logits(rng, n)))
    xd = to_dev_bf16(x, gpu)
    y = M.moe_forward(xd, ids, w, experts.table)
    xq, xs = K.act_quant(xd)
    counts, offsets, sorted_slot, _ = M.permute(ids, E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), experts.table, K_TOP)
    out = M.down(hq, hs, offsets, sorted_slot, experts.table, T, K_TOP)
    torch.cuda.synchronize()
    touched = np.unique(ids_ref).size
    assert touched > (100 if T == 64 else 200), touched
    for e in np.unique(ids_ref).tolist():
        experts.host(e)  # host bytes first: the oracle's workers only read them
    y_ref = OM.moe_forward(x, ids_ref, w_ref, experts, experts.host("shared"), workers=8)
    assert_layer_close(f32(y), y_ref, f"moe decode T={T} ({touched} experts)")
    perm = OM.permute(ids_ref, E)
    hq_n, hs_n, out_n = u8(hq), f32(hs), f32(out)
    worst = 0.0
    for e in np.unique(ids_ref).tolist() + ["shared"]:
        if e == "shared":
            p0, p1 = T * K_TOP, T * K_TOP + T
            tok, top = np.arange(T), np.full(T, K_TOP)
        else:
            p0, p1 = perm["offsets"][e], perm["offsets"][e + 1]
            sl = perm["sorted_slot"][p0:p1]
            tok, top = sl // K_TOP, sl % K_TOP
        ex = experts.host(e) if e == "shared" else experts[e]
        ref = OM.fp8_gemm(hq_n[p0:p1], hs_n[p0:p1], ex["w2"], ex["s2"])
        worst = max(worst, gemm_err_stats(out_n[tok, top], ref)["max_ratio"])
        assert_gemm_close(out_n[tok, top], ref, f"down expert {e} on the device's h")
    print(f"down GEMMs on the device's h: worst element at {worst:.3f}x the bound", flush=True)
    experts.cache.clear()


@pytest.mark.parametrize("T,kind", [(512, "zipf"), (8192, "uniform")])
def test_layer_stages_at_full_size(gpu, experts, T, kind):
    """Integer stages bit-exact at full size; expert rows for a sample of
    experts within the GEMM tolerance; the combine exact given the rows."""
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    print(f"layer stages T={T} {kind}", flush=True)
    rng = np.random.default_rng(T)
    x = bf16_values(rng, (T, H))
    draw = (lambda n: zipf_logits(rng, n)) if kind == "zipf" else \
        (lambda n: rng.standard_normal((n, E)).astype(np.float32))
    logits = _untie(rng, draw(T), draw)
    w, ids, w_ref, ids_ref = _route(gpu, logits)
    xd = to_dev_bf16(x, gpu)
    xq, xs = K.act_quant(xd)
    counts, offsets, sorted_slot, slot_pos = M.permute(ids, E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), experts.table, K_TOP)
    out = M.down(hq, hs, offsets, sorted_slot, experts.table, T, K_TOP)
    y = M.combine(out, ids, True)
    y_layer = M.moe_forward(xd, ids, w, experts.table)
    torch.cuda.synchronize()
    perm = OM.permute(ids_ref, E)
    for name, dev in (("counts", counts), ("offsets", offsets), ("sorted_slot", sorted_slot),
                      ("slot_pos", slot_pos)):
        np.testing.assert_array_equal(dev.cpu().numpy(), perm[name], err_msg=name)
    np.testing.assert_array_equal(u8(y), u8(y_layer))  # the one-call layer = the stages
    # the activation quant bytes of a row sample (the full quant is pinned in test_gpu_quant)
    xq_n, xs_n = u8(xq), f32(xs)
    rows = rng.choice(T, 32, replace=False)
    q_ref, s_ref = Q.scale_mode_quant(x[rows], 0, 128)
    np.testing.assert_array_equal(xq_n[rows], q_ref)
    np.testing.assert_array_equal(xs_n[rows].view(np.uint32), s_ref.view(np.uint32))
    # expert rows: hottest, coldest touched, a one-row expert, shared (first 256 rows)
    cnt = perm["counts"]
    nz = np.nonzero(cnt)[0]
    sample = {int(nz[np.argmax(cnt[nz])]), int(nz[np.argmin(cnt[nz])])}
    ones = np.nonzero(cnt == 1)[0]
    if ones.size:
        sample.add(int(ones[0]))
    hq_n, hs_n, out_n = u8(hq), f32(hs), f32(out)
    for e in sorted(sample):
        p0, p1 = perm["offsets"][e], perm["offsets"][e + 1]
        sl = perm["sorted_slot"][p0:p1]
        tok, top = sl // K_TOP, sl % K_TOP
        tr = {}
        ref = OM.expert_forward(x[tok], experts[e], w_ref[tok, top][:, None], trace=tr)
        assert_requant_close(hq_n[p0:p1], hs_n[p0:p1], tr["hq"], tr["hs"], f"h expert {e} ({p1 - p0} rows)")
        ex = experts[e]
        assert_gemm_close(out_n[tok, top], OM.fp8_gemm(hq_n[p0:p1], hs_n[p0:p1], ex["w2"], ex["s2"]),
                          f"down expert {e} on the device's h ({p1 - p0} rows)")
        assert_layer_close(out_n[tok, top], ref, f"expert {e} vs the oracle's expert")
    P = T * K_TOP
    n_sh = min(T, 256)
    tr = {}
    ref = OM.expert_forward(x[:n_sh], experts.host("shared"), None, trace=tr)
    assert_requant_close(hq_n[P:P + n_sh], hs_n[P:P + n_sh], tr["hq"], tr["hs"], "h shared")
    exs = experts.host("shared")
    assert_gemm_close(out_n[:n_sh, K_TOP], OM.fp8_gemm(hq_n[P:P + n_sh], hs_n[P:P + n_sh], exs["w2"],
                                                        exs["s2"]), "down shared on the device's h")
    assert_layer_close(out_n[:n_sh, K_TOP], ref, "shared vs the oracle's expert")
    # the combine is exact given the device's expert rows: fp32 sum in
    # ascending expert id, then the shared row, bf16
    order = np.argsort(ids_ref, axis=1, kind="stable")
    acc = np.zeros((T, H), np.float32)
    for jj in range(K_TOP):
        acc = (acc + np.take_along_axis(out_n[:, :K_TOP], order[:, jj][:, None, None], 1)[:, 0]
               ).astype(np.float32)
    acc = (acc + out_n[:, K_TOP]).astype(np.float32)
    np.testing.assert_array_equal(f32(y).view(np.uint32), Q.bf16_round(acc).view(np.uint32))
    experts.cache.clear()


@pytest.mark.parametrize("frag", [False, True])
def test_fp4_prefill_T8192_stages(gpu, experts, frag):
    """MXFP4 routed experts (the reference's live format) with the FP8 shared
    expert at the prefill shape, T = 8192, uniform routing, row-major tiles
    or the register-fed kernels over fragment-layout copies: the integer
    stages bit-exact, the one-call layer equal to the stages, the hottest,
    coldest and a one-row expert's requantized h and down GEMM (on the
    device's own h) against the oracle, the shared expert's first 256 rows,
    and the combine exact given the device's rows."""
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    print(f"fp4 prefill T=8192 uniform, frag={frag}", flush=True)
    rng = np.random.default_rng(8192 + frag)
    T = 8192
    g = torch.Generator(device=gpu)
    g.manual_seed(19)
    u8t = torch.uint8
    w13 = torch.randint(0, 256, (E, 2, I, H // 2), dtype=u8t, device=gpu, generator=g)
    s13 = torch.randint(119, 122, (E, 2, I, H // 32), dtype=u8t, device=gpu, generator=g)
    w2 = torch.randint(0, 256, (E, H, I // 2), dtype=u8t, device=gpu, generator=g)
    s2 = torch.randint(119, 122, (E, H, I // 32), dtype=u8t, device=gpu, generator=g)
    e8 = torch.float8_e8m0fnu
    ent = [(w13[e, 0], w13[e, 1], w2[e], s13[e, 0].view(e8), s13[e, 1].view(e8), s2[e].view(e8))
           for e in range(E)]
    table = M.ExpertTable.build(ent, tuple(experts.table.keep[-6:]), frag_layout=frag)
    x = bf16_values(rng, (T, H))
    draw = lambda n: rng.standard_normal((n, E)).astype(np.float32)  # noqa: E731
    w, ids, w_ref, ids_ref = _route(gpu, _untie(rng, draw(T), draw))
    xd = to_dev_bf16(x, gpu)
    xq, xs = K.act_quant(xd)
    counts, offsets, sorted_slot, slot_pos = M.permute(ids, E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), table, K_TOP)
    out = M.down(hq, hs, offsets, sorted_slot, table, T, K_TOP)
    y = M.combine(out, ids, True)
    y_layer = M.moe_forward(xd, ids, w, table)
    torch.cuda.synchronize()
    perm = OM.permute(ids_ref, E)
    for name, dev in (("counts", counts), ("offsets", offsets), ("sorted_slot", sorted_slot),
                      ("slot_pos", slot_pos)):
        np.testing.assert_array_equal(dev.cpu().numpy(), perm[name], err_msg=name)
    np.testing.assert_array_equal(u8(y), u8(y_layer))

    def host(e):
        return {"fmt": "fp4", "w1": u8(w13[e, 0]), "w3": u8(w13[e, 1]), "w2": u8(w2[e]),
                "s1": u8(s13[e, 0]), "s3": u8(s13[e, 1]), "s2": u8(s2[e])}

    cnt = perm["counts"]
    nz = np.nonzero(cnt)[0]
    sample = {int(nz[np.argmax(cnt[nz])]), int(nz[np.argmin(cnt[nz])])}
    ones = np.nonzero(cnt == 1)[0]
    if ones.size:
        sample.add(int(ones[0]))
    hq_n, hs_n, out_n = u8(hq), f32(hs), f32(out)
    for e in sorted(sample):
        p0, p1 = perm["offsets"][e], perm["offsets"][e + 1]
        sl = perm["sorted_slot"][p0:p1]
        tok, top = sl // K_TOP, sl % K_TOP
        he = host(e)
        tr = {}
        ref = OM.expert_forward(x[tok], he, w_ref[tok, top][:, None], trace=tr)
        assert_requant_close(hq_n[p0:p1], hs_n[p0:p1], tr["hq"], tr["hs"], f"fp4 h expert {e} ({p1 - p0} rows)")
        assert_gemm_close(out_n[tok, top], F4.fp4_gemm(hq_n[p0:p1], hs_n[p0:p1], he["w2"], he["s2"]),
                          f"fp4 down expert {e} on the device's h ({p1 - p0} rows)")
        assert_layer_close(out_n[tok, top], ref, f"fp4 expert {e} vs the oracle's expert")
    P = T * K_TOP
    n_sh = 256
    tr = {}
    ref = OM.expert_forward(x[:n_sh], experts.host("shared"), None, trace=tr)
    assert_requant_close(hq_n[P:P + n_sh], hs_n[P:P + n_sh], tr["hq"], tr["hs"], "h shared")
    exs = experts.host("shared")
    assert_gemm_close(out_n[:n_sh, K_TOP], OM.fp8_gemm(hq_n[P:P + n_sh], hs_n[P:P + n_sh], exs["w2"],
                                                        exs["s2"]), "down shared on the device's h")
    order = np.argsort(ids_ref, axis=1, kind="stable")
    acc = np.zeros((T, H), np.float32)
    for jj in range(K_TOP):
        acc = (acc + np.take_along_axis(out_n[:, :K_TOP], order[:, jj][:, None, None], 1)[:, 0]
               ).astype(np.float32)
    acc = (acc + out_n[:, K_TOP]).astype(np.float32)
    np.testing.assert_array_equal(f32(y).view(np.uint32), Q.bf16_round(acc).view(np.uint32))
    del table, w13, w2
    experts.cache.clear()


@pytest.mark.parametrize("M_", [1024, 4096])
def test_dense_gemm_config_shape(gpu, experts, M_):
    """N = 4096, K = 7168: the 128 x 128 (M = 1024) and 128 x 256 (M = 4096)
    tile paths over 56 K stages against the dequantize-to-fp32 product."""
    from sglang_lite_amd import kernel as K

    print(f"dense gemm M={M_}", flush=True)
    N, KK = 4096, 7168
    g = torch.Generator(device=gpu)
    g.manual_seed(M_)
    a = torch.randn(M_, KK, generator=g, device=gpu).to(torch.bfloat16)
    aq, sa = K.act_quant(a)
    bq, sb = K.per_block_cast_to_fp8(torch.randn(N, KK, generator=g, device=gpu) * 0.02, False)
    c = K.fp8_gemm(aq, sa, bq, sb)
    torch.cuda.synchronize()
    ref = OM.fp8_gemm(u8(aq), f32(sa), u8(bq), f32(sb))
    assert_gemm_close(f32(c), ref, f"dense M={M_}")


def test_fp4_decode_T64_layer_matches_oracle(gpu, experts):
    """MXFP4 routed experts (packed e2m1 codes drawn uniformly, every code
    including 8 present, e8m0 1x32 scales) with the FP8 shared expert, decode
    T = 64 Zipf: per
    touched expert the requantized h against the oracle's and the down GEMM
    on the device's own h at the single-GEMM bound; the layer against the
    oracle's layer."""
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    print("fp4 decode T=64 zipf, full layer", flush=True)
    rng = np.random.default_rng(65)
    T = 64
    g = torch.Generator(device=gpu)
    g.manual_seed(9)
    u8t = torch.uint8
    w13 = torch.randint(0, 256, (E, 2, I, H // 2), dtype=u8t, device=gpu, generator=g)
    # uniform codes (std 2.93 in e2m1 units) under scales 2^-8 .. 2^-6: weight
    # std ~0.028, the magnitude of the N(0, 0.02) FP8 experts, so the layer
    # outputs are O(1) as at the configuration
    s13 = torch.randint(119, 122, (E, 2, I, H // 32), dtype=u8t, device=gpu, generator=g)
    w2 = torch.randint(0, 256, (E, H, I // 2), dtype=u8t, device=gpu, generator=g)
    s2 = torch.randint(119, 122, (E, H, I // 32), dtype=u8t, device=gpu, generator=g)
    e8 = torch.float8_e8m0fnu
    ent = [(w13[e, 0], w13[e, 1], w2[e], s13[e, 0].view(e8), s13[e, 1].view(e8), s2[e].view(e8))
           for e in range(E)]
    sh = experts.table.keep[-6:]
    table = M.ExpertTable.build(ent, tuple(sh))
    x = bf16_values(rng, (T, H))
    w, ids, w_ref, ids_ref = _route(gpu, _untie(rng, zipf_logits(rng, T), lambda n: zipf_logits(rng, n)))
    xd = to_dev_bf16(x, gpu)
    y = M.moe_forward(xd, ids, w, table)
    xq, xs = K.act_quant(xd)
    counts, offsets, sorted_slot, _ = M.permute(ids, E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), table, K_TOP)
    out = M.down(hq, hs, offsets, sorted_slot, table, T, K_TOP)
    torch.cuda.synchronize()

    def host(e):
        return {"fmt": "fp4", "w1": u8(w13[e, 0]), "w3": u8(w13[e, 1]), "w2": u8(w2[e]),
                "s1": u8(s13[e, 0]), "s3": u8(s13[e, 1]), "s2": u8(s2[e])}

    perm = OM.permute(ids_ref, E)
    hq_n, hs_n, out_n = u8(hq), f32(hs), f32(out)
    fp4_host = {}
    worst = 0.0
    for e in np.unique(ids_ref).tolist():
        fp4_host[e] = host(e)
        p0, p1 = perm["offsets"][e], perm["offsets"][e + 1]
        sl = perm["sorted_slot"][p0:p1]
        tok, top = sl // K_TOP, sl % K_TOP
        tr = {}
        OM.expert_forward(x[tok], fp4_host[e], w_ref[tok, top][:, None], trace=tr)
        assert_requant_close(hq_n[p0:p1], hs_n[p0:p1], tr["hq"], tr["hs"], f"fp4 h expert {e}")
        ref = F4.fp4_gemm(hq_n[p0:p1], hs_n[p0:p1], fp4_host[e]["w2"], fp4_host[e]["s2"])
        worst = max(worst, gemm_err_stats(out_n[tok, top], ref)["max_ratio"])
        assert_gemm_close(out_n[tok, top], ref, f"fp4 down expert {e} on the device's h")
    print(f"fp4 down GEMMs on the device's h: worst element at {worst:.3f}x the bound", flush=True)
    y_ref = OM.moe_forward(x, ids_ref, w_ref, fp4_host, experts.host("shared"))
    assert_layer_close(f32(y), y_ref, "fp4 moe decode T=64")
    experts.cache.clear()
