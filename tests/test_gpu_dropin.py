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
from helpers import (assert_gemm_close, assert_layer_close, bf16_values, f32, to_dev_bf16, to_dev_f32,
                     to_dev_fp8, u8)
from oracle import fp4 as F4
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


def _dev_fp4_expert(e, dev):
    def w4(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).view(torch.float4_e2m1fn_x2)

    def s8(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).view(torch.float8_e8m0fnu)

    return (w4(e["w1"]), w4(e["w3"]), w4(e["w2"]), s8(e["s1"]), s8(e["s3"]), s8(e["s2"]))


def test_fp4_linear_expert_and_moe_dropins(official, gpu):
    """The reference's live configuration: FP4 routed experts, FP8 shared
    expert, scale_fmt "ue8m0" with e8m0 activation scales (model.py:40-42,
    113-115, 623-626): the official linear() through the patched
    kernel.fp4_gemm, Expert.forward and MoE.forward, against the oracle."""
    from sglang_lite_amd import v4_deep_gemm as D
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    M.scale_fmt = "ue8m0"
    M.scale_dtype = torch.float8_e8m0fnu
    rng = np.random.default_rng(43)
    T, H, I, E, k = 40, 512, 256, 8, 2
    x = bf16_values(rng, (T, H))
    experts = [OM.make_fp4_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    W = (rng.standard_normal((E, H)) * H ** -0.5).astype(np.float32)
    gate = M.Gate(to_dev_f32(W, gpu), k)
    moe = M.MoE(H, gate, [M.Expert(_dev_fp4_expert(e, gpu)) for e in experts],
                M.Expert(_dev_expert(sh, gpu)))
    st = D.attach_v4_deep_gemm(moe)
    assert st["enabled"] and st["scale_cache"] == 3 * (E + 1)
    assert K.fp4_gemm is M.fp4_gemm and getattr(K.fp4_gemm, D.MARK, False)
    assert MF.attach_v4_moe_fast(moe)["enabled"]
    xd = to_dev_bf16(x, gpu)
    mode = 1  # scale_fmt "ue8m0" with the torch formula: power-of-two activation scales
    q_ref, s_ref = Q.per_token_cast_to_fp8(x, True, 128)
    # official linear() -> patched act_quant + fp4_gemm (e8m0 activation scales)
    ex0 = moe.experts[0]
    y_lin = M.linear(xd, ex0.w1.weight)
    assert y_lin.dtype == torch.get_default_dtype()
    assert_gemm_close(f32(y_lin), F4.fp4_gemm(q_ref, s_ref, experts[0]["w1"], experts[0]["s1"],
                                              out_bf16=False), "linear fp4")
    # Expert.forward of one FP4 expert
    w = rng.uniform(0.1, 1.0, (T, 1)).astype(np.float32)
    y_ex = ex0(xd, to_dev_f32(w, gpu))
    assert_gemm_close(f32(y_ex), OM.expert_forward(x, experts[0], w, mode=mode), "Expert.forward fp4")
    # MoE.forward: FP4 routed + FP8 shared
    y = moe(xd.view(1, T, H), torch.zeros(1, T, dtype=torch.long, device=gpu))
    logits = F.linear(xd.float(), gate.weight.float()).cpu().numpy()
    w_ref, ids_ref = OM.route_topk(logits, k)
    assert OM.topk_margin(logits, k) > 1e-6
    y_ref = OM.moe_forward(x, ids_ref, w_ref, experts, sh, mode=mode)
    assert_gemm_close(f32(y[0]), y_ref, "patched MoE.forward fp4")


def test_moe_forward_with_bf16_and_hash_gates(official, gpu):
    """MoE.forward with the checkpoint's bf16 router weight: the fused gate
    kernel for a score-routed layer (sqrtsoftplus + bias, route_scale 1.5) and
    a hash-routed one (tid2eid[input_ids]), each against the oracle."""
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    rng = np.random.default_rng(44)
    T, H, I, E, k, V = 40, 512, 256, 16, 4, 500
    x = bf16_values(rng, (T, H))
    Wb = bf16_values(rng, (E, H), scale=H ** -0.5)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    tid2eid = np.stack([rng.permutation(E)[:k] for _ in range(V)]).astype(np.int32)
    input_ids = rng.integers(0, V, (1, T))
    xd = to_dev_bf16(x, gpu)
    iid = torch.from_numpy(input_ids).to(gpu)
    for hashed in (False, True):
        gate = M.Gate(to_dev_bf16(Wb, gpu), k, "sqrtsoftplus", 1.5,
                      None if hashed else to_dev_f32(bias, gpu),
                      torch.from_numpy(tid2eid).to(gpu) if hashed else None)
        moe = M.MoE(H, gate, [M.Expert(_dev_expert(e, gpu)) for e in experts],
                    M.Expert(_dev_expert(sh, gpu)))
        assert MF.attach_v4_moe_fast(moe)["enabled"]
        y = moe(xd.view(1, T, H), iid)
        logits = OM.router_logits(x, Wb)
        if hashed:
            w_ref, ids_ref = OM.route_hash(logits, tid2eid, input_ids, k, "sqrtsoftplus", 1.5)
        else:
            assert OM.topk_margin(logits, k, "sqrtsoftplus", bias) > 1e-5
            w_ref, ids_ref = OM.route_topk(logits, k, "sqrtsoftplus", bias, 1.5)
        y_ref = OM.moe_forward(x, ids_ref, w_ref, experts, sh)
        assert_gemm_close(f32(y[0]), y_ref, f"MoE.forward bf16 gate hash={hashed}")


@pytest.mark.parametrize("frag", [False, True])
def test_moe_layer_captures_into_a_hip_graph(official, gpu, monkeypatch, frag):
    """The patched MoE.forward captured the way the reference's decode runner
    captures the model (v4_runner/cuda_graph.py:98-137: warmup, synchronize,
    capture, replay into static buffers).  The official forward cannot be
    captured (bincount().tolist() syncs, model.py:634); this one launches
    only HIP kernels on torch's stream.  Every replay, with eager work and
    syncs between replays, equals the eager forward on the same input bit
    for bit.  ``frag``: with fragment-layout weight copies (the register-fed
    GEMMs, which need K >= 2048: H = I = 2048)."""
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    monkeypatch.setenv("SGLANG_LITE_AMD_FRAG_LAYOUT", "1" if frag else "0")
    rng = np.random.default_rng(45)
    T, H, I, E, k = (64, 2048, 2048, 8, 2) if frag else (64, 512, 256, 16, 4)
    Wb = bf16_values(rng, (E, H), scale=H ** -0.5)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    gate = M.Gate(to_dev_bf16(Wb, gpu), k, "sqrtsoftplus", 1.5,
                  to_dev_f32((rng.standard_normal(E) * 0.05).astype(np.float32), gpu))
    moe = M.MoE(H, gate, [M.Expert(_dev_expert(e, gpu)) for e in experts],
                M.Expert(_dev_expert(sh, gpu)))
    assert MF.attach_v4_moe_fast(moe)["enabled"]
    assert bool(MF.expert_table(moe).fmt & 4) == frag
    ids0 = torch.zeros(1, T, dtype=torch.long, device=gpu)
    x_static = to_dev_bf16(bf16_values(rng, (T, H)), gpu).view(1, T, H)
    for _ in range(3):
        moe(x_static, ids0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_static = moe(x_static, ids0)
    for i in range(4):
        xi = to_dev_bf16(bf16_values(rng, (T, H)), gpu).view(1, T, H)
        x_static.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        eager = moe(xi.clone(), ids0)  # eager launches between replays
        torch.cuda.synchronize()
        np.testing.assert_array_equal(u8(y_static), u8(eager), err_msg=f"replay {i}")
    # and the eager result is the oracle's layer
    x_last = f32(xi[0])
    logits = OM.router_logits(x_last, Wb)
    w_ref, ids_ref = OM.route_topk(logits, k, "sqrtsoftplus", f32(gate.bias), 1.5)
    assert_gemm_close(f32(eager[0]), OM.moe_forward(x_last, ids_ref, w_ref, experts, sh), "graph MoE")


def test_graph_replay_after_the_workspace_grows(official, gpu):
    """A decode graph captured at T = 64 keeps its workspace address.  An eager
    call with more tokens grows the module's workspace; the captured buffer
    must stay allocated (not return to torch's pool, where the tensor
    allocated next could take it), so replaying the T = 64 graph afterwards
    still equals the eager forward bit for bit and leaves other tensors alone."""
    from sglang_lite_amd import moe as HM
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    rng = np.random.default_rng(46)
    T, H, I, E, k = 64, 512, 256, 16, 4
    Wb = bf16_values(rng, (E, H), scale=H ** -0.5)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    gate = M.Gate(to_dev_bf16(Wb, gpu), k, "softmax", 1.0, None)
    moe = M.MoE(H, gate, [M.Expert(_dev_expert(e, gpu)) for e in experts],
                M.Expert(_dev_expert(sh, gpu)))
    assert MF.attach_v4_moe_fast(moe)["enabled"]
    ids0 = torch.zeros(1, T, dtype=torch.long, device=gpu)
    x_static = to_dev_bf16(bf16_values(rng, (T, H)), gpu).view(1, T, H)
    for _ in range(3):
        moe(x_static, ids0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_static = moe(x_static, ids0)
    ws = moe._sgl_ws
    captured = ws.buf.data_ptr()
    # an eager prefill-sized call grows the workspace
    T_big = 1024
    xb = to_dev_bf16(bf16_values(rng, (T_big, H)), gpu).view(1, T_big, H)
    moe(xb, torch.zeros(1, T_big, dtype=torch.long, device=gpu))
    torch.cuda.synchronize()
    assert ws.buf.data_ptr() != captured
    assert any(b.data_ptr() == captured for b in ws.retired)
    # tensors allocated now must not receive the graph's writes
    fence = [torch.full((n,), 0xA5, dtype=torch.uint8, device=gpu)
             for n in (r.numel() for r in ws.retired)]
    for i in range(3):
        xi = to_dev_bf16(bf16_values(rng, (T, H)), gpu).view(1, T, H)
        x_static.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        eager = moe(xi.clone(), ids0)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(u8(y_static), u8(eager), err_msg=f"replay {i}")
    for f in fence:
        assert bool((f == 0xA5).all()), "a graph replay wrote into a tensor allocated after capture"
    assert isinstance(ws, HM.MoEWorkspace)


def test_moe_forward_with_frag_layout_switch(official, gpu, monkeypatch):
    """SGLANG_LITE_AMD_FRAG_LAYOUT=1: the patched MoE.forward builds its expert
    table with fragment-layout weight copies (the register-fed GEMMs at
    H = I = 2048) and returns the same bytes as the row-major table; both
    against the oracle."""
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    rng = np.random.default_rng(45)
    T, H, I, E, k = 40, 2048, 2048, 8, 2
    x = bf16_values(rng, (T, H))
    W = (rng.standard_normal((E, H)) * H ** -0.5).astype(np.float32)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    gate = M.Gate(to_dev_f32(W, gpu), k)
    xd = to_dev_bf16(x, gpu)
    iid = torch.zeros(1, T, dtype=torch.long, device=gpu)
    ys = {}
    for on in (False, True):
        monkeypatch.setenv("SGLANG_LITE_AMD_FRAG_LAYOUT", "1" if on else "0")
        moe = M.MoE(H, gate, [M.Expert(_dev_expert(e, gpu)) for e in experts],
                    M.Expert(_dev_expert(sh, gpu)))
        assert MF.attach_v4_moe_fast(moe)["enabled"]
        ys[on] = moe(xd.view(1, T, H), iid)
        assert bool(MF.expert_table(moe).fmt & 4) == on
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u8(ys[True]), u8(ys[False]))
    logits = F.linear(xd.float(), gate.weight.float()).cpu().numpy()
    w_ref, ids_ref = OM.route_topk(logits, k)
    assert OM.topk_margin(logits, k) > 1e-6
    y_ref = OM.moe_forward(x, ids_ref, w_ref, experts, sh)
    assert_gemm_close(f32(ys[True][0]), y_ref, "MoE.forward with fragment-layout weights")


def test_kv_pack_with_the_attached_act_quant_takes_the_fused_kernel(official, gpu, monkeypatch):
    """attach_v4_deep_gemm replaces kernel.act_quant by the package's wrapper;
    pack_dsv4_kv_bf16 / pack_dsv4_kv_paged / write_packed_kv_bf16 given that
    function (as engine/v4_sparse_mla.py:85,91 passes it) run the fused kernel
    and produce the bytes of the package's own act_quant."""
    from sglang_lite_amd import dsv4_kv_pack as KVP
    from sglang_lite_amd import kernel as HK
    from sglang_lite_amd import v4_deep_gemm as D

    M, K = official
    assert D.attach_v4_deep_gemm(None)["enabled"]
    assert K.act_quant is not HK.act_quant
    rng = np.random.default_rng(42)
    kv = to_dev_bf16(bf16_values(rng, (130, 512)), gpu)
    want = KVP.pack_dsv4_kv_bf16(kv, act_quant_fn=HK.act_quant)

    def unfused(*a, **k):
        raise AssertionError("the attached act_quant took the unfused path")

    monkeypatch.setattr(KVP, "_pack_rows_with", unfused)
    got = KVP.pack_dsv4_kv_bf16(kv, act_quant_fn=K.act_quant)
    assert torch.equal(got, want)
    pages = KVP.pack_dsv4_kv_paged(kv, 64, act_quant_fn=K.act_quant)
    assert torch.equal(pages, KVP.to_paged_hnd(want, 64))
    pool = torch.zeros(1, 4, 1, 64, 584, dtype=torch.uint8, device=gpu)
    KVP.write_packed_kv_bf16(pool, [2, 0, 3], 0, kv, act_quant_fn=K.act_quant)
    torch.cuda.synchronize()
    assert torch.equal(pool[0, 2, 0], want[:64]) and torch.equal(pool[0, 0, 0], want[64:128])
    assert torch.equal(pool[0, 3, 0, :2], want[128:130])


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
def test_expert_sharded_ranks(official, gpu, fmt):
    """The layer as the reference runs it on an expert-sharded world
    (deepseek_infer/model.py:616-625: rank r builds experts [r E/W, (r+1) E/W)
    and None elsewhere; engine/v4_moe_fast.py:79-106): each of W = 4 ranks is
    built in turn with world_size = 4 and dist.all_reduce stubbed.
    * The fp32 sum each rank hands to all_reduce equals, bit for bit, the
      ascending fp32 sum of the device's own expert rows of that rank's
      experts (the unsharded grouped launches' rows), and the oracle's rank
      sum (moe_local_partial) within the layer tolerance.
    * With all_reduce as identity, the rank's output is bf16(partial + shared
      row) exactly.
    * With all_reduce summing the four ranks' partials, the output matches the
      whole layer's oracle."""
    import types

    from sglang_lite_amd import moe as HM
    from sglang_lite_amd import v4_moe_fast as MF

    M, K = official
    rng = np.random.default_rng(44 if fmt == "fp8" else 45)
    T, H, I, E, k, W = 48, 512, 256, 16, 4, 4
    x = bf16_values(rng, (T, H))
    Wg = (rng.standard_normal((E, H)) * H ** -0.5).astype(np.float32)
    if fmt == "fp8":
        experts = [OM.make_expert(rng, H, I) for _ in range(E)]
        dev = [_dev_expert(e, gpu) for e in experts]
    else:
        experts = [OM.make_fp4_expert(rng, H, I) for _ in range(E)]
        dev = [_dev_fp4_expert(e, gpu) for e in experts]
    sh = OM.make_expert(rng, H, I)
    sh_dev = _dev_expert(sh, gpu)
    gate = M.Gate(to_dev_f32(Wg, gpu), k)
    xd = to_dev_bf16(x, gpu).view(1, T, H)
    in_ids = torch.zeros(1, T, dtype=torch.long, device=gpu)
    # routing and the device's own expert rows from the unsharded launches
    logits = F.linear(xd[0].float(), gate.weight.float()).cpu().numpy()
    w_ref, ids_ref = OM.route_topk(logits, k)
    assert OM.topk_margin(logits, k) > 1e-6
    full_tab = HM.ExpertTable.build(dev, sh_dev)
    from sglang_lite_amd import kernel as HK

    w_d, ids_d = HM.route_topk(F.linear(xd[0].float(), gate.weight.float()), k)
    xq, xs = HK.act_quant(xd[0])
    _, offsets, sorted_slot, _ = HM.permute(ids_d, E)
    hq, hs = HM.gate_up(xq, xs, offsets, sorted_slot, w_d.reshape(-1), full_tab, k)
    rows = f32(HM.down(hq, hs, offsets, sorted_slot, full_tab, T, k))  # [T, k+1, H]
    ids_np = ids_d.cpu().numpy()
    np.testing.assert_array_equal(ids_np, ids_ref)

    M.world_size = W
    partials = []

    def record(t):
        partials.append(t.clone())

    M.dist = types.SimpleNamespace(all_reduce=record)
    MF.attach_v4_moe_fast(torch.nn.Module())
    per = E // W
    mods = []
    for r in range(W):
        lo, hi = r * per, (r + 1) * per
        moe = M.MoE(H, gate, [M.Expert(dev[e]) if lo <= e < hi else None for e in range(E)],
                    M.Expert(sh_dev))
        moe.experts_start_idx, moe.experts_end_idx = lo, hi
        mods.append(moe)
        y_r = moe(xd, in_ids)
        part = partials[-1]
        assert part.dtype == torch.float32 and part.shape == (T, H)
        p_np = part.cpu().numpy()
        # bit for bit: the ascending fp32 sum of the device's rows of local experts
        want = np.zeros((T, H), np.float32)
        for t in range(T):
            for j in np.argsort(ids_np[t], kind="stable"):
                if lo <= ids_np[t, j] < hi:
                    want[t] = (want[t] + rows[t, j]).astype(np.float32)
        np.testing.assert_array_equal(p_np.view(np.uint32), want.view(np.uint32))
        ref = OM.moe_local_partial(x, ids_ref, w_ref, experts, lo, hi)
        assert_layer_close(p_np, ref, f"rank {r} partial ({fmt})")
        # identity all_reduce: the rank's output is bf16(partial + shared row)
        y_want = Q.bf16_round((p_np + rows[:, k]).astype(np.float32))
        np.testing.assert_array_equal(f32(y_r[0]).view(np.uint32), y_want.view(np.uint32))
    # all ranks' partials summed by the collective
    total = partials[0].clone()
    for p_ in partials[1:W]:
        total += p_

    def reduce_sum(t):
        t.copy_(total)

    M.dist = types.SimpleNamespace(all_reduce=reduce_sum)
    y = mods[1](xd, in_ids)
    y_ref = OM.moe_forward(x, ids_ref, w_ref, experts, sh)
    assert_layer_close(f32(y[0]), y_ref, f"expert-sharded layer, {W} ranks ({fmt})")
    np.testing.assert_array_equal(
        f32(y[0]).view(np.uint32),
        Q.bf16_round((total.cpu().numpy() + rows[:, k]).astype(np.float32)).view(np.uint32))
    M.world_size = 1


@pytest.mark.parametrize("T", [2049, 40])
def test_local_range_partial_is_the_ordered_sum_of_the_rows(gpu, T):
    """moe_forward_local over several expert ranges -- the whole range, an
    inner one, an empty one -- at a size that takes the chunked permute (T*k
    = 16392 slots) and a small one: the fp32 partial equals, bit for bit, the
    ascending fp32 sum of the device's own expert rows whose expert lies in
    the range, and moe_add_shared adds the shared row in fp32 and rounds."""
    from sglang_lite_amd import kernel as HK
    from sglang_lite_amd import moe as HM

    print(f"local-range partial T={T}", flush=True)
    rng = np.random.default_rng(46 + T)
    H, I, E, k = 512, 256, 16, 8
    x = bf16_values(rng, (T, H))
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    tab = HM.ExpertTable.build([_dev_expert(e, gpu) for e in experts], _dev_expert(sh, gpu))
    logits = to_dev_f32(rng.standard_normal((T, E)).astype(np.float32), gpu)
    w_d, ids_d = HM.route_topk(logits, k)
    xd = to_dev_bf16(x, gpu)
    xq, xs = HK.act_quant(xd)
    _, offsets, sorted_slot, _ = HM.permute(ids_d, E)
    hq, hs = HM.gate_up(xq, xs, offsets, sorted_slot, w_d.reshape(-1), tab, k)
    rows = f32(HM.down(hq, hs, offsets, sorted_slot, tab, T, k))
    ids_np = ids_d.cpu().numpy()
    order = np.argsort(ids_np, axis=1, kind="stable")
    ws = HM.MoEWorkspace()
    for lo, hi in ((0, E), (3, 11), (5, 5)):
        part = HM.moe_forward_local(xd, ids_d, w_d, tab, lo, hi, workspace=ws)
        want = np.zeros((T, H), np.float32)
        for j in range(k):
            e = np.take_along_axis(ids_np, order[:, j:j + 1], axis=1)[:, 0]
            r = rows[np.arange(T), order[:, j]]
            local = (e >= lo) & (e < hi)
            want[local] = (want[local] + r[local]).astype(np.float32)
        np.testing.assert_array_equal(part.cpu().numpy().view(np.uint32), want.view(np.uint32))
        y = HM.moe_add_shared(part, tab, k, ws)
        y_want = Q.bf16_round((want + rows[:, k]).astype(np.float32))
        np.testing.assert_array_equal(f32(y).view(np.uint32), y_want.view(np.uint32))
    # the whole range is the whole layer
    y_full = HM.moe_forward(xd, ids_d, w_d, tab)
    part = HM.moe_forward_local(xd, ids_d, w_d, tab, 0, E, workspace=ws)
    assert torch.equal(HM.moe_add_shared(part, tab, k, ws), y_full)
