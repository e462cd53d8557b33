"""Pins of the routing oracle against torch's CPU routines (library ops)."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import moe as OM


def _torch_scores(lg, score_func):
    s = torch.from_numpy(lg)
    if score_func == "softmax":
        return s.softmax(dim=-1)
    if score_func == "sigmoid":
        return s.sigmoid()
    return F.softplus(s).sqrt()


def test_route_hash_matches_torch_gather():
    rng = np.random.default_rng(0)
    T, E, k, V = 50, 64, 6, 300
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    tid2eid = np.stack([rng.permutation(E)[:k] for _ in range(V)]).astype(np.int32)
    ids_in = rng.integers(0, V, T)
    for sf in ("sqrtsoftplus", "softmax", "sigmoid"):
        w, ids = OM.route_hash(lg, tid2eid, ids_in, k, sf, 1.5)
        sc = _torch_scores(lg, sf)
        tids = torch.from_numpy(tid2eid)[torch.from_numpy(ids_in)].long()
        tw = sc.gather(1, tids)
        if sf != "softmax":
            tw = tw / tw.sum(dim=-1, keepdim=True)
        tw = tw * 1.5
        np.testing.assert_array_equal(ids, tids.numpy())
        np.testing.assert_allclose(w, tw.numpy(), rtol=1e-6, atol=1e-7)
        if sf != "softmax":
            np.testing.assert_allclose(w.sum(-1), 1.5, rtol=1e-5)


def test_router_logits_exact_for_bf16_operands():
    rng = np.random.default_rng(1)
    x = torch.randn(9, 256).bfloat16()
    W = torch.randn(16, 256).bfloat16()
    ref = (x.double() @ W.double().T).float().numpy()
    got = OM.router_logits(x.float().numpy(), W.float().numpy())
    np.testing.assert_array_equal(got, ref)


def test_moe_forward_workers_same_bytes():
    """The threaded oracle layer (experts on worker threads, combined in
    ascending expert order) is the serial layer, byte for byte; the per-expert
    outputs it reports are the serial ones too."""
    from oracle import quant as Q

    rng = np.random.default_rng(12)
    T, H, I, E, k = 48, 256, 128, 8, 2
    x = Q.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    w, ids = OM.route_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    experts = [OM.make_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    o1, o4 = {}, {}
    y1 = OM.moe_forward(x, ids, w, experts, sh, swiglu_limit=5.0, expert_outputs=o1)
    y4 = OM.moe_forward(x, ids, w, experts, sh, swiglu_limit=5.0, expert_outputs=o4, workers=4)
    np.testing.assert_array_equal(y1.view(np.uint32), y4.view(np.uint32))
    assert o1.keys() == o4.keys()
    for key in o1:
        a, b = o1[key], o4[key]
        a, b = (a[2], b[2]) if isinstance(a, tuple) else (a, b)
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    # and the serial layer is the reference's full loop (model.py:629-644)
    np.testing.assert_array_equal(
        y1.view(np.uint32),
        OM.moe_forward_full_loop(x, ids, w, experts, sh, swiglu_limit=5.0).view(np.uint32))
