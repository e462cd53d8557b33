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
