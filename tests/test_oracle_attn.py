"""Pins of the sparse-attention oracle: the blocked bf16-P restatement against
the float64 closed form, and special cases the mathematics fixes."""

from __future__ import annotations

import numpy as np

from helpers import bf16_values
from oracle import attn as OA
from oracle import quant as Q


def test_blocked_matches_closed_form():
    rng = np.random.default_rng(0)
    B, M, H, D, n, K = 2, 3, 16, 64, 300, 200
    q = bf16_values(rng, (B, M, H, D))
    kv = bf16_values(rng, (B, n, D))
    sink = rng.standard_normal(H).astype(np.float32)
    idx = rng.integers(-1, n, (B, M, K)).astype(np.int32)
    blk = OA.sparse_attn_blocked(q, kv, sink, idx, D ** -0.5)
    ex = OA.sparse_attn_exact(q, kv, sink, idx, D ** -0.5)
    rel = np.linalg.norm(blk - ex) / np.linalg.norm(ex)
    assert rel < 5e-3  # bf16 probabilities and output


def test_single_row_and_sink_closed_form():
    """One valid row j: o = kv_j * p / (p + e^(sink - s)) with p = 1 at the max."""
    rng = np.random.default_rng(1)
    H, D = 16, 64
    q = bf16_values(rng, (1, 1, H, D))
    kv = bf16_values(rng, (1, 10, D))
    sink = rng.standard_normal(H).astype(np.float32)
    idx = np.full((1, 1, 70), -1, np.int32)
    idx[0, 0, 65] = 7  # in the second block
    o = OA.sparse_attn_blocked(q, kv, sink, idx, 0.125)
    s = (q[0, 0].astype(np.float64) @ kv[0, 7].astype(np.float64)) * 0.125
    w = 1.0 / (1.0 + np.exp(sink.astype(np.float64) - s))
    want = Q.bf16_round((w[:, None] * kv[0, 7][None, :]).astype(np.float32))
    np.testing.assert_allclose(o[0, 0], want, rtol=2 ** -7, atol=1e-6)


def test_all_masked_gives_zero_and_no_sink_averages():
    rng = np.random.default_rng(2)
    H, D = 16, 32
    q = bf16_values(rng, (1, 1, H, D))
    kv = bf16_values(rng, (1, 5, D))
    o = OA.sparse_attn_blocked(q, kv, np.zeros(H, np.float32), np.full((1, 1, 8), -1, np.int32), 1.0)
    assert np.all(o == 0)
    # identical rows and a sink of -inf: the output is the row itself
    kv2 = np.repeat(kv[:, :1], 5, axis=1)
    idx = np.arange(5, dtype=np.int32).reshape(1, 1, 5)
    o2 = OA.sparse_attn_blocked(q, kv2, np.full(H, -np.inf, np.float32), idx, 1.0)
    np.testing.assert_allclose(o2[0, 0], np.repeat(kv2[0, :1], H, axis=0), rtol=2 ** -7)
