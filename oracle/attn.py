"""Oracle: sparse multi-head attention with an attention sink, restated in numpy.

Test infrastructure only (see ``oracle/__init__.py``).  Arrays hold bf16
values as float32.
"""

from __future__ import annotations

import numpy as np

from . import quant as Q


def _gather(kv_b: np.ndarray, idx_m: np.ndarray):
    n = kv_b.shape[0]
    valid = (idx_m >= 0) & (idx_m < n)
    rows = np.where(valid[:, None], kv_b[np.clip(idx_m, 0, max(n - 1, 0))], 0.0).astype(np.float32)
    return rows, valid


def sparse_attn_blocked(q: np.ndarray, kv: np.ndarray, sink: np.ndarray, idx: np.ndarray,
                        scale: float, block: int = 64) -> np.ndarray:
    """deepseek_infer/kernel.py:276-347 sparse_attn_kernel: per query token, the
    gathered rows in blocks of 64 with a running max / sum (fp32), the block's
    probabilities cast to bf16 for the P.V product (fp32 accumulation), the
    sink added to the normaliser at the end, bf16 output.
    q [B, M, H, D], kv [B, n, D], sink [H], idx [B, M, K] -> o [B, M, H, D]."""
    B, M, H, D = q.shape
    K = idx.shape[-1]
    sc = np.float32(scale)
    out = np.zeros((B, M, H, D), np.float32)
    for b in range(B):
        for m in range(M):
            rows, valid = _gather(kv[b], idx[b, m])
            qh = q[b, m].astype(np.float64)
            mx = np.full(H, -np.inf, np.float32)
            l = np.zeros(H, np.float32)
            acc = np.zeros((H, D), np.float32)
            for j0 in range(0, K, block):
                r = rows[j0:j0 + block].astype(np.float64)
                v = valid[j0:j0 + block]
                s = ((qh @ r.T).astype(np.float32) * sc).astype(np.float32)
                s[:, ~v] = -np.inf
                m_new = np.maximum(mx, s.max(axis=1))
                ref = np.where(np.isneginf(m_new), np.float32(0), m_new).astype(np.float32)
                with np.errstate(invalid="ignore"):
                    alpha = np.exp(mx - ref).astype(np.float32)
                p = np.exp(s - ref[:, None]).astype(np.float32)
                l = (l * alpha + p.sum(axis=1, dtype=np.float32)).astype(np.float32)
                pb = Q.bf16_round(p).astype(np.float64)
                acc = (acc * alpha[:, None] + (pb @ r).astype(np.float32)).astype(np.float32)
                mx = m_new
            ref = np.where(np.isneginf(mx), np.float32(0), mx).astype(np.float32)
            denom = (l + np.exp(np.asarray(sink, np.float32) - ref)).astype(np.float32)
            out[b, m] = Q.bf16_round((acc / denom[:, None]).astype(np.float32))
    return out


def sparse_attn_exact(q: np.ndarray, kv: np.ndarray, sink: np.ndarray, idx: np.ndarray,
                      scale: float) -> np.ndarray:
    """The same attention in float64 without blocking or bf16 probabilities:
    o = sum_j e^(s_j - c) kv_j / (sum_j e^(s_j - c) + e^(sink - c)) (the
    closed form that engine/v4_sparse_torch.py:68-106 computes in fp32)."""
    B, M, H, D = q.shape
    out = np.zeros((B, M, H, D), np.float64)
    for b in range(B):
        for m in range(M):
            rows, valid = _gather(kv[b], idx[b, m])
            s = (q[b, m].astype(np.float64) @ rows.astype(np.float64).T) * float(scale)
            s[:, ~valid] = -np.inf
            c = np.maximum(s.max(axis=1), np.asarray(sink, np.float64))
            e = np.exp(s - c[:, None])
            denom = e.sum(axis=1) + np.exp(np.asarray(sink, np.float64) - c)
            out[b, m] = (e @ rows.astype(np.float64)) / denom[:, None]
    return out
