"""Sparse MLA attention on gfx950: drop-in for the official ``sparse_attn`` and
the fused consumer of the packed FP8 KV cache.

* ``sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale)`` — the official
  ``kernel.sparse_attn`` contract (deepseek_infer/kernel.py:350-368, kernel
  :276-347): bf16 ``q [B, S, H, 512]``, bf16 ``kv [B, T, 512]``, fp32 sink per
  head, int32 ``topk_idxs [B, S, K]`` with -1 pads; prefill and decode.
* ``sparse_attn_packed(q, cache, ...)`` — the same attention reading the
  584-byte layout A rows (or their footer pages) that
  ``dsv4_kv_pack.pack_dsv4_kv_bf16`` / ``write_packed_kv_bf16`` produce, so no
  bf16 KV and no per-step pack is needed (the "pack tax" of
  engine/v4_sparse_mla.py:34-122, which packs bf16 KV before every decode).
* ``attach_v4_sparse_mla()`` — patches ``kernel.sparse_attn`` /
  ``model.sparse_attn`` (engine/v4_sparse_mla.py:144-250), selected with the
  reference's ``SGLANG_LITE_V4_SPARSE`` switch (``official`` keeps TileLang).
"""

from __future__ import annotations

import logging
import os
import sys
from typing import Any, Optional

import torch

from . import _lib

logger = logging.getLogger("sglang_lite_amd.v4_sparse_mla")
MARK = "_sglang_lite_sparse"
HEAD_DIM = 512
PACKED_BYTES = 584


def _check_q(q: torch.Tensor, topk_idxs: torch.Tensor, attn_sink: torch.Tensor):
    if q.dim() != 4 or topk_idxs.dim() != 3:
        raise ValueError(f"bad ranks q={tuple(q.shape)} topk={tuple(topk_idxs.shape)}")
    b, s, h, d = q.shape
    if d != HEAD_DIM:
        raise ValueError(f"expected head_dim {HEAD_DIM}, got {d}")
    if topk_idxs.shape[0] != b or topk_idxs.shape[1] != s:
        raise ValueError(f"topk {tuple(topk_idxs.shape)} incompatible with q {tuple(q.shape)}")
    if q.dtype != torch.bfloat16:
        raise TypeError(f"sparse_attn: q must be bfloat16, got {q.dtype}")
    if attn_sink.numel() != h:
        raise ValueError(f"attn_sink has {attn_sink.numel()} entries for {h} heads")
    return b, s, h


def _rows_contiguous(t: torch.Tensor) -> bool:
    """Each batch element's rows are dense (any batch stride, e.g. a slice of a pool)."""
    want = 1
    for size, stride in zip(reversed(t.shape[1:]), reversed(t.stride()[1:])):
        if size != 1 and stride != want:
            return False
        want *= size
    return t.data_ptr() % 16 == 0 and t.stride(0) % 8 == 0


def _launch(q, kv, fmt, page, n, bstride, ld, attn_sink, topk_idxs, softmax_scale):
    b, s, h, _ = q.shape
    qc = q.contiguous()
    idx = topk_idxs.to(torch.int32).contiguous()
    sink = attn_sink.to(torch.float32).contiguous()
    o = torch.empty_like(qc)
    k = idx.shape[-1]
    ws_bytes = int(_lib.load().sgl_sparse_attn_workspace_size(b, s, h, k)) if k > 0 else 0
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=qc.device)
    _lib.call("sgl_sparse_attn", qc.data_ptr(), b, s, h, kv.data_ptr(), fmt, page, n, bstride, ld,
              sink.data_ptr(), idx.data_ptr(), k, float(softmax_scale), o.data_ptr(),
              ws.data_ptr(), ws_bytes, _lib.stream_of(qc))
    return o


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor,
                topk_idxs: torch.Tensor, softmax_scale: float) -> torch.Tensor:
    """Sparse multi-head attention with a sink (kernel.py:350-368): bf16 out like q."""
    b, s, h = _check_q(q, topk_idxs, attn_sink)
    _lib.require_device(q, kv, attn_sink, topk_idxs, what="sparse_attn")
    if kv.dim() != 3 or kv.shape[0] != b or kv.shape[2] != HEAD_DIM:
        raise ValueError(f"kv {tuple(kv.shape)} incompatible with q {tuple(q.shape)}")
    if kv.dtype != torch.bfloat16:
        raise TypeError(f"sparse_attn: kv must be bfloat16, got {kv.dtype}")
    kvc = kv if (kv.stride(2) == 1 and kv.stride(1) % 8 == 0 and kv.stride(0) % 8 == 0
                 and kv.data_ptr() % 16 == 0) else kv.contiguous()
    return _launch(q, kvc, _lib.ATTN_KV_BF16, 0, kvc.shape[1], kvc.stride(0) * 2, kvc.stride(1),
                   attn_sink, topk_idxs, softmax_scale)


def sparse_attn_packed(q: torch.Tensor, cache: torch.Tensor, attn_sink: torch.Tensor,
                       topk_idxs: torch.Tensor, softmax_scale: float,
                       n_rows: Optional[int] = None) -> torch.Tensor:
    """The same attention over the packed FP8 cache: ``cache`` uint8
    ``[B, T, 584]`` layout A rows, or ``[B, P, 1, page, 584]`` footer pages
    (``n_rows`` valid rows, default all); rows are dequantized on the way in."""
    b, s, h = _check_q(q, topk_idxs, attn_sink)
    _lib.require_device(q, cache, attn_sink, topk_idxs, what="sparse_attn_packed")
    if cache.dtype != torch.uint8 or cache.shape[-1] != PACKED_BYTES or cache.shape[0] != b:
        raise ValueError(f"expected a uint8 [B, ..., 584] layout A cache, got {cache.dtype} "
                         f"{tuple(cache.shape)}")
    c = cache if _rows_contiguous(cache) else cache.contiguous()
    if c.dim() == 3:
        n = c.shape[1] if n_rows is None else int(n_rows)
        return _launch(q, c, _lib.ATTN_KV_A, 0, n, c.stride(0), 0, attn_sink, topk_idxs,
                       softmax_scale)
    if c.dim() == 5 and c.shape[2] == 1:
        page = c.shape[3]
        n = c.shape[1] * page if n_rows is None else int(n_rows)
        return _launch(q, c, _lib.ATTN_KV_A_PAGED, page, n, c.stride(0), 0, attn_sink,
                       topk_idxs, softmax_scale)
    raise ValueError(f"cache must be [B, T, 584] or [B, P, 1, page, 584], got {tuple(c.shape)}")


def _sparse_backend_preference() -> str:
    """The reference's switch (v4_sparse_mla.py:125-141): ``official`` keeps the
    official kernel; anything else arms the gfx950 kernel."""
    raw = os.environ.get("SGLANG_LITE_V4_SPARSE", "hip").strip().lower()
    return "official" if raw in ("official", "tilelang") else "hip"


def attach_v4_sparse_mla(backend: Any = None, *, window_size: int = 128) -> bool:
    """Patch ``kernel.sparse_attn`` / ``model.sparse_attn`` with the gfx950 kernel
    (prefill and decode).  Returns True when armed; never raises."""
    del window_size
    K = sys.modules.get("kernel")
    M = sys.modules.get("model")
    if K is None and M is None:
        logger.warning("attach_v4_sparse_mla: official modules not loaded")
        return False
    orig = getattr(M, "sparse_attn", None) or getattr(K, "sparse_attn", None)
    if orig is None or _sparse_backend_preference() == "official":
        return False
    if getattr(orig, MARK, False):
        return True
    import sglang_lite_amd

    if not sglang_lite_amd.probe().get("ok"):
        return False

    def routed(q, kv, attn_sink, topk_idxs, softmax_scale):
        return sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale)

    setattr(routed, MARK, True)
    routed._official = orig  # type: ignore[attr-defined]
    for mod in (K, M):
        if mod is not None and getattr(mod, "sparse_attn", None) is not None:
            mod.sparse_attn = routed
    if backend is not None:
        try:
            backend._official_sparse_attn = orig
            backend._v4_sparse_attn_routed = routed
        except Exception:  # noqa: BLE001
            pass
    print("[sglang-lite-amd] v4 sparse: gfx950 HIP path (prefill + decode, bf16 MFMA)")
    return True


def detach_v4_sparse_mla() -> None:
    for name in ("kernel", "model"):
        mod = sys.modules.get(name)
        f = getattr(mod, "sparse_attn", None) if mod is not None else None
        if f is not None and getattr(f, MARK, False):
            mod.sparse_attn = f._official


__all__ = ["attach_v4_sparse_mla", "detach_v4_sparse_mla", "sparse_attn", "sparse_attn_packed"]
