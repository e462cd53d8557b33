"""DeepSeek-V4 packed FP8 KV rows on gfx950: drop-in for ``engine/dsv4_kv_pack.py``.

Same constants, function names, argument meaning, shapes and exceptions as
the reference module (``dsv4_kv_pack.py:28-175``); every function runs a HIP
kernel and refuses CPU tensors.

Layout A (the reference's, 584 B logical row, :3-37)::

    [0:448)   NoPE as e4m3 in blocks of 64
    [448:576) RoPE as 64 x bf16 (bytes as given)
    [576:583) 7 x ue8m0 block scales
    [583]     0

Footer pages of ``page_size`` rows (:104-146): ``[page*576 data | page*8 scales]``.

Layout B (576-dim latent+rope rows, no reference producer; 656 B)::

    [0:512)   latent as e4m3, 4 groups of 128, SGL_SCALE_TORCH_FP32 formula
    [512:640) RoPE as 64 x bf16
    [640:656) 4 x fp32 scales (little endian)

``act_quant_fn`` (dsv4_kv_pack.py:58-61): None quantizes with the reference's
torch fallback formula (``_torch_fp8_ue8m0_quant``, :78-101); the official
``kernel.act_quant`` (TileLang, ``kernel.py:22-37,79-96``) or this package's
``kernel.act_quant`` are computed by the fused HIP kernel with that
function's ue8m0 formula; any other function is called on the NoPE part as
the reference calls it, and its bytes are packed.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

DSV4_HEAD_DIM = 512
DSV4_NOPE_DIM = 448
DSV4_ROPE_DIM = 64
DSV4_PACKED_BYTES = 584
DSV4_DATA_BYTES = 576
DSV4_SCALE_BYTES = 7
DSV4_SCALE_STRIDE = 8
DSV4_FP8_BLOCK = 64
DSV4_PAGE_SIZE = 64
DSV4_FP8_MAX = 448.0

LATENT_DIM = 512
LATENT_ROPE_DIM = 576
LATENT_PACKED_BYTES = 656

_DT = {torch.bfloat16: _lib.SGL_BF16, torch.float16: _lib.SGL_F16, torch.float32: _lib.SGL_F32}


def _rows(x: torch.Tensor, dim: int) -> Tuple[torch.Tensor, int]:
    z = x.reshape(-1, dim)
    if z.stride(-1) != 1 or (z.numel() and z.stride(0) < dim):
        z = z.contiguous()
    if z.numel() and (z.data_ptr() % 16 or (z.stride(0) * z.element_size()) % 16):
        z = z.contiguous()
    return z, z.shape[0]


def _fused_quant_mode(act_quant_fn) -> Optional[int]:
    """The sgl_scale_mode the fused pack kernel computes in place of
    ``act_quant_fn(nope, 64, "ue8m0", float8_e8m0fnu, False)``, or None when
    the function is not one whose formula the kernel holds (then it is called)."""
    if act_quant_fn is None:
        return _lib.SCALE_KV_UE8M0
    from . import kernel as HK

    # this package's act_quant, or a wrapper of it such as the kernel.act_quant
    # that attach_v4_deep_gemm installs (v4_sparse_mla.py:85,91 resolves that name)
    if act_quant_fn is HK.act_quant or getattr(act_quant_fn, HK.FUSED_ACT_QUANT, False):
        return HK.scale_mode_for("ue8m0")
    if getattr(act_quant_fn, "__module__", None) == "kernel" and \
            getattr(act_quant_fn, "__name__", None) == "act_quant":
        return _lib.SCALE_TILELANG_UE8M0  # the official TileLang act_quant's ue8m0 rule
    return None


def _pack_rows_with(kv: torch.Tensor, act_quant_fn) -> torch.Tensor:
    """dsv4_kv_pack.py:55-75 with a caller's quantizer: call it on the NoPE
    part and place its e4m3 bytes, the RoPE bytes and its 7 e8m0 scale bytes."""
    nope = kv[..., :DSV4_NOPE_DIM].contiguous()
    rope = kv[..., DSV4_NOPE_DIM:].contiguous()
    y, s = act_quant_fn(nope, DSV4_FP8_BLOCK, "ue8m0", torch.float8_e8m0fnu, False)
    out = torch.empty(*kv.shape[:-1], DSV4_PACKED_BYTES, dtype=torch.uint8, device=kv.device)
    out[..., :DSV4_NOPE_DIM] = y.view(torch.uint8).view(*y.shape[:-1], DSV4_NOPE_DIM)
    out[..., DSV4_NOPE_DIM:DSV4_DATA_BYTES] = rope.view(torch.uint8).view(
        *rope.shape[:-1], DSV4_ROPE_DIM * 2)
    out[..., DSV4_DATA_BYTES:DSV4_DATA_BYTES + DSV4_SCALE_BYTES] = s.view(torch.uint8).view(
        *s.shape[:-1], DSV4_SCALE_BYTES)
    out[..., DSV4_PACKED_BYTES - 1] = 0
    return out


def pack_dsv4_kv_bf16(kv: torch.Tensor, *, act_quant_fn=None) -> torch.Tensor:
    """Pack KV ``[..., 512]`` -> logical uint8 ``[..., 584]`` (dsv4_kv_pack.py:40-75)."""
    if kv.shape[-1] != DSV4_HEAD_DIM:
        raise ValueError(f"expected head_dim={DSV4_HEAD_DIM}, got {kv.shape[-1]}")
    if kv.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"unsupported kv dtype {kv.dtype}")
    _lib.require_device(kv, what="pack_dsv4_kv_bf16")
    if kv.dtype == torch.float32:
        # the reference views fp32 rope bytes into a 128-byte slot, which fails
        raise RuntimeError("pack_dsv4_kv_bf16: fp32 rope does not fit the 128-byte rope slot")
    mode = _fused_quant_mode(act_quant_fn)
    if mode is None:
        return _pack_rows_with(kv, act_quant_fn)
    z, T = _rows(kv, DSV4_HEAD_DIM)
    out = torch.empty(*kv.shape[:-1], DSV4_PACKED_BYTES, dtype=torch.uint8, device=kv.device)
    _lib.call("sgl_kv_pack", _lib.ptr(z) if T else None, _DT[kv.dtype], T,
              z.stride(0) if T else DSV4_HEAD_DIM, _lib.KV_LAYOUT_A, mode, 0, 0,
              out.data_ptr(), _lib.stream_of(kv))
    return out


def pack_dsv4_kv_paged(kv: torch.Tensor, page_size: int = DSV4_PAGE_SIZE, *,
                       act_quant_fn=None) -> torch.Tensor:
    """Fused ``to_paged_hnd(pack_dsv4_kv_bf16(kv), page_size)`` for ``[T, 512]``:
    one kernel writes the footer pages (``[P, 1, page_size, 584]``) directly."""
    if kv.dim() != 2 or kv.shape[-1] != DSV4_HEAD_DIM:
        raise ValueError(f"expected [T, {DSV4_HEAD_DIM}], got {tuple(kv.shape)}")
    if kv.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"unsupported kv dtype {kv.dtype}")
    _lib.require_device(kv, what="pack_dsv4_kv_paged")
    mode = _fused_quant_mode(act_quant_fn)
    if mode is None:
        return to_paged_hnd(_pack_rows_with(kv, act_quant_fn), page_size)
    z, T = _rows(kv, DSV4_HEAD_DIM)
    n_pages = (T + page_size - 1) // page_size
    out = torch.empty(n_pages, 1, page_size, DSV4_PACKED_BYTES, dtype=torch.uint8, device=kv.device)
    _lib.call("sgl_kv_pack", _lib.ptr(z) if T else None, _DT[kv.dtype], T,
              z.stride(0) if T else DSV4_HEAD_DIM, _lib.KV_LAYOUT_A, mode, 1, page_size,
              out.data_ptr(), _lib.stream_of(kv))
    return out


def write_packed_kv_bf16(pool: torch.Tensor, block_table, start_pos: int, kv: torch.Tensor, *,
                         layer_idx: int = 0, act_quant_fn=None) -> None:
    """Packed-page writer: ``pack_dsv4_kv_bf16(kv)`` written straight into a
    RadixCache packed pool ``[layers, blocks, 1, page, 584]`` (the write of
    engine/kv_cache.py:340-390 ``write_packed_kv`` as
    engine/v4_dual_pool.py:73-128 feeds it) in one kernel.  ``block_table`` is
    a list of block ids (checked on the host against the pool, as the
    reference does) or a device int32 tensor (graph-capturable; entries
    outside the pool are skipped).  ``act_quant_fn`` must be None or an
    ``act_quant`` whose formula the fused kernel holds (the official or this
    package's); rows quantized by another function are packed with
    ``pack_dsv4_kv_bf16`` and written by the caller."""
    mode = _fused_quant_mode(act_quant_fn)
    if mode is None:
        raise TypeError("write_packed_kv_bf16: act_quant_fn must be None or kernel.act_quant; "
                        "pack rows from another quantizer with pack_dsv4_kv_bf16")
    if pool.dim() != 5 or pool.dtype != torch.uint8 or pool.shape[2] != 1 or \
            pool.shape[-1] != DSV4_PACKED_BYTES or not pool.is_contiguous():
        raise ValueError(f"expected a contiguous uint8 [layers, blocks, 1, page, 584] pool, "
                         f"got {pool.dtype} {tuple(pool.shape)}")
    num_layers, num_blocks, _, page, _ = pool.shape
    if layer_idx < 0 or layer_idx >= num_layers:
        raise ValueError(f"layer_idx {layer_idx} out of range ({num_layers})")
    if kv.shape[-1] != DSV4_HEAD_DIM:
        raise ValueError(f"expected head_dim={DSV4_HEAD_DIM}, got {kv.shape[-1]}")
    if kv.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"unsupported kv dtype {kv.dtype}")
    _lib.require_device(pool, kv, what="write_packed_kv_bf16")
    if not isinstance(block_table, torch.Tensor):
        if not block_table:
            raise ValueError("write_packed_kv requires block_table")
        bad = [b for b in block_table if not 0 <= int(b) < num_blocks]
        if bad:
            raise RuntimeError(f"block id {bad[0]} out of range ({num_blocks})")
        block_table = torch.tensor([int(b) for b in block_table], dtype=torch.int32).to(pool.device)
    bt = block_table.to(torch.int32).contiguous()
    _lib.require_device(bt, what="write_packed_kv_bf16")
    z, T = _rows(kv, DSV4_HEAD_DIM)
    if T == 0:
        return
    try:
        _lib.call("sgl_kv_pack_to_pages", z.data_ptr(), _DT[kv.dtype], T, z.stride(0), mode,
                  bt.data_ptr(), bt.numel(), int(start_pos), int(page), int(num_blocks),
                  int(layer_idx), int(num_layers), pool.data_ptr(), _lib.stream_of(kv))
    except ValueError as e:  # the reference raises RuntimeError for a short table
        if "block_table too short" in str(e):
            raise RuntimeError(str(e)) from None
        raise


def fp8_ue8m0_quant(x: torch.Tensor, block_size: int = DSV4_FP8_BLOCK):
    """The reference's ``_torch_fp8_ue8m0_quant`` (dsv4_kv_pack.py:78-101) on the
    device: returns ``(y float8_e4m3fn, s float8_e8m0fnu [..., n // block])``."""
    n = x.shape[-1]
    if n % block_size != 0:
        raise ValueError(f"last dim {n} not divisible by block_size={block_size}")
    from .kernel import act_quant

    if x.dtype != torch.bfloat16:
        raise TypeError(f"fp8_ue8m0_quant: expected bfloat16 input, got {x.dtype}")
    return act_quant(x, block_size, "ue8m0", torch.float8_e8m0fnu, False,
                     scale_mode=_lib.SCALE_KV_UE8M0)


def to_paged_hnd(packed_tokens: torch.Tensor, page_size: int = DSV4_PAGE_SIZE) -> torch.Tensor:
    """``[T, 584]`` logical -> ``[num_pages, 1, page_size, 584]`` footer pages
    (dsv4_kv_pack.py:104-146); padding rows are zero."""
    if packed_tokens.dim() != 2 or packed_tokens.shape[-1] != DSV4_PACKED_BYTES:
        raise ValueError(f"expected [T, 584], got {tuple(packed_tokens.shape)}")
    _lib.require_device(packed_tokens, what="to_paged_hnd")
    src = packed_tokens.contiguous()
    t = src.shape[0]
    n_pages = (t + page_size - 1) // page_size
    physical = torch.empty(n_pages, page_size * DSV4_PACKED_BYTES, dtype=torch.uint8,
                           device=src.device)
    _lib.call("sgl_kv_to_paged", _lib.ptr(src) if t else None, t, page_size,
              physical.data_ptr(), _lib.stream_of(src))
    return physical.view(n_pages, 1, page_size, DSV4_PACKED_BYTES)


def split_swa_compress_indices(
    topk_idxs: torch.Tensor,
    window_size: int,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Split concatenated top-k ``[B, S, K]`` into SWA + compressed (relative)
    indices (dsv4_kv_pack.py:149-175).  Returns int32
    ``(swa_idx [B*S, min(W,K)], swa_lens [B*S], comp_idx [B*S, K-swa], comp_lens [B*S])``."""
    if topk_idxs.dim() != 3:
        raise ValueError(f"expected [B,S,K], got {tuple(topk_idxs.shape)}")
    _lib.require_device(topk_idxs, what="split_swa_compress_indices")
    if topk_idxs.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"expected int32/int64 indices, got {topk_idxs.dtype}")
    b, s, k = topk_idxs.shape
    swa_k = min(window_size, k)
    src = topk_idxs.contiguous()
    dev = src.device
    swa = torch.empty(b * s, swa_k, dtype=torch.int32, device=dev)
    swa_lens = torch.empty(b * s, dtype=torch.int32, device=dev)
    comp = torch.empty(b * s, k - swa_k, dtype=torch.int32, device=dev)
    comp_lens = torch.empty(b * s, dtype=torch.int32, device=dev)
    _lib.call("sgl_split_swa_compress_indices", _lib.ptr(src) if src.numel() else None,
              int(src.dtype == torch.int64), b * s, k, int(window_size),
              _lib.ptr(swa) if swa.numel() else None, swa_lens.data_ptr(),
              _lib.ptr(comp) if comp.numel() else None, comp_lens.data_ptr(), _lib.stream_of(src))
    return swa, swa_lens, comp, comp_lens


def pack_kv_latent_rope(kv: torch.Tensor) -> torch.Tensor:
    """Layout B: ``[..., 576]`` (512 latent + 64 rope) -> uint8 ``[..., 656]``."""
    if kv.shape[-1] != LATENT_ROPE_DIM:
        raise ValueError(f"expected last dim {LATENT_ROPE_DIM}, got {kv.shape[-1]}")
    if kv.dtype not in _DT:
        raise TypeError(f"unsupported kv dtype {kv.dtype}")
    _lib.require_device(kv, what="pack_kv_latent_rope")
    z, T = _rows(kv, LATENT_ROPE_DIM)
    out = torch.empty(*kv.shape[:-1], LATENT_PACKED_BYTES, dtype=torch.uint8, device=kv.device)
    _lib.call("sgl_kv_pack", _lib.ptr(z) if T else None, _DT[kv.dtype], T,
              z.stride(0) if T else LATENT_ROPE_DIM, _lib.KV_LAYOUT_B, _lib.SCALE_TORCH_FP32, 0,
              0, out.data_ptr(), _lib.stream_of(kv))
    return out


def gather_dequant(cache: torch.Tensor, indices: torch.Tensor, *, layout: str = "A",
                   page_size: Optional[int] = None, out: Optional[torch.Tensor] = None
                   ) -> torch.Tensor:
    """Sparse-MLA gather-dequant: ``out[q, i] = dequant(cache[indices[q, i]])``
    as bf16, zero rows for index -1.

    ``cache``: layout A logical ``[T, 584]``, layout A footer pages
    ``[P, 1, page, 584]`` (pass ``page_size``), or layout B ``[T, 656]``.
    ``indices``: int32 ``[nq, nsel]``.  Returns bf16 ``[nq, nsel, 512 | 576]``."""
    _lib.require_device(cache, indices, what="gather_dequant")
    if indices.dtype != torch.int32 or indices.dim() != 2:
        raise TypeError("gather_dequant: indices must be int32 [nq, nsel]")
    lay = {"A": _lib.KV_LAYOUT_A, "B": _lib.KV_LAYOUT_B}[layout]
    c = cache.contiguous()
    paged = page_size is not None
    if lay == _lib.KV_LAYOUT_A:
        if paged:
            if c.dim() != 4 or c.shape[-1] != DSV4_PACKED_BYTES or c.shape[2] != page_size:
                raise ValueError(f"expected [P, 1, {page_size}, 584] pages, got {tuple(c.shape)}")
            n_rows = c.shape[0] * page_size
        else:
            if c.dim() != 2 or c.shape[-1] != DSV4_PACKED_BYTES:
                raise ValueError(f"expected [T, 584], got {tuple(c.shape)}")
            n_rows = c.shape[0]
        odim = DSV4_HEAD_DIM
    else:
        if paged or c.dim() != 2 or c.shape[-1] != LATENT_PACKED_BYTES:
            raise ValueError(f"expected [T, 656] layout-B rows, got {tuple(c.shape)}")
        n_rows = c.shape[0]
        odim = LATENT_ROPE_DIM
    idx = indices.contiguous()
    nq, nsel = idx.shape
    if out is None:
        out = torch.empty(nq, nsel, odim, dtype=torch.bfloat16, device=c.device)
    _lib.call("sgl_kv_gather_dequant", _lib.ptr(c) if c.numel() else None, lay, int(paged),
              int(page_size or 0), n_rows, idx.data_ptr(), nq, nsel, out.data_ptr(),
              _lib.stream_of(c))
    return out


__all__ = [
    "DSV4_DATA_BYTES", "DSV4_FP8_BLOCK", "DSV4_FP8_MAX", "DSV4_HEAD_DIM", "DSV4_NOPE_DIM",
    "DSV4_PACKED_BYTES", "DSV4_PAGE_SIZE", "DSV4_ROPE_DIM", "DSV4_SCALE_BYTES",
    "DSV4_SCALE_STRIDE", "LATENT_PACKED_BYTES", "fp8_ue8m0_quant", "gather_dequant",
    "pack_dsv4_kv_bf16", "pack_dsv4_kv_paged", "pack_kv_latent_rope", "split_swa_compress_indices",
    "to_paged_hnd", "write_packed_kv_bf16",
]
