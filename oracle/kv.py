"""Oracle: FP8 KV pack (layouts A and B), footer paging, gather-dequant and
index split, restated in numpy.  Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

from . import quant as Q

NOPE, ROPE, HEAD = 448, 64, 512
ROW_A, DATA_A = 584, 576
LAT, ROW_B = 512, 656


def pack_layout_a(kv: np.ndarray, rope_bytes: np.ndarray, scale_mode: int = 4) -> np.ndarray:
    """engine/dsv4_kv_pack.py:40-75 pack_dsv4_kv_bf16.

    ``kv``: float32 [T, 512] holding the input values; ``rope_bytes``: uint8
    [T, 128], the RoPE part's raw 16-bit bytes (copied verbatim, :69-71).
    scale_mode 4 = the torch fallback (:78-101); 3 = the injected
    ``act_quant(..., "ue8m0", float8_e8m0fnu)`` (:58-61, kernel.py:22-37,79-96);
    1 = an injected quantizer with the torch ue8m0 formula
    (deep_gemm_sm120/utils/math.py:13-37, group 64).
    """
    kv = np.asarray(kv, dtype=np.float32)
    T = kv.shape[0]
    nope = kv[:, :NOPE]
    if scale_mode == 4:
        q, s = Q.kv_ue8m0_quant(nope, 64)
    elif scale_mode == 3:
        q, s = Q.act_quant_tilelang(nope, 64, round_scale=True)
    elif scale_mode == 1:
        q, s = Q.per_token_cast_to_fp8(nope, True, 64)
    else:
        raise ValueError(scale_mode)
    out = np.zeros((T, ROW_A), dtype=np.uint8)
    out[:, :NOPE] = q
    out[:, NOPE:DATA_A] = rope_bytes
    out[:, DATA_A:DATA_A + 7] = Q.e8m0_byte(s)
    out[:, 583] = 0
    return out


def to_paged_hnd(packed: np.ndarray, page_size: int = 64) -> np.ndarray:
    """engine/dsv4_kv_pack.py:104-146: pad to pages with zero rows; each page is
    ``[page*576 data bytes | page*8 scale bytes]``, viewed [P, 1, page, 584]."""
    t = packed.shape[0]
    pad = (page_size - t % page_size) % page_size
    if pad:
        packed = np.concatenate([packed, np.zeros((pad, ROW_A), np.uint8)], axis=0)
    n = packed.shape[0] // page_size
    logical = packed.reshape(n, page_size, ROW_A)
    phys = np.empty((n, page_size * ROW_A), dtype=np.uint8)
    phys[:, : page_size * DATA_A] = logical[:, :, :DATA_A].reshape(n, -1)
    phys[:, page_size * DATA_A:] = logical[:, :, DATA_A:].reshape(n, -1)
    return phys.reshape(n, 1, page_size, ROW_A)


def pack_layout_b(latent: np.ndarray, rope_bytes: np.ndarray) -> np.ndarray:
    """Layout B (no reference producer; closed form): latent [T, 512] quantized
    1x128 with the torch fp32 formula (utils/math.py:25-37), rope bytes verbatim,
    then the 4 fp32 scales little endian.  Row = 656 bytes."""
    q, s = Q.per_token_cast_to_fp8(np.asarray(latent, np.float32), False, 128)
    T = q.shape[0]
    out = np.zeros((T, ROW_B), dtype=np.uint8)
    out[:, :LAT] = q
    out[:, LAT:640] = rope_bytes
    out[:, 640:656] = np.ascontiguousarray(s.astype("<f4")).view(np.uint8).reshape(T, 16)
    return out


def dequant_row_a(rows: np.ndarray) -> np.ndarray:
    """Layout A row -> 512 fp32 values: e4m3 * 2^(e8m0 - 127) (exact; the
    quant-dequant of kernel.py:84-91 with power-of-two scales) + rope (bf16)."""
    rows = np.asarray(rows, dtype=np.uint8)
    n = rows.shape[0]
    q = Q.e4m3_to_f32(rows[:, :NOPE]).reshape(n, 7, 64)
    s = np.ldexp(np.float32(1.0), rows[:, DATA_A:DATA_A + 7].astype(np.int32) - 127).astype(np.float32)
    nope = (q * s[:, :, None]).reshape(n, NOPE)
    rope = Q.bits_to_bf16_f32(np.ascontiguousarray(rows[:, NOPE:DATA_A]).view("<u2"))
    return np.concatenate([nope, rope], axis=1).astype(np.float32)


def dequant_row_b(rows: np.ndarray) -> np.ndarray:
    """Layout B row -> 576 bf16 values: bf16(fp32(e4m3) * scale) + rope."""
    rows = np.asarray(rows, dtype=np.uint8)
    n = rows.shape[0]
    q = Q.e4m3_to_f32(rows[:, :LAT]).reshape(n, 4, 128)
    s = np.ascontiguousarray(rows[:, 640:656]).view("<f4").reshape(n, 4)
    lat = Q.bf16_round((q * s[:, :, None]).astype(np.float32).reshape(n, LAT))
    rope = Q.bits_to_bf16_f32(np.ascontiguousarray(rows[:, LAT:640]).view("<u2"))
    return np.concatenate([lat, rope], axis=1).astype(np.float32)


def gather_dequant(rows: np.ndarray, idx: np.ndarray, layout: str = "A") -> np.ndarray:
    """Closed form of the sparse-MLA gather (engine/v4_sparse_torch.py:77-83,
    deepseek_infer/kernel.py:322-325): out[q, i] = dequant(rows[idx[q, i]]),
    zero row for -1 (and for indices past the end)."""
    idx = np.asarray(idx)
    deq = dequant_row_a(rows) if layout == "A" else dequant_row_b(rows)
    dim = deq.shape[1]
    valid = (idx >= 0) & (idx < rows.shape[0])
    out = np.zeros(idx.shape + (dim,), dtype=np.float32)
    out[valid] = deq[idx[valid]]
    return out


def unpage(pages: np.ndarray, page_size: int) -> np.ndarray:
    """Inverse of to_paged_hnd: footer pages -> logical [P*page, 584] rows."""
    n = pages.shape[0]
    flat = pages.reshape(n, page_size * ROW_A)
    data = flat[:, : page_size * DATA_A].reshape(n, page_size, DATA_A)
    foot = flat[:, page_size * DATA_A:].reshape(n, page_size, 8)
    return np.concatenate([data, foot], axis=2).reshape(n * page_size, ROW_A)


def split_swa_compress_indices(topk: np.ndarray, window: int
                               ) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """engine/dsv4_kv_pack.py:149-175."""
    b, s, k = topk.shape
    swa_k = min(window, k)
    swa = topk[:, :, :swa_k].reshape(b * s, swa_k).astype(np.int32)
    swa_lens = (swa >= 0).sum(axis=-1).astype(np.int32)
    if k > swa_k:
        comp = topk[:, :, swa_k:].reshape(b * s, k - swa_k).astype(np.int32)
        valid = comp >= 0
        comp = np.where(valid, comp - window, comp).astype(np.int32)
        comp_lens = valid.sum(axis=-1).astype(np.int32)
    else:
        comp = np.zeros((b * s, 0), np.int32)
        comp_lens = np.zeros(b * s, np.int32)
    return swa, swa_lens, comp, comp_lens


def write_packed_pages(pool: np.ndarray, block_table, start_pos: int, rows: np.ndarray,
                       layer_idx: int) -> np.ndarray:
    """engine/kv_cache.py:340-390 write_packed_kv: token start_pos + t goes to
    pool[layer, block_table[(start_pos + t) // page], 0, (start_pos + t) % page].
    ``pool`` uint8 [layers, blocks, 1, page, D]; returns the updated copy."""
    out = np.array(pool, copy=True)
    page = out.shape[3]
    for t in range(rows.shape[0]):
        pos = start_pos + t
        out[layer_idx, block_table[pos // page], 0, pos % page] = rows[t]
    return out
