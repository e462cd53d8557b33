"""Oracle: FP8 x MXFP4 GEMM and the FP4 -> FP8 weight repack, restated in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Formats.  An FP4 weight is stored as ``[N, K/2]`` bytes of packed OCP e2m1
codes (torch ``float4_e2m1fn_x2``): byte ``b`` of a row holds logical element
``2b`` in its low nibble and ``2b + 1`` in its high nibble
(deepseek_infer/convert.py:31-33 unpacks ``low`` first).  Its scales are one
e8m0 byte per 32 consecutive K elements, ``[N, K/32]``
(deepseek_infer/model.py:129-137).
"""

from __future__ import annotations

import numpy as np

from . import quant as Q

# deepseek_infer/convert.py:11-14 (the OCP MX e2m1 value set: sign, 2-bit
# exponent with bias 1, 1-bit mantissa).  Code 8 is the format's -0; the
# converter's table (and deep_gemm_sm120/utils/math.py `_dequantize_from_fp4_e2m1`,
# which negates only nonzero magnitudes) give +0.0 there, so the repack of a
# code-8 nibble is the e4m3 byte 0x00.
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                 0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


def e2m1_to_f32(code: np.ndarray) -> np.ndarray:
    return E2M1[np.asarray(code, dtype=np.uint8) & 0xF]


def unpack_fp4(packed: np.ndarray) -> np.ndarray:
    """[N, K/2] packed bytes -> [N, K] e2m1 codes (low nibble first)."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0x0F
    out[..., 1::2] = p >> 4
    return out


def pack_fp4(codes: np.ndarray) -> np.ndarray:
    """[N, K] e2m1 codes -> [N, K/2] packed bytes (inverse of unpack_fp4)."""
    c = np.asarray(codes, dtype=np.uint8) & 0xF
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def e8m0_to_f32(b: np.ndarray) -> np.ndarray:
    """float8_e8m0fnu -> float32 (torch ``.float()``): 2^(b - 127), 0xFF NaN."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    out = np.exp2(np.minimum(b - 127, 127).astype(np.float64)).astype(np.float32)
    out[b == 0xFF] = np.nan
    return out


# value pair (low nibble, high nibble) of every packed byte
_PAIR = np.stack([E2M1[np.arange(256) & 0xF], E2M1[np.arange(256) >> 4]], axis=-1).astype(np.float32)


def dequant_fp4(packed: np.ndarray, sb: np.ndarray) -> np.ndarray:
    """fp32 value of an FP4 weight: e2m1 * 2^(e8m0 - 127) per 1 x 32 block
    (exact: a power-of-two scale times a 2-bit significand)."""
    p = np.asarray(packed, dtype=np.uint8)
    v = _PAIR[p].reshape(*p.shape[:-1], p.shape[-1] * 2)
    s = e8m0_to_f32(sb)
    g = v.reshape(*v.shape[:-1], v.shape[-1] // 32, 32) * s[..., None]
    return g.reshape(v.shape).astype(np.float32)


def fp4_gemm(aq: np.ndarray, sa: np.ndarray, bp: np.ndarray, sb: np.ndarray,
             out_bf16: bool = True) -> np.ndarray:
    """deepseek_infer/kernel.py:519-536 fp4_gemm as a dequantize-to-fp32
    reference: C = (A_e4m3 * sa[m, k/128]) @ (B_e2m1 * sb[n, k/32])^T, summed
    in float64, rounded once to fp32 (and to bf16 when ``out_bf16``)."""
    a = Q.dequant_rows(aq, sa, 128).astype(np.float64)
    b = dequant_fp4(bp, sb).astype(np.float64)
    c = (a @ b.T).astype(np.float32)
    return Q.bf16_round(c) if out_bf16 else c


def fp4_gemm_blocked(aq: np.ndarray, sa: np.ndarray, bp: np.ndarray, sb: np.ndarray) -> np.ndarray:
    """The TileLang kernel's accumulation structure (kernel.py:485-513): for
    every 32-deep K block an fp32 partial of the unscaled e4m3 x e2m1 products
    (exact: each product has at most 5 significant bits and 32 of them fit
    fp32), then ``acc += partial * sa[m, k/128] * sb[n, k/32]`` in fp32,
    left to right.  Returns fp32 [M, N]."""
    a = Q.e4m3_to_f32(aq).astype(np.float64)
    b = e2m1_to_f32(unpack_fp4(bp)).astype(np.float64)
    M, K = a.shape
    N = b.shape[0]
    saf = np.asarray(sa, dtype=np.float32)
    sbf = e8m0_to_f32(sb)
    acc = np.zeros((M, N), dtype=np.float32)
    for kb in range(K // 32):
        sl = slice(kb * 32, (kb + 1) * 32)
        part = (a[:, sl] @ b[:, sl].T).astype(np.float32)
        t = (part * saf[:, kb // 4][:, None]).astype(np.float32)
        acc = (acc + (t * sbf[:, kb][None, :]).astype(np.float32)).astype(np.float32)
    return acc


def fp4_to_fp8_repack(bp: np.ndarray, sb: np.ndarray):
    """deepseek_infer/convert.py:17-52 cast_e2m1fn_to_e4m3fn.

    Per 128 x 128 block: smax = max of the block's 512 (power-of-two) scales,
    s = smax / 2^6; each element becomes e4m3(e2m1 * (scale / s)) (|value| <=
    6 * 2^6 = 384 < 448, exact unless a scale sits more than 2^6 below smax and
    the product needs e4m3 subnormal rounding).  Returns
    (q e4m3 uint8 [N, K], s e8m0 uint8 [N/128, K/128])."""
    codes = unpack_fp4(bp)
    N, K = codes.shape
    if N % 128 or K % 128:
        raise ValueError("repack needs N and K multiples of 128")
    v = e2m1_to_f32(codes).astype(np.float64)
    sf = e8m0_to_f32(sb).astype(np.float64)  # [N, K/32]
    blk = sf.reshape(N // 128, 128, K // 128, 4)
    smax = blk.max(axis=(1, 3))  # [N/128, K/128]
    s = smax / 64.0
    off = sf / np.repeat(np.repeat(s, 128, axis=0), 4, axis=1)  # [N, K/32], powers of two
    q = Q.f32_to_e4m3((v * np.repeat(off, 32, axis=1)).astype(np.float32))
    return q, Q.e8m0_byte(s.astype(np.float32))


def quant_fp4_weight(w: np.ndarray):
    """Synthetic MXFP4 weight from fp32 [N, K] (a test-input generator, not a
    restated kernel): per 1 x 32 block scale 2^ceil(log2(amax / 6)) (the
    power-of-two rule of kernel.py:128-200 fp4_quant_kernel), codes = nearest
    e2m1 value of w / scale, ties to the even code.  Returns (packed, sb e8m0)."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    g = w.reshape(N, K // 32, 32).astype(np.float64)
    amax = np.maximum(np.abs(g).max(axis=-1), 6.0 * 2.0**-126)
    e = np.ceil(np.log2(amax / 6.0))
    scale = np.exp2(e)
    y = np.clip(g / scale[..., None], -6.0, 6.0)
    mag = np.abs(y)
    grid = E2M1[:8].astype(np.float64)
    d = np.abs(mag[..., None] - grid)  # distance to each magnitude
    best = np.argmin(d + (np.arange(8) % 2) * 1e-12, axis=-1)  # ties -> even code
    codes = (best | np.where(np.signbit(y) & (best > 0), 8, 0)).astype(np.uint8)
    sb = (e + 127).astype(np.uint8)
    return pack_fp4(codes.reshape(N, K)), sb


def make_fp4_weight(rng: np.random.Generator, N: int, K: int, std: float = 0.02):
    """Synthetic N(0, std) weight quantized to MXFP4 (packed, sb)."""
    w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return quant_fp4_weight(w)
