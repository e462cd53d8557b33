"""Oracle: FP8 e4m3 quantization formulas of the reference, restated in numpy.

Test infrastructure only (see ``oracle/__init__.py``).  Arrays are float32
unless stated; bf16 inputs are passed as float32 arrays holding bf16 values.
"""

from __future__ import annotations

import numpy as np

FP8_MAX = np.float32(448.0)
INV448 = np.float32(1.0) / np.float32(448.0)  # fp32(1/448): torch scalar ops use it

# ------------------------------------------------------------------ formats


def _e4m3_decode(code: np.ndarray) -> np.ndarray:
    """OCP e4m3fn bytes -> float32 from the bit fields (exact): sign bit 7,
    exponent bits 6..3 with bias 7 (0 = subnormal, m * 2^-9), mantissa bits
    2..0; S.1111.111 is NaN."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0**-9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = (sign * mag).astype(np.float32)
    out[(e == 0xF) & (m == 0x7)] = np.nan
    return out


_E4M3_LUT = _e4m3_decode(np.arange(256, dtype=np.uint8))


def e4m3_to_f32(code: np.ndarray) -> np.ndarray:
    """Decode OCP e4m3fn bytes (exact): the bit-field decode tabulated over
    all 256 codes."""
    return _E4M3_LUT[np.asarray(code, dtype=np.uint8)]


# the 127 non-negative finite e4m3 values, increasing with the code
_E4M3_POS = e4m3_to_f32(np.arange(127, dtype=np.uint8)).astype(np.float64)


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest e4m3fn code, ties to the even code.

    Restates torch's ``Tensor.to(torch.float8_e4m3fn)`` (used by
    deep_gemm_sm120/utils/math.py:36 and engine/dsv4_kv_pack.py:95-97):
    magnitudes above 464 (the midpoint of 448 and the NaN code) and NaN/Inf
    give the NaN code S.1111.111.  Implemented by table search over the 127
    representable magnitudes, independently of the kernels' bit arithmetic.
    """
    xf = np.asarray(x, dtype=np.float32)
    bits = xf.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    with np.errstate(invalid="ignore"):
        a = np.abs(xf.astype(np.float64))
    out = np.zeros(xf.shape, dtype=np.uint8)
    nanlike = ~np.isfinite(a) | (a > 464.0)
    fin = ~nanlike
    af = np.where(fin, np.minimum(a, 448.0), 0.0)
    hi = np.searchsorted(_E4M3_POS, af, side="left")  # first value >= af
    hi = np.clip(hi, 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    vlo = _E4M3_POS[lo]
    vhi = _E4M3_POS[hi]
    dlo = af - vlo
    dhi = vhi - af
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((hi & 1) == 0))
    code = np.where(af == vhi, hi, np.where(pick_hi, hi, lo))
    # 448 < |x| <= 464 rounds to 448 (464 ties to the even code 0x7E)
    code = np.where(a > 448.0, 126, code)
    out[fin] = code[fin].astype(np.uint8)
    out[nanlike] = 0x7F
    return out | sign


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest even), returned as float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    isn = np.isnan(np.asarray(x, dtype=np.float32))
    if isn.any():
        out = out.copy()
        out[isn] = np.float32(np.nan)
    return out


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 values after RNE rounding."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_bf16_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def ceil_to_ue8m0(x: np.ndarray) -> np.ndarray:
    """deep_gemm_sm120/utils/math.py:13-16: next power of two >= |x|,
    biased exponent clamped to [1, 254]."""
    bits = np.abs(np.asarray(x, dtype=np.float32)).view(np.uint32)
    exp = ((bits >> 23) & 0xFF).astype(np.int64) + ((bits & 0x7FFFFF) != 0)
    return (np.clip(exp, 1, 254).astype(np.uint32) << 23).view(np.float32)


def pow2_ceil_log2_bits(x: np.ndarray) -> np.ndarray:
    """deepseek_infer/kernel.py:22-37 fast_round_scale: 2^(exponent + (mantissa != 0))."""
    bits = np.asarray(x, dtype=np.float32).view(np.uint32)
    e = ((bits >> 23) & 0xFF).astype(np.int64) - 127 + ((bits & 0x7FFFFF) != 0)
    return ((e + 127).astype(np.uint32) << 23).view(np.float32)


def e8m0_byte(p: np.ndarray) -> np.ndarray:
    """e8m0 byte of exact powers of two (torch float8_e8m0fnu cast of 2^k)."""
    return ((np.asarray(p, dtype=np.float32).view(np.uint32) >> 23) & 0xFF).astype(np.uint8)


# ---------------------------------------------------------- group formulas


def _groups(x: np.ndarray, group: int) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if x.shape[-1] % group != 0:
        raise ValueError(f"last dim {x.shape[-1]} not divisible by group {group}")
    return x.reshape(*x.shape[:-1], x.shape[-1] // group, group)


def _amax(g: np.ndarray) -> np.ndarray:
    # NaN propagates like torch.amax
    return np.max(np.abs(g), axis=-1)


def per_token_cast_to_fp8(x: np.ndarray, use_ue8m0: bool = False, gran_k: int = 128):
    """deep_gemm_sm120/utils/math.py:25-37 (K a multiple of gran_k).

    amax = max|x| clamped >= 1e-4; sf = amax / 448 (IEEE); optionally
    ceil_to_ue8m0; q = e4m3(x * (1/sf)) with no clamp.  Returns (q uint8, sf f32).
    """
    g = _groups(x, gran_k)
    amax = np.maximum(_amax(g), np.float32(1e-4))
    amax = np.where(np.isnan(_amax(g)), np.float32(np.nan), amax).astype(np.float32)
    sf = (amax / FP8_MAX).astype(np.float32)
    if use_ue8m0:
        sf = ceil_to_ue8m0(sf)
    inv = (np.float32(1.0) / sf).astype(np.float32)
    q = f32_to_e4m3((g * inv[..., None]).astype(np.float32))
    return q.reshape(np.asarray(x).shape), sf


def act_quant_tilelang(x: np.ndarray, block_size: int = 128, round_scale: bool = False):
    """deepseek_infer/kernel.py:79-83,93-96 (act_quant_kernel, inplace=False).

    amax clamped >= 1e-4; s = amax * fp32(1/448), or fast_round_scale of it;
    q = e4m3(clamp(x / s, -448, 448)).  Returns (q uint8, s f32).
    TileLang's own code generation is not available here: the restated
    formula uses IEEE division (parity with TileLang's exact bits unpinned).
    """
    g = _groups(x, block_size)
    am = _amax(g)
    amax = np.where(np.isnan(am), np.float32(np.nan), np.maximum(am, np.float32(1e-4)))
    amax = amax.astype(np.float32)
    raw = (amax * INV448).astype(np.float32)
    s = pow2_ceil_log2_bits(raw) if round_scale else raw
    y = np.clip((g / s[..., None]).astype(np.float32), -FP8_MAX, FP8_MAX)
    q = f32_to_e4m3(y)
    return q.reshape(np.asarray(x).shape), s


def act_quant_inplace_tilelang(x: np.ndarray, block_size: int = 128, round_scale: bool = False):
    """deepseek_infer/kernel.py:84-91: bf16(fp32(e4m3(clamp(x/s))) * s)."""
    q, s = act_quant_tilelang(x, block_size, round_scale)
    g = e4m3_to_f32(q).reshape(*q.shape[:-1], q.shape[-1] // block_size, block_size)
    y = (g * s[..., None]).astype(np.float32)
    return bf16_round(y).reshape(q.shape), s


def kv_ue8m0_quant(x: np.ndarray, block_size: int = 64):
    """engine/dsv4_kv_pack.py:78-101 _torch_fp8_ue8m0_quant.

    amax clamped >= 1e-12; raw = amax * fp32(1/448);
    scale = 2^ceil(log2(max(raw, 2^-30))) with log2 the correctly rounded fp32
    log2 (what torch.log2 returns on the CPU); y = e4m3(clamp(x/scale, +-448)).
    Returns (q uint8, scale f32 powers of two).
    """
    g = _groups(x, block_size)
    am = _amax(g)
    amax = np.where(np.isnan(am), np.float32(np.nan), np.maximum(am, np.float32(1e-12)))
    raw = (amax.astype(np.float32) * INV448).astype(np.float32)
    raw = np.maximum(raw, np.float32(2.0**-30))
    with np.errstate(invalid="ignore", over="ignore"):
        l2 = np.log2(raw.astype(np.float64)).astype(np.float32)
        scale = np.exp2(np.ceil(l2)).astype(np.float32)
    y = np.clip((g / scale[..., None]).astype(np.float32), -FP8_MAX, FP8_MAX)
    q = f32_to_e4m3(y)
    return q.reshape(np.asarray(x).shape), scale


def scale_mode_quant(x: np.ndarray, mode: int, group: int):
    """Dispatch over the kernels' scale modes (sgl_scale_mode)."""
    if mode == 0:
        return per_token_cast_to_fp8(x, False, group)
    if mode == 1:
        return per_token_cast_to_fp8(x, True, group)
    if mode == 2:
        return act_quant_tilelang(x, group, False)
    if mode == 3:
        return act_quant_tilelang(x, group, True)
    if mode == 4:
        return kv_ue8m0_quant(x, group)
    raise ValueError(f"bad scale mode {mode}")


def per_block_cast_to_fp8(w: np.ndarray, use_ue8m0: bool = False, gran: int = 128):
    """deep_gemm_sm120/utils/math.py:50-60: 128x128 block quant of [N, K],
    zero padding at ragged edges.  Returns (q uint8 [N, K], sf f32 [ceil(N/128), ceil(K/128)])."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    pn, pk = -(-n // gran) * gran, -(-k // gran) * gran
    pad = np.zeros((pn, pk), dtype=np.float32)
    pad[:n, :k] = w
    v = pad.reshape(pn // gran, gran, pk // gran, gran)
    amax = np.maximum(np.abs(v).max(axis=(1, 3)), np.float32(1e-4)).astype(np.float32)
    sf = (amax / FP8_MAX).astype(np.float32)
    if use_ue8m0:
        sf = ceil_to_ue8m0(sf)
    inv = (np.float32(1.0) / sf).astype(np.float32)
    q = f32_to_e4m3((v * inv[:, None, :, None]).astype(np.float32))
    return q.reshape(pn, pk)[:n, :k].copy(), sf


def dequant_rows(q: np.ndarray, s: np.ndarray, group: int = 128) -> np.ndarray:
    """fp32 value of 1 x group quantized rows: e4m3 * scale."""
    v = e4m3_to_f32(q).astype(np.float32)
    g = v.reshape(*v.shape[:-1], v.shape[-1] // group, group)
    return (g * np.asarray(s, dtype=np.float32)[..., None]).reshape(v.shape)


def dequant_blocks(q: np.ndarray, s: np.ndarray, gran: int = 128) -> np.ndarray:
    """fp32 value of a 128x128 block-quantized weight (sglang deepseek_v4.py
    _dequant_fp8 semantics: w * s[n // 128, k // 128])."""
    v = e4m3_to_f32(q).astype(np.float32)
    n, k = v.shape
    s = np.asarray(s, dtype=np.float32)
    if n % gran == 0 and k % gran == 0:
        blk = v.reshape(n // gran, gran, k // gran, gran) * s[:n // gran, None, :k // gran, None]
        return blk.reshape(n, k)
    rs = np.repeat(np.repeat(s, gran, 0), gran, 1)[:n, :k]
    return v * rs
