"""Drop-in leaf ops of the official DeepSeek-V4 ``kernel`` module, on gfx950.

Same names, arguments, return values and assertions as
``engine/vendor/deepseek_infer/kernel.py`` (``act_quant`` :105-125,
``fp8_gemm`` :257-273, ``fp4_gemm`` :519-536), the FP4 -> FP8 weight repack of
``deepseek_infer/convert.py:17-52``, plus the DeepGEMM quant helpers
(``deep_gemm_sm120/utils/math.py:25-37,50-60``) the synthetic weights use.
Every op runs a hand-written HIP kernel from ``libsglang_lite_amd.so``; CPU
tensors are refused.

Scale formula.  The official TileLang ``act_quant`` computes
``s = amax * (1/448)`` and ``clamp(x / s)``; DeepGEMM's torch
``per_token_cast_to_fp8`` computes ``sf = amax / 448`` and ``x * (1/sf)``.
They can differ by one ulp in the scale and one e4m3 code.  ``act_quant``
uses the torch formula by default (the bit-exact target); set
``SGLANG_LITE_AMD_ACT_QUANT=tilelang`` for the TileLang formula.
"""

from __future__ import annotations

import os
from typing import Optional, Tuple

import torch

from . import _lib

FP8 = torch.float8_e4m3fn
E8M0 = torch.float8_e8m0fnu
FP4 = torch.float4_e2m1fn_x2  # two e2m1 codes per byte, low nibble = even K

# Attribute set on functions that compute exactly this module's ``act_quant``
# (``act_quant`` itself and wrappers of it): a quantizer injected into the KV
# pack that carries it is computed by the fused pack kernel instead of called.
FUSED_ACT_QUANT = "_sglang_lite_amd_act_quant"


def act_quant_formula() -> str:
    raw = os.environ.get("SGLANG_LITE_AMD_ACT_QUANT", "torch").strip().lower()
    if raw not in ("torch", "tilelang"):
        raise ValueError(f"SGLANG_LITE_AMD_ACT_QUANT must be 'torch' or 'tilelang', got {raw!r}")
    return raw


def scale_mode_for(scale_fmt: Optional[str], formula: Optional[str] = None) -> int:
    """sgl_scale_mode for an ``act_quant`` call (scale_fmt None -> fp32 scales)."""
    formula = formula or act_quant_formula()
    if formula == "torch":
        return _lib.SCALE_TORCH_FP32 if scale_fmt is None else _lib.SCALE_TORCH_UE8M0
    return _lib.SCALE_TILELANG_FP32 if scale_fmt is None else _lib.SCALE_TILELANG_UE8M0


def act_quant(
    x: torch.Tensor,
    block_size: int = 128,
    scale_fmt: Optional[str] = None,
    scale_dtype: torch.dtype = torch.float32,
    inplace: bool = False,
    *,
    scale_mode: Optional[int] = None,
):
    """Block-wise FP8 quantization (deepseek_infer/kernel.py:105-125).

    Returns ``(y_e4m3, s)`` with ``s`` of shape ``[*x.shape[:-1], N // block_size]``
    in ``scale_dtype``; ``inplace=True`` writes the quant-dequant back into ``x``
    and returns ``x``.  ``scale_mode`` overrides the formula (sgl_scale_mode).
    """
    N = x.size(-1)
    assert N % block_size == 0
    _lib.require_device(x, what="act_quant")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"act_quant: expected bfloat16 input, got {x.dtype}")
    if scale_dtype not in (torch.float32, E8M0):
        raise TypeError(f"act_quant: scale_dtype must be float32 or float8_e8m0fnu, got {scale_dtype}")
    mode = scale_mode_for(scale_fmt) if scale_mode is None else int(scale_mode)
    z = x.contiguous()
    y = torch.empty_like(z) if inplace else torch.empty_like(z, dtype=FP8)
    s = z.new_empty(*z.size()[:-1], N // block_size, dtype=scale_dtype)
    M = z.numel() // N if N else 0
    _lib.call(
        "sgl_act_quant",
        z.data_ptr(), M, N, N, y.data_ptr(), N, s.data_ptr(), N // block_size,
        block_size, mode, int(scale_dtype == E8M0), int(inplace), _lib.stream_of(z),
    )
    if inplace:
        x.copy_(y)
        return x
    return y, s


setattr(act_quant, FUSED_ACT_QUANT, True)


def per_token_cast_to_fp8(x: torch.Tensor, use_ue8m0: bool, gran_k: int = 128):
    """DeepGEMM ``per_token_cast_to_fp8`` (utils/math.py:25-37) for K % gran_k == 0."""
    assert x.dim() == 2
    mode = _lib.SCALE_TORCH_UE8M0 if use_ue8m0 else _lib.SCALE_TORCH_FP32
    return act_quant(x, gran_k, None, torch.float32, False, scale_mode=mode)


def per_block_cast_to_fp8(x: torch.Tensor, use_ue8m0: bool, gran_k: int = 128):
    """DeepGEMM ``per_block_cast_to_fp8`` (utils/math.py:50-60): 128x128 block
    scales of a 2-D fp32 / bf16 weight; returns (e4m3 [N, K], f32 [ceil(N/128), ceil(K/128)])."""
    assert x.dim() == 2 and gran_k == 128
    _lib.require_device(x, what="per_block_cast_to_fp8")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"per_block_cast_to_fp8: expected float32/bfloat16, got {x.dtype}")
    w = x.contiguous()
    n, k = w.shape
    q = torch.empty(n, k, dtype=FP8, device=w.device)
    s = torch.empty((n + 127) // 128, (k + 127) // 128, dtype=torch.float32, device=w.device)
    dt = _lib.SGL_F32 if w.dtype == torch.float32 else _lib.SGL_BF16
    _lib.call(
        "sgl_weight_quant_128x128",
        w.data_ptr(), dt, n, k, k, q.data_ptr(), k, s.data_ptr(), s.size(1), int(use_ue8m0),
        _lib.stream_of(w),
    )
    return q, s


def e8m0_to_f32(s: torch.Tensor) -> torch.Tensor:
    """float8_e8m0fnu -> float32 powers of two on the device."""
    _lib.require_device(s, what="e8m0_to_f32")
    src = s.contiguous()
    out = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    _lib.call("sgl_e8m0_to_f32", src.data_ptr(), out.data_ptr(), src.numel(), _lib.stream_of(src))
    return out


def fp8_weight_to_frag(w: torch.Tensor) -> torch.Tensor:
    """e4m3 weight [N, K] -> a new [N * K] uint8 tensor in the MFMA fragment
    layout of ``sgl_fp8_weight_to_frag`` (2 KB per 16-row x 128-deep block,
    lane-major), the layout ``EXPERT_FRAG_COPY`` expert records point at.
    A layout step of this build with no counterpart in the reference."""
    _lib.require_device(w, what="fp8_weight_to_frag")
    if w.dtype != FP8 or w.dim() != 2:
        raise TypeError("fp8_weight_to_frag: w must be a 2-D float8_e4m3fn tensor")
    src = w.contiguous()
    N, K = src.shape
    out = torch.empty(N * K, dtype=torch.uint8, device=src.device)
    _lib.call("sgl_fp8_weight_to_frag", src.data_ptr(), N, K, out.data_ptr(), _lib.stream_of(src))
    return out


def fp4_weight_to_frag(b: torch.Tensor, s: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Packed e2m1 weight [N, K/2] with e8m0 scales [N, K/32] -> new uint8
    tensors (weights [N * K/2], scales [N * K/32]) in the FP4 fragment layout
    of ``sgl_fp4_weight_to_frag`` (the layout ``EXPERT_FRAG_COPY`` records of
    FP4 experts point at).  A layout step of this build with no counterpart
    in the reference."""
    wb = fp4_bytes(b).contiguous()
    sc = fp4_weight_scale(s).view(torch.uint8).contiguous()
    _lib.require_device(wb, sc, what="fp4_weight_to_frag")
    N, KH = wb.shape
    K = 2 * KH
    if tuple(sc.shape) != (N, K // 32):
        raise ValueError(f"fp4_weight_to_frag: scales must be [{N}, {K // 32}], got {tuple(sc.shape)}")
    ow = torch.empty(N * KH, dtype=torch.uint8, device=wb.device)
    os_ = torch.empty(N * (K // 32), dtype=torch.uint8, device=wb.device)
    _lib.call("sgl_fp4_weight_to_frag", wb.data_ptr(), sc.data_ptr(), N, K, ow.data_ptr(),
              os_.data_ptr(), _lib.stream_of(wb))
    return ow, os_


def _scale_flag(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.float32:
        return 0
    if t.dtype == E8M0:
        return 1
    raise TypeError(f"{what}: scales must be float32 or float8_e8m0fnu, got {t.dtype}")


def fp8_gemm(
    a: torch.Tensor,
    a_s: torch.Tensor,
    b: torch.Tensor,
    b_s: torch.Tensor,
    scale_dtype: torch.dtype = torch.float32,
    *,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """C[M,N] = A[M,K] @ B[N,K]^T with per-128 block FP8 scaling on both A and B
    (deepseek_infer/kernel.py:257-273).  Output dtype is torch's default dtype
    (bf16 or fp32).  ``scale_dtype`` is accepted for signature parity; the
    scale tensors' own dtypes (fp32 or e8m0) decide how they are read."""
    del scale_dtype
    assert a.is_contiguous() and b.is_contiguous(), "Input tensors must be contiguous"
    assert a_s.is_contiguous() and b_s.is_contiguous(), "Scaling factor tensors must be contiguous"
    _lib.require_device(a, a_s, b, b_s, what="fp8_gemm")
    if a.dtype != FP8 or b.dtype != FP8:
        raise TypeError(f"fp8_gemm: operands must be float8_e4m3fn, got {a.dtype}, {b.dtype}")
    K = a.size(-1)
    M = a.numel() // K
    N = b.size(0)
    odt = torch.get_default_dtype()
    if odt not in (torch.bfloat16, torch.float32):
        raise TypeError(f"fp8_gemm: default dtype must be bfloat16 or float32, got {odt}")
    if out is None:
        out = a.new_empty(*a.size()[:-1], N, dtype=odt)
    else:
        assert out.is_contiguous() and out.dtype == odt and out.numel() == M * N
    # split-K shapes keep their fp32 partials in a workspace allocated here with
    # torch (inside a graph capture it comes from the graph's pool), as the
    # reference's adapter allocates its output (engine/v4_deep_gemm.py:186-188)
    nws = int(_lib.load().sgl_fp8_gemm_workspace_size(M, N, K)) if M else 0
    ws = torch.empty(nws, dtype=torch.uint8, device=a.device) if nws else None
    _lib.call(
        "sgl_fp8_gemm",
        a.data_ptr(), a_s.data_ptr(), _scale_flag(a_s, "fp8_gemm a_s"), b.data_ptr(), b_s.data_ptr(),
        _scale_flag(b_s, "fp8_gemm b_s"),
        out.data_ptr(), _lib.SGL_BF16 if odt == torch.bfloat16 else _lib.SGL_F32,
        M, N, K, _lib.ptr(ws), nws, _lib.stream_of(a),
    )
    return out


def fp4_bytes(b: torch.Tensor) -> torch.Tensor:
    """Packed e2m1 weight [N, K/2] (float4_e2m1fn_x2, or its int8 / uint8 view
    as convert.py stores it) as a uint8 view."""
    if b.dtype not in (FP4, torch.int8, torch.uint8):
        raise TypeError(f"FP4 weight must be float4_e2m1fn_x2 / int8 / uint8, got {b.dtype}")
    return b.view(torch.uint8)


def fp4_weight_scale(s: torch.Tensor) -> torch.Tensor:
    """e8m0 [N, K/32] weight scales (fp32 powers of two are cast to e8m0)."""
    if s.dtype == E8M0:
        return s.contiguous()
    if s.dtype == torch.float32:
        return s.contiguous().to(E8M0)
    raise TypeError(f"FP4 weight scales must be float8_e8m0fnu or float32, got {s.dtype}")


def fp4_gemm(
    a: torch.Tensor,
    a_s: torch.Tensor,
    b: torch.Tensor,
    b_s: torch.Tensor,
    scale_dtype: torch.dtype = torch.float32,
    *,
    out: Optional[torch.Tensor] = None,
    a_scale_pow2: Optional[bool] = None,
) -> torch.Tensor:
    """C[M,N] = A_fp8[M,K] @ B_fp4[N,K]^T (deepseek_infer/kernel.py:519-536).

    A has one scale per 128 K (fp32 or e8m0), B one e8m0 scale per 32 K and is
    stored as [N, K//2] float4_e2m1fn_x2 (2 FP4 values per byte, packed along
    K).  Output dtype is torch's default dtype (bf16 or fp32).  With e8m0
    activation scales (or ``a_scale_pow2=True`` for fp32 powers of two) both
    scales are applied inside the MFMA; otherwise each 128-deep partial is
    promoted with the fp32 activation scale.  K % 256 == 0."""
    del scale_dtype
    assert a.is_contiguous() and b.is_contiguous(), "Input tensors must be contiguous"
    assert a_s.is_contiguous() and b_s.is_contiguous(), "Scaling factor tensors must be contiguous"
    _lib.require_device(a, a_s, b, b_s, what="fp4_gemm")
    if a.dtype != FP8:
        raise TypeError(f"fp4_gemm: activations must be float8_e4m3fn, got {a.dtype}")
    bq = fp4_bytes(b)
    K = a.size(-1)
    M = a.numel() // K
    N = b.size(0)
    if bq.dim() != 2 or bq.size(1) * 2 != K:
        raise ValueError(f"fp4_gemm: weight must be [N, K/2] = [{N}, {K // 2}], got {tuple(b.shape)}")
    odt = torch.get_default_dtype()
    if odt not in (torch.bfloat16, torch.float32):
        raise TypeError(f"fp4_gemm: default dtype must be bfloat16 or float32, got {odt}")
    if out is None:
        out = a.new_empty(*a.size()[:-1], N, dtype=odt)
    else:
        assert out.is_contiguous() and out.dtype == odt and out.numel() == M * N
    if _scale_flag(a_s, "fp4_gemm a_s"):
        fmt = _lib.ASCALE_E8M0  # read as bytes, applied in the MFMA
    else:
        fmt = _lib.ASCALE_F32_POW2 if a_scale_pow2 else _lib.ASCALE_F32
    bs = fp4_weight_scale(b_s)
    _lib.call(
        "sgl_fp4_gemm",
        a.data_ptr(), a_s.data_ptr(), fmt, bq.data_ptr(), bs.data_ptr(),
        out.data_ptr(), _lib.SGL_BF16 if odt == torch.bfloat16 else _lib.SGL_F32,
        M, N, K, _lib.stream_of(a),
    )
    return out


def cast_e2m1fn_to_e4m3fn(x: torch.Tensor, scale: torch.Tensor):
    """Lossless FP4 -> FP8 weight repack (deepseek_infer/convert.py:17-52):
    packed e2m1 [out, in/2] (int8 / uint8 / float4_e2m1fn_x2) with e8m0 scales
    [out, in/32] -> (e4m3 [out, in], e8m0 [out/128, in/128])."""
    xb = fp4_bytes(x)
    assert xb.ndim == 2
    out_dim, in_dim = xb.size()
    in_dim *= 2
    assert in_dim % 128 == 0 and out_dim % 128 == 0
    assert scale.size(0) == out_dim and scale.size(1) == in_dim // 32
    _lib.require_device(xb, scale, what="cast_e2m1fn_to_e4m3fn")
    sb = fp4_weight_scale(scale)
    q = torch.empty(out_dim, in_dim, dtype=FP8, device=xb.device)
    s = torch.empty(out_dim // 128, in_dim // 128, dtype=E8M0, device=xb.device)
    _lib.call("sgl_fp4_to_fp8_weight", xb.contiguous().data_ptr(), sb.data_ptr(), out_dim, in_dim,
              q.data_ptr(), s.data_ptr(), _lib.stream_of(xb))
    return q, s


__all__ = [
    "act_quant",
    "act_quant_formula",
    "cast_e2m1fn_to_e4m3fn",
    "e8m0_to_f32",
    "fp4_gemm",
    "fp8_gemm",
    "per_block_cast_to_fp8",
    "per_token_cast_to_fp8",
    "scale_mode_for",
]
