"""Drop-in leaf ops of the official DeepSeek-V4 ``kernel`` module, on gfx950.

Same names, arguments, return values and assertions as
``engine/vendor/deepseek_infer/kernel.py`` (``act_quant`` :105-125,
``fp8_gemm`` :257-273), plus the DeepGEMM quant helpers
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
    if _scale_flag(a_s, "fp8_gemm a_s"):
        a_s = e8m0_to_f32(a_s)  # the kernel streams fp32 activation scales
    _lib.call(
        "sgl_fp8_gemm",
        a.data_ptr(), a_s.data_ptr(), b.data_ptr(), b_s.data_ptr(),
        _scale_flag(b_s, "fp8_gemm b_s"),
        out.data_ptr(), _lib.SGL_BF16 if odt == torch.bfloat16 else _lib.SGL_F32,
        M, N, K, _lib.stream_of(a),
    )
    return out


__all__ = [
    "act_quant",
    "act_quant_formula",
    "e8m0_to_f32",
    "fp8_gemm",
    "per_block_cast_to_fp8",
    "per_token_cast_to_fp8",
    "scale_mode_for",
]
