"""FP8 / FP4 block-scaled GEMM call-site adapter for the official DeepSeek-V4 graph on gfx950.

Drop-in counterpart of ``engine/v4_deep_gemm.py`` (probe :97-133, scale cache
:136-166, ``fp4_gemm_nt`` adapter :169-218, drop-in :221-230, prewarm :267-281,
attach :284-347, ``is_armed`` :350-351).  Both weight branches of the official
``linear()`` (model.py:108-120) run on the HIP kernels: FP8 x MXFP4
(``kernel.fp4_gemm``, the reference's live DeepGEMM branch) and FP8 x FP8
128x128 (``kernel.fp8_gemm``).  ``attach_v4_deep_gemm`` patches
``kernel.act_quant`` / ``kernel.fp8_gemm`` / ``kernel.fp4_gemm`` (and the names
``model.py`` imported from ``kernel`` at load, so ``linear()`` picks them up)
after a probe on the device.

Env: ``SGLANG_LITE_V4_DEEP_GEMM=0`` keeps the official kernels (same switch
as the reference).
"""

from __future__ import annotations

import logging
import os
import sys
from typing import Any, Optional, Tuple

import torch

from . import _lib
from . import kernel as HK

logger = logging.getLogger("sglang_lite_amd.v4_deep_gemm")

_PATCHED = False
_PROBE_OK: Optional[bool] = None
MARK = "_sglang_lite_amd"


def deep_gemm_enabled() -> bool:
    raw = os.environ.get("SGLANG_LITE_V4_DEEP_GEMM", "1").strip().lower()
    return raw not in ("0", "false", "no", "off")


def probe_fp8_gemm(device: str = "cuda") -> dict:
    """Tiny FP8 x FP8 GEMM on the device against its dequantized product.
    Returns ``{"ok", "error", "version", "source"}`` (v4_deep_gemm.py:97-133)."""
    global _PROBE_OK
    import sglang_lite_amd

    out: dict = {"ok": False, "error": None, "version": sglang_lite_amd.__version__,
                 "source": sglang_lite_amd.library_path()}
    if device == "cpu" or not torch.cuda.is_available():
        out["error"] = "no_gpu"
        _PROBE_OK = False
        return out
    info = sglang_lite_amd.probe()
    if not info["ok"]:
        out["error"] = info["error"]
        _PROBE_OK = False
        return out
    try:
        m, n, k = 16, 64, 128
        g = torch.Generator(device=device).manual_seed(0)
        a = torch.randn(m, k, device=device, generator=g).to(torch.bfloat16)
        aq, a_s = HK.act_quant(a)
        b = torch.randn(n, k, device=device, generator=g) * 0.05
        bq, b_s = HK.per_block_cast_to_fp8(b, False)
        c = HK.fp8_gemm(aq, a_s, bq, b_s)
        torch.cuda.synchronize()
        ref = (aq.float() * a_s.repeat_interleave(128, 1)) @ (bq.float() * b_s.repeat_interleave(
            128, 0)[:n].repeat_interleave(128, 1)).T
        err = float((c.float() - ref).norm() / ref.norm().clamp_min(1e-30))
        if not err < 1e-2:
            raise RuntimeError(f"probe GEMM rel error {err:.3e}")
        # FP8 x FP4 on the same activations: e2m1 codes 0..15 cycling, unit scales
        k4 = 256
        a4 = torch.randn(m, k4, device=device, generator=g).to(torch.bfloat16)
        aq4, a4_s = HK.act_quant(a4)
        codes = (torch.arange(n * k4, device=device) % 16).to(torch.uint8).view(n, k4)
        b4 = (codes[:, 0::2] | (codes[:, 1::2] << 4)).contiguous()
        b4_s = torch.full((n, k4 // 32), 127, dtype=torch.uint8, device=device).view(HK.E8M0)
        c4 = HK.fp4_gemm(aq4, a4_s, b4, b4_s)
        torch.cuda.synchronize()
        e2m1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                             -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], device=device)
        ref4 = (aq4.float() * a4_s.repeat_interleave(128, 1)) @ e2m1[codes.long()].T
        err4 = float((c4.float() - ref4).norm() / ref4.norm().clamp_min(1e-30))
        if not err4 < 1e-2:
            raise RuntimeError(f"probe FP4 GEMM rel error {err4:.3e}")
        out["ok"] = True
    except Exception as e:  # noqa: BLE001 - the probe reports, never raises
        out["error"] = f"{type(e).__name__}: {e}"
    _PROBE_OK = out["ok"]
    return out


# the reference's name for its probe, kept for call sites that import it
probe_deep_gemm_sm120 = probe_fp8_gemm


def scale_to_f32(scale: torch.Tensor) -> torch.Tensor:
    """e8m0 / fp32 scales -> fp32 (v4_deep_gemm.py:136-141), on the device."""
    if scale.dtype == torch.float32:
        return scale
    if scale.dtype == torch.float8_e8m0fnu and scale.is_cuda:
        return HK.e8m0_to_f32(scale)
    raise TypeError(f"scale_to_f32: unsupported {scale.dtype} on {scale.device}")


def ensure_weight_cache(weight: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Cache the fp32 scale of an FP8 weight Parameter once (``_dg_s_f32``,
    v4_deep_gemm.py:151-166).  Returns ``(weight, scale_f32)``."""
    s_f = getattr(weight, "_dg_s_f32", None)
    if s_f is None:
        scale = getattr(weight, "scale", None)
        if scale is None:
            raise RuntimeError("FP8 weight missing .scale")
        s_f = scale_to_f32(scale.data).contiguous()
        try:
            weight._dg_s_f32 = s_f  # type: ignore[attr-defined]
        except Exception:  # noqa: BLE001
            pass
    return weight, s_f


ensure_weight_dg_cache = ensure_weight_cache


def is_fp4_weight(weight: torch.Tensor) -> bool:
    """FP4 packed weight: float4_e2m1fn_x2, or int8 / uint8 whose ``.scale``
    has one column per 32 inputs (the reference's heuristic, v4_deep_gemm.py:239-245)."""
    if weight.dtype == HK.FP4:
        return True
    sc = getattr(weight, "scale", None)
    return (weight.dtype in (torch.int8, torch.uint8) and sc is not None and sc.dim() == 2
            and sc.shape[-1] == (weight.shape[-1] * 2) // 32)


def ensure_fp4_weight_cache(weight: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Cache the uint8 view and the e8m0 scales of an FP4 weight Parameter once
    (``_dg_w_i8`` / ``_dg_s_f32`` of v4_deep_gemm.py:151-166; the kernel reads
    e8m0 bytes, so fp32 scales are cast once here)."""
    w_u8 = getattr(weight, "_sgl_w_u8", None)
    s_e8 = getattr(weight, "_sgl_s_e8m0", None)
    if w_u8 is None or s_e8 is None:
        scale = getattr(weight, "scale", None)
        if scale is None:
            raise RuntimeError("FP4 weight missing .scale")
        w_u8 = HK.fp4_bytes(weight.data).contiguous()
        s_e8 = HK.fp4_weight_scale(scale.data)
        try:
            weight._sgl_w_u8 = w_u8  # type: ignore[attr-defined]
            weight._sgl_s_e8m0 = s_e8  # type: ignore[attr-defined]
        except Exception:  # noqa: BLE001
            pass
    return w_u8, s_e8


def fp8_gemm_nt(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor, *,
                out: Optional[torch.Tensor] = None,
                out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """C[..., N] = A_fp8[..., K] @ B_fp8[N, K]^T with 1x128 / 128x128 scales: the
    call-site contract of ``fp4_gemm_nt`` (v4_deep_gemm.py:169-218) for FP8 weights."""
    K = a.size(-1)
    M = a.numel() // K
    N = b.size(0)
    odt = out_dtype or torch.get_default_dtype()
    a2 = a.reshape(M, K)
    if not a2.is_contiguous():
        a2 = a2.contiguous()
    as2 = a_s.reshape(M, -1)
    if not as2.is_contiguous():
        as2 = as2.contiguous()
    if getattr(b, "_dg_s_f32", None) is not None:
        bs = b._dg_s_f32  # type: ignore[attr-defined]
    elif getattr(b, "scale", None) is not None and b_s is b.scale:
        _, bs = ensure_weight_cache(b)
    else:
        bs = b_s.contiguous()
    bb = b if b.is_contiguous() else b.contiguous()
    res = out if out is not None and out.dtype == odt and out.is_contiguous() else None
    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(odt)
        c = HK.fp8_gemm(a2, as2, bb, bs, out=res.view(M, N) if res is not None else None)
    finally:
        torch.set_default_dtype(prev)
    c = c.view(*a.shape[:-1], N)
    if out is not None and res is None:
        out.copy_(c)
        return out
    return c


def fp4_gemm_nt(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor, *,
                out: Optional[torch.Tensor] = None,
                out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """C[..., N] = A_fp8[..., K] @ B_fp4[N, K]^T (v4_deep_gemm.py:169-218, same
    contract as ``kernel.fp4_gemm``): 1x128 activation scales (fp32 or e8m0),
    packed e2m1 weight [N, K/2] with e8m0 1x32 scales.  e8m0 activation scales
    (the live ``scale_dtype``) are applied inside the MFMA with the weight's."""
    _lib.require_device(a, a_s, b, b_s, what="fp4_gemm_nt")
    K = a.size(-1)
    M = a.numel() // K
    N = b.size(0)
    odt = out_dtype or torch.get_default_dtype()
    a2 = a.reshape(M, K)
    if not a2.is_contiguous():
        a2 = a2.contiguous()
    as2 = a_s.reshape(M, -1)
    if not as2.is_contiguous():
        as2 = as2.contiguous()
    if getattr(b, "_sgl_w_u8", None) is not None and getattr(b, "_sgl_s_e8m0", None) is not None:
        bi, bs = b._sgl_w_u8, b._sgl_s_e8m0  # type: ignore[attr-defined]
    elif getattr(b, "scale", None) is not None and b_s is b.scale:
        bi, bs = ensure_fp4_weight_cache(b)
    else:
        bi = HK.fp4_bytes(b if b.is_contiguous() else b.contiguous())
        bs = HK.fp4_weight_scale(b_s)
    res = out if out is not None and out.dtype == odt and out.is_contiguous() else None
    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(odt)
        c = HK.fp4_gemm(a2, as2, bi, bs, out=res.view(M, N) if res is not None else None)
    finally:
        torch.set_default_dtype(prev)
    c = c.view(*a.shape[:-1], N)
    if out is not None and res is None:
        out.copy_(c)
        return out
    return c


def _fp4_gemm_dropin(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
                     scale_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Drop-in for the official ``kernel.fp4_gemm`` (kernel.py:519-536;
    v4_deep_gemm.py:221-230)."""
    del scale_dtype
    return fp4_gemm_nt(a, a_s, b, b_s)


def _fp8_gemm_dropin(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
                     scale_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Drop-in for the official ``kernel.fp8_gemm`` (kernel.py:257-273)."""
    del scale_dtype
    return fp8_gemm_nt(a, a_s, b, b_s)


def _act_quant_dropin(x: torch.Tensor, block_size: int = 128, scale_fmt: Optional[str] = None,
                      scale_dtype: torch.dtype = torch.float32, inplace: bool = False):
    """Drop-in for the official ``kernel.act_quant`` (kernel.py:105-125)."""
    return HK.act_quant(x, block_size, scale_fmt, scale_dtype, inplace)


# the KV pack (dsv4_kv_pack.py:58-61 injects kernel.act_quant, which after the
# attach is this function) computes this function's formula in its fused kernel
setattr(_act_quant_dropin, HK.FUSED_ACT_QUANT, True)


def prewarm_model_scales(model: Any) -> int:
    """Materialize the scale cache of every FP8 (fp32 scales) and FP4 (uint8
    view + e8m0 scales) weight (v4_deep_gemm.py:267-281)."""
    n = 0
    for mod in model.modules():
        w = getattr(mod, "weight", None)
        if w is None or not hasattr(w, "scale"):
            continue
        try:
            if w.dtype == torch.float8_e4m3fn:
                ensure_weight_cache(w)
            elif is_fp4_weight(w):
                ensure_fp4_weight_cache(w)
            else:
                continue
            n += 1
        except Exception:  # noqa: BLE001
            pass
    return n


def _mark(fn):
    setattr(fn, MARK, True)
    return fn


def attach_v4_deep_gemm(model: Optional[Any] = None) -> dict:
    """Patch the official ``kernel.act_quant`` / ``kernel.fp8_gemm`` (and the
    copies ``model`` imported) with the gfx950 kernels.  Safe no-op when
    disabled, when the probe fails, or when already patched; never raises."""
    global _PATCHED
    stats: dict = {"enabled": False, "patched": False, "probe": None, "scale_cache": 0,
                   "backend": "tilelang"}
    if not deep_gemm_enabled():
        stats["backend"] = "disabled"
        return stats
    probe = probe_fp8_gemm()
    stats["probe"] = probe
    if not probe.get("ok"):
        logger.warning("gfx950 FP8 GEMM probe failed: %s", probe.get("error"))
        print(f"[sglang-lite-amd] FP8 GEMM skipped (probe failed: {probe.get('error')})")
        return stats
    if not _PATCHED:
        K = sys.modules.get("kernel")
        if K is None:
            stats["error"] = "kernel_not_importable: official kernel module not loaded"
            print("[sglang-lite-amd] FP8 GEMM probe OK but kernel not on path yet; "
                  "call attach after the official graph import")
            return stats
        if not getattr(K.fp8_gemm, MARK, False):
            K._fp8_gemm_tilelang = K.fp8_gemm
            K._act_quant_tilelang = K.act_quant
            K.fp8_gemm = _mark(_fp8_gemm_dropin)
            K.act_quant = _mark(_act_quant_dropin)
        if getattr(K, "fp4_gemm", None) is not None and not getattr(K.fp4_gemm, MARK, False):
            K._fp4_gemm_tilelang = K.fp4_gemm
            K.fp4_gemm = _mark(_fp4_gemm_dropin)
        M = sys.modules.get("model")
        if M is not None:
            for name in ("fp8_gemm", "fp4_gemm", "act_quant"):
                f = getattr(M, name, None)
                if f is not None and not getattr(f, MARK, False):
                    setattr(M, name, getattr(K, name))
        _PATCHED = True
        stats["patched"] = True
    if model is not None:
        stats["scale_cache"] = prewarm_model_scales(model)
    stats["enabled"] = True
    stats["backend"] = "gfx950_hip"
    print(f"[sglang-lite-amd] FP8/FP4 GEMM armed (a1x128 / b128x128 e4m3, b1x32 e2m1; gfx950 "
          f"MFMA); scale_cache={stats['scale_cache']}")
    return stats


def detach_v4_deep_gemm() -> None:
    """Restore the official kernels (for tests and A/B runs)."""
    global _PATCHED
    K = sys.modules.get("kernel")
    if K is not None and getattr(K, "_fp8_gemm_tilelang", None) is not None:
        K.fp8_gemm = K._fp8_gemm_tilelang
        K.act_quant = K._act_quant_tilelang
        if getattr(K, "_fp4_gemm_tilelang", None) is not None:
            K.fp4_gemm = K._fp4_gemm_tilelang
        M = sys.modules.get("model")
        if M is not None:
            for name in ("fp8_gemm", "fp4_gemm", "act_quant"):
                f = getattr(M, name, None)
                if f is not None and getattr(f, MARK, False):
                    setattr(M, name, getattr(K, name))
    _PATCHED = False


def is_armed() -> bool:
    return bool(_PATCHED and _PROBE_OK)


__all__ = ["attach_v4_deep_gemm", "deep_gemm_enabled", "detach_v4_deep_gemm",
           "ensure_fp4_weight_cache", "ensure_weight_cache", "fp4_gemm_nt", "fp8_gemm_nt",
           "is_armed", "is_fp4_weight", "prewarm_model_scales", "probe_fp8_gemm", "scale_to_f32"]
