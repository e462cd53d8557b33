"""FP8 block-scaled GEMM call-site adapter for the official DeepSeek-V4 graph on gfx950.

Drop-in counterpart of ``engine/v4_deep_gemm.py`` (probe :97-133, scale cache
:136-166, ``fp4_gemm_nt`` adapter :169-218, drop-in :221-230, prewarm :267-281,
attach :284-347, ``is_armed`` :350-351).  The reference's live branch is
DeepGEMM's FP8 x MXFP4; this build serves the FP8 x FP8 128x128 branch
(``kernel.fp8_gemm``, model.py:116-118): ``attach_v4_deep_gemm`` patches
``kernel.act_quant`` / ``kernel.fp8_gemm`` (and the names ``model.py``
imported from ``kernel`` at load, so ``linear()`` picks them up) with the HIP
kernels, after a probe on the device.

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


def fp4_gemm_nt(*args, **kwargs):
    """FP8 x MXFP4 (the reference's live DeepGEMM branch) is not built on gfx950 yet."""
    raise NotImplementedError("sglang_lite_amd: FP8 x MXFP4 GEMM is not implemented")


def _fp8_gemm_dropin(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
                     scale_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Drop-in for the official ``kernel.fp8_gemm`` (kernel.py:257-273)."""
    del scale_dtype
    return fp8_gemm_nt(a, a_s, b, b_s)


def _act_quant_dropin(x: torch.Tensor, block_size: int = 128, scale_fmt: Optional[str] = None,
                      scale_dtype: torch.dtype = torch.float32, inplace: bool = False):
    """Drop-in for the official ``kernel.act_quant`` (kernel.py:105-125)."""
    return HK.act_quant(x, block_size, scale_fmt, scale_dtype, inplace)


def prewarm_model_scales(model: Any) -> int:
    """Materialize the fp32 scale cache of every FP8 weight (v4_deep_gemm.py:267-281)."""
    n = 0
    for mod in model.modules():
        w = getattr(mod, "weight", None)
        if w is None or not hasattr(w, "scale") or w.dtype != torch.float8_e4m3fn:
            continue
        try:
            ensure_weight_cache(w)
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
        M = sys.modules.get("model")
        if M is not None:
            if getattr(M, "fp8_gemm", None) is not None and not getattr(M.fp8_gemm, MARK, False):
                M.fp8_gemm = K.fp8_gemm
            if getattr(M, "act_quant", None) is not None and not getattr(M.act_quant, MARK, False):
                M.act_quant = K.act_quant
        _PATCHED = True
        stats["patched"] = True
    if model is not None:
        stats["scale_cache"] = prewarm_model_scales(model)
    stats["enabled"] = True
    stats["backend"] = "gfx950_hip"
    print(f"[sglang-lite-amd] FP8 GEMM armed (e4m3 a1x128 / b128x128, gfx950 MFMA); "
          f"scale_cache={stats['scale_cache']}")
    return stats


def detach_v4_deep_gemm() -> None:
    """Restore the official kernels (for tests and A/B runs)."""
    global _PATCHED
    K = sys.modules.get("kernel")
    if K is not None and getattr(K, "_fp8_gemm_tilelang", None) is not None:
        K.fp8_gemm = K._fp8_gemm_tilelang
        K.act_quant = K._act_quant_tilelang
        M = sys.modules.get("model")
        if M is not None:
            if getattr(M.fp8_gemm, MARK, False):
                M.fp8_gemm = K.fp8_gemm
            if getattr(M.act_quant, MARK, False):
                M.act_quant = K.act_quant
    _PATCHED = False


def is_armed() -> bool:
    return bool(_PATCHED and _PROBE_OK)


__all__ = ["attach_v4_deep_gemm", "deep_gemm_enabled", "detach_v4_deep_gemm", "ensure_weight_cache",
           "fp4_gemm_nt", "fp8_gemm_nt", "is_armed", "prewarm_model_scales", "probe_fp8_gemm",
           "scale_to_f32"]
