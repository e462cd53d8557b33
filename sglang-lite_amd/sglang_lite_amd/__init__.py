"""MI355X (gfx950) FP8 MoE expert path and FP8 KV pack of DeepSeek-V4-Flash.

A drop-in for the reference's (ParaTensor/sglang-lite) hot path:

* ``kernel``        -- ``act_quant`` / ``fp8_gemm`` of the official ``kernel`` module
* ``moe``           -- routing, permutation, grouped gate/up + down GEMMs, combine
* ``v4_moe_fast``   -- ``MoE.forward`` / ``Expert.forward`` replacements + attach
* ``v4_deep_gemm``  -- FP8 GEMM call-site adapter: probe, attach, scale caches
* ``dsv4_kv_pack``  -- FP8 KV row pack / paging / gather-dequant / index split

All compute runs in hand-written HIP kernels of ``lib/libsglang_lite_amd.so``
(C ABI: ``include/sglang_lite_amd.h``); torch only provides device memory and
the current stream.  There is no CPU fallback.
"""

from . import _lib  # noqa: F401

__version__ = "0.1.0"


def library_path() -> str:
    return str(_lib.LIB_PATH)


def probe() -> dict:
    """{"ok", "error", "version", "source"} like the reference's probe_deep_gemm_sm120."""
    out = {"ok": False, "error": None, "version": __version__, "source": library_path()}
    try:
        lib = _lib.load()
    except Exception as e:  # missing / stale library
        out["error"] = f"{type(e).__name__}: {e}"
        return out
    import torch

    if not torch.cuda.is_available():
        out["error"] = "no_gpu"
        return out
    if lib.sgl_probe() != 1:
        out["error"] = _lib.last_error()
        return out
    out["ok"] = True
    return out
