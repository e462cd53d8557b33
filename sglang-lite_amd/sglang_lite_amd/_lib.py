"""ctypes binding of ``libsglang_lite_amd.so`` (the C ABI in include/sglang_lite_amd.h).

The library is built in-tree (``__graft_entry__.build()`` or
``make -C sglang-lite_amd/csrc``).  There is no fallback: when the library is
missing or a call fails, the caller gets an exception.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path
from typing import Optional

LIB_DIR = Path(__file__).resolve().parent / "lib"
# SGLANG_LITE_AMD_LIB names another build of the same library (an A/B build
# of a kernel variant); by default the in-tree build is loaded
LIB_PATH = Path(os.environ.get("SGLANG_LITE_AMD_LIB") or (LIB_DIR / "libsglang_lite_amd.so"))

ABI_VERSION = 3

SGL_OK = 0
SGL_ERR_INVALID_ARG = -1
SGL_ERR_UNSUPPORTED = -2
SGL_ERR_HIP = -3
SGL_ERR_WORKSPACE = -4

# sgl_dtype
SGL_BF16, SGL_F16, SGL_F32 = 0, 1, 2
# activation-scale formats of sgl_fp4_gemm (SGL_ASCALE_*)
ASCALE_F32, ASCALE_F32_POW2, ASCALE_E8M0 = 0, 1, 2
# sgl_scale_mode
SCALE_TORCH_FP32 = 0
SCALE_TORCH_UE8M0 = 1
SCALE_TILELANG_FP32 = 2
SCALE_TILELANG_UE8M0 = 3
SCALE_KV_UE8M0 = 4
# sgl_score_func
SCORE_SOFTMAX, SCORE_SIGMOID, SCORE_SQRTSOFTPLUS = 0, 1, 2
# sgl_kv_layout
KV_LAYOUT_A, KV_LAYOUT_B = 0, 1
# sgl_expert_format
EXPERT_FP8_BLOCK128, EXPERT_FP4_E2M1 = 0, 1
EXPERT_POW2_SCALES = 2  # flag: every FP8 block scale is a power of two
EXPERT_FRAG_COPY = 4  # flag: a second record set with the FP8 weights in the MFMA fragment layout
# sgl_attn_kv_format
ATTN_KV_BF16, ATTN_KV_A, ATTN_KV_A_PAGED = 0, 1, 2

P = c_void_p
I64 = c_int64

# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES = {
    "sgl_abi_version": (c_int, []),
    "sgl_last_error": (ctypes.c_char_p, []),
    "sgl_probe": (c_int, []),
    "sgl_act_quant": (c_int, [P, I64, I64, I64, P, I64, P, I64, c_int, c_int, c_int, c_int, P]),
    "sgl_weight_quant_128x128": (c_int, [P, c_int, I64, I64, I64, P, I64, P, I64, c_int, P]),
    "sgl_e8m0_to_f32": (c_int, [P, P, I64, P]),
    "sgl_check_conversions": (c_int, [P, P]),
    "sgl_hbm_stream": (c_int, [P, P, I64, P, P]),
    "sgl_mfma_mix": (c_int, [c_int, P, I64, P]),
    "sgl_mfma_mix_threads": (c_int, []),
    "sgl_fp8_gemm": (c_int, [P, P, c_int, P, P, c_int, P, c_int, I64, I64, I64, P, c_size_t, P]),
    "sgl_fp8_gemm_workspace_size": (c_size_t, [I64, I64, I64]),
    "sgl_fp4_gemm": (c_int, [P, P, c_int, P, P, P, c_int, I64, I64, I64, P]),
    "sgl_fp4_to_fp8_weight": (c_int, [P, P, I64, I64, P, P, P]),
    "sgl_fp8_weight_to_frag": (c_int, [P, I64, I64, P, P]),
    "sgl_fp4_weight_to_frag": (c_int, [P, P, I64, I64, P, P, P]),
    "sgl_moe_route_topk": (c_int, [P, I64, c_int, c_int, c_int, P, c_float, P, P, P]),
    "sgl_moe_gate": (
        c_int,
        [P, P, I64, I64, c_int, c_int, c_int, P, c_float, P, I64, P, c_int, P, P, P, P],
    ),
    "sgl_moe_permute": (c_int, [P, I64, c_int, c_int, P, P, P, P, P]),
    "sgl_moe_gate_up": (
        c_int,
        [P, P, I64, I64, I64, c_int, c_int, P, P, P, P, c_int, c_int, c_float, c_int, P, P, P],
    ),
    "sgl_moe_down": (
        c_int, [P, P, I64, I64, I64, c_int, c_int, P, P, P, c_int, c_int, c_int, P, P]
    ),
    "sgl_moe_combine": (c_int, [P, P, I64, c_int, I64, c_int, P, P]),
    "sgl_moe_workspace_size": (c_size_t, [I64, I64, I64, c_int, c_int, c_int]),
    "sgl_moe_forward": (
        c_int,
        [P, I64, I64, I64, c_int, c_int, P, P, P, c_int, c_int, c_float, c_int, P, c_size_t, P, P],
    ),
    "sgl_moe_forward_local": (
        c_int,
        [P, I64, I64, I64, c_int, c_int, P, P, P, c_int, c_int, c_int, c_int, c_float, c_int, P,
         c_size_t, P, P],
    ),
    "sgl_moe_add_shared": (c_int, [P, P, c_size_t, I64, I64, I64, c_int, c_int, P, P]),
    "sgl_moe_forward_noalloc": (
        c_int, [P, I64, I64, I64, c_int, c_int, P, P, P, c_int, c_int, c_float, c_int, P, P],
    ),
    "sgl_kv_pack": (c_int, [P, c_int, I64, I64, c_int, c_int, c_int, c_int, P, P]),
    "sgl_kv_pack_to_pages": (
        c_int, [P, c_int, I64, I64, c_int, P, I64, I64, c_int, I64, c_int, c_int, P, P]
    ),
    "sgl_sparse_attn": (
        c_int,
        [P, I64, I64, c_int, P, c_int, c_int, I64, I64, I64, P, P, I64, c_float, P, P, c_size_t, P],
    ),
    "sgl_sparse_attn_workspace_size": (c_size_t, [I64, I64, c_int, I64]),
    "sgl_kv_to_paged": (c_int, [P, I64, c_int, P, P]),
    "sgl_kv_gather_dequant": (c_int, [P, c_int, c_int, c_int, I64, P, I64, I64, P, P]),
    "sgl_split_swa_compress_indices": (c_int, [P, c_int, I64, I64, I64, P, P, P, P, P]),
    "sgl_host_f32_to_e4m3": (c_int, [P, P, I64]),
    "sgl_host_e4m3_to_f32": (c_int, [P, P, I64]),
    "sgl_host_group_scale": (c_int, [c_int, P, P, I64]),
    "sgl_host_quant_elem": (c_int, [c_int, P, P, P, I64]),
}

_LIB: Optional[ctypes.CDLL] = None


class SglError(RuntimeError):
    """A C-ABI call returned an error status."""

    def __init__(self, what: str, status: int, message: str):
        super().__init__(f"{what}: status {status}: {message}")
        self.status = status
        self.message = message


def load(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Load the library once and bind every declared symbol (raises if any is missing)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    # torch first: the library's libamdhip64.so.7 dependency then resolves to
    # the HIP runtime torch already loaded (same SONAME), so the process has a
    # single runtime and device memory / streams are shared with torch.
    import torch  # noqa: F401

    p = Path(path) if path is not None else LIB_PATH
    if not p.is_file():
        raise RuntimeError(
            f"sglang_lite_amd: native library not built ({p}); run "
            "`python -c 'import __graft_entry__ as g; g.build()'` or "
            "`make -C sglang-lite_amd/csrc`"
        )
    lib = ctypes.CDLL(str(p))
    missing = []
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            missing.append(name)
            continue
        fn.restype = res
        fn.argtypes = args
    if missing:
        raise RuntimeError(f"sglang_lite_amd: library {p} lacks symbols {missing}")
    ver = lib.sgl_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"sglang_lite_amd: ABI version {ver}, expected {ABI_VERSION}")
    if path is None:
        _LIB = lib
    return lib


def last_error() -> str:
    msg = load().sgl_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(status: int, what: str) -> None:
    """Map a C status to the exception type the reference raises for the same condition."""
    if status == SGL_OK:
        return
    msg = last_error()
    if status == SGL_ERR_INVALID_ARG:
        raise ValueError(f"{what}: {msg}")
    if status == SGL_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise SglError(what, status, msg)


def call(name: str, *args) -> None:
    fn = getattr(load(), name)
    check(fn(*args), name)


def ptr(t) -> Optional[int]:
    """Raw device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    """HIP stream handle torch is currently using on ``t``'s device."""
    import torch

    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors, what: str) -> None:
    """The product path runs only on a ROCm device: refuse CPU tensors loudly."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"{what}: sglang_lite_amd runs only on a ROCm (gfx950) device tensor; "
                f"got a {t.device} tensor (there is no CPU path)"
            )
