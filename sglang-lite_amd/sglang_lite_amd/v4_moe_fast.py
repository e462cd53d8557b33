"""MoE / Expert forward replacements for the official DeepSeek-V4 graph on gfx950.

Drop-in counterpart of ``engine/v4_moe_fast.py`` (``moe_fast_enabled`` :26-28,
``_expert_forward_fused`` :43-76, ``_moe_forward_activated_only`` :79-106,
``attach_v4_moe_fast`` :109-152).  Where the reference walks the activated
experts on the host (``torch.unique(...).tolist()`` and one ``torch.where``
per expert, both device->host syncs), the replacement runs the whole layer as
five HIP launches with no host sync: 1x128 act quant, stable permutation,
grouped gate/up (+SwiGLU, routing weight, requant), grouped down, ordered
combine with the shared expert.  Routed experts may be FP8 (128x128 scales)
or MXFP4 (``expert_dtype="fp4"``, model.py:623-624: packed e2m1 with e8m0
1x32 scales, the reference's live format); the shared expert is FP8.  Results follow the reference's arithmetic:
weight applied before ``w2``, fp32 sum over experts in ascending id, shared
expert added last, bf16 out.

Routing: the router projection stays ``F.linear(x.float(), W.float())`` as
in ``Gate.forward`` (model.py:565; a plain fp32 library GEMM), then the HIP
top-k kernel applies score function, bias, top-k, renormalisation and
route_scale.  Hash-routed layers (model.py:576-577) keep the official gate.

Env: ``SGLANG_LITE_V4_MOE_FAST=0`` keeps the official forwards (same switch as
the reference).
"""

from __future__ import annotations

import logging
import os
import sys
from typing import Any, Optional

import torch
import torch.nn.functional as F

from . import kernel as HK
from . import moe as HM
from .v4_deep_gemm import is_fp4_weight

logger = logging.getLogger("sglang_lite_amd.v4_moe_fast")
MARK = "_sglang_lite_moe_fast"


def moe_fast_enabled() -> bool:
    raw = os.environ.get("SGLANG_LITE_V4_MOE_FAST", "1").strip().lower()
    return raw not in ("0", "false", "no", "off")


def frag_layout_enabled() -> bool:
    """``SGLANG_LITE_AMD_FRAG_LAYOUT=1``: the MoE layers' expert tables also
    keep fragment-layout copies of the FP8 expert weights (the register-fed
    GEMMs; a second copy of those weights).  Off by default.  A switch of this
    build, not of the reference."""
    raw = os.environ.get("SGLANG_LITE_AMD_FRAG_LAYOUT", "0").strip().lower()
    return raw in ("1", "true", "yes", "on")


def _official_model():
    M = sys.modules.get("model")
    if M is None:
        raise RuntimeError("official DeepSeek-V4 'model' module is not loaded")
    return M


def _is_fp8(linear) -> bool:
    w = getattr(linear, "weight", None)
    return w is not None and w.dtype == torch.float8_e4m3fn and getattr(w, "scale", None) is not None


def _is_fp4(linear) -> bool:
    w = getattr(linear, "weight", None)
    return w is not None and getattr(w, "scale", None) is not None and is_fp4_weight(w)


def _quantized(expert) -> bool:
    """Every projection FP8, or every projection FP4."""
    lins = (expert.w1, expert.w3, expert.w2)
    return all(_is_fp8(l) for l in lins) or all(_is_fp4(l) for l in lins)


def _expert_entry(expert):
    return (expert.w1.weight.data, expert.w3.weight.data, expert.w2.weight.data,
            expert.w1.weight.scale.data, expert.w3.weight.scale.data, expert.w2.weight.scale.data)


def _scale_mode():
    M = sys.modules.get("model")
    return HK.scale_mode_for(getattr(M, "scale_fmt", None) if M is not None else None)


def expert_table(moe) -> HM.ExpertTable:
    """Device pointer table of a MoE module's experts + shared expert (cached);
    the experts another rank holds (None, model.py:616-625) get null records."""
    tab = getattr(moe, "_sgl_table", None)
    if tab is None:
        experts = [None if e is None else _expert_entry(e) for e in moe.experts]
        tab = HM.ExpertTable.build(experts, _expert_entry(moe.shared_experts),
                                   frag_layout=frag_layout_enabled())
        moe._sgl_table = tab
    return tab


def _expert_forward_fused(self, x: torch.Tensor, weights: Optional[torch.Tensor] = None):
    """Expert SwiGLU (model.py:596-606 / v4_moe_fast.py:43-76) for FP8 or FP4
    experts as a one-expert grouped launch; bf16 experts use the official forward."""
    if not _quantized(self):
        return self._sgl_orig_forward(x, weights)  # bf16 experts: not this path
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    T = x2.shape[0]
    tab = getattr(self, "_sgl_table", None)
    if tab is None:
        tab = HM.ExpertTable.build([_expert_entry(self)])
        self._sgl_table = tab
    ids = torch.zeros(T, 1, dtype=torch.int32, device=x.device)
    if weights is None:
        w = torch.ones(T, 1, dtype=torch.float32, device=x.device)
    else:
        w = weights.reshape(T, 1).to(torch.float32)
    lim = float(getattr(self, "swiglu_limit", 0) or 0)
    xb = x2 if x2.dtype == torch.bfloat16 else x2.to(torch.bfloat16)
    y = HM.moe_forward(xb, ids, w, tab, swiglu_limit=lim, scale_mode=_scale_mode())
    return y.to(x.dtype).view(*shape[:-1], y.shape[-1])


def _gate_topk(gate, x: torch.Tensor, input_ids: torch.Tensor):
    """Gate.forward (model.py:564-584).  bf16 router weights (the checkpoint's
    dtype) take the fused gate kernel, hash-routed layers included; other
    dtypes keep torch's fp32 projection followed by the top-k kernel."""
    hashed = bool(getattr(gate, "hash", False))
    if gate.weight.dtype == torch.bfloat16 and x.dtype == torch.bfloat16:
        return HM.gate(x, gate.weight, int(gate.topk), str(gate.score_func),
                       None if hashed else getattr(gate, "bias", None), float(gate.route_scale),
                       tid2eid=gate.tid2eid if hashed else None,
                       input_ids=input_ids if hashed else None)
    if hashed:
        return gate(x, input_ids.flatten())
    logits = F.linear(x.float(), gate.weight.float())
    weights, ids = HM.route_topk(logits, int(gate.topk), str(gate.score_func),
                                 getattr(gate, "bias", None), float(gate.route_scale))
    return weights, ids


def _local_range(moe):
    """``(ok, lo, hi)`` of a MoE module, decided once and cached: the rank's
    expert range ``[experts_start_idx, experts_end_idx)`` (model.py:616-625),
    and whether the device path can run it -- every expert in the range
    present and quantized alike (all FP8 or all FP4) and an FP8 shared expert."""
    st = getattr(moe, "_sgl_range", None)
    if st is None:
        E = len(moe.experts)
        lo = int(getattr(moe, "experts_start_idx", 0))
        hi = int(getattr(moe, "experts_end_idx", E))
        local = list(moe.experts[lo:hi]) if 0 <= lo <= hi <= E else []
        ok = bool(local) and all(e is not None for e in local) and \
            _is_fp8(moe.shared_experts.w1) and _quantized(moe.shared_experts) and \
            (all(_is_fp8(e.w1) and _quantized(e) for e in local) or
             all(_is_fp4(e.w1) and _quantized(e) for e in local))
        st = (ok, lo, hi)
        moe._sgl_range = st
    return st


def _moe_forward_fused(self, x: torch.Tensor, input_ids: torch.Tensor):
    """The whole MoE layer (v4_moe_fast.py:79-106) on the device, no host sync.

    An expert-sharded rank (``world_size > 1``, or a module that holds only
    the experts ``[experts_start_idx, experts_end_idx)``) computes the fp32 sum
    of its local experts' outputs, calls ``dist.all_reduce`` on it exactly
    where the reference does (v4_moe_fast.py:103-104), then adds the shared
    expert and rounds to bf16."""
    ok, lo, hi = _local_range(self)
    if not ok:  # bf16 experts, mixed formats, missing local experts: not this path
        return self._sgl_orig_forward(x, input_ids)
    M = sys.modules.get("model")
    world = int(getattr(M, "world_size", 1) or 1) if M is not None else 1
    shape = x.size()
    x2 = x.view(-1, self.dim)
    weights, ids = _gate_topk(self.gate, x2, input_ids)
    lim = float(getattr(self.shared_experts, "swiglu_limit", 0) or 0)
    xb = x2 if x2.dtype == torch.bfloat16 else x2.to(torch.bfloat16)
    ws = getattr(self, "_sgl_ws", None)
    if ws is None:
        ws = HM.MoEWorkspace()
        self._sgl_ws = ws
    tab = expert_table(self)
    if world == 1 and lo == 0 and hi == len(self.experts):
        y = HM.moe_forward(xb, ids, weights, tab, swiglu_limit=lim, scale_mode=_scale_mode(),
                           workspace=ws)
        return y.type_as(x).view(shape)
    y32 = HM.moe_forward_local(xb, ids, weights, tab, lo, hi, swiglu_limit=lim,
                               scale_mode=_scale_mode(), workspace=ws)
    if world > 1:
        M.dist.all_reduce(y32)
    y = HM.moe_add_shared(y32, tab, ids.shape[1], ws)
    return y.type_as(x).view(shape)


def attach_v4_moe_fast(model: Any) -> dict:
    """Patch the official ``MoE.forward`` / ``Expert.forward`` (class level)
    after a device probe.  Returns the reference's stats keys plus
    ``backend`` and ``probe``; never raises."""
    stats = {"enabled": False, "moe_class_patched": 0, "expert_class_patched": 0,
             "moe_modules": 0, "expert_modules": 0, "backend": "official", "probe": None}
    if not moe_fast_enabled():
        return stats
    import sglang_lite_amd

    probe = sglang_lite_amd.probe()
    stats["probe"] = probe
    if not probe.get("ok"):
        print(f"[sglang-lite-amd] MoE fast skipped (probe failed: {probe.get('error')})")
        return stats
    try:
        M = _official_model()
    except RuntimeError as e:
        stats["error"] = str(e)
        return stats
    MoE, Expert = M.MoE, M.Expert
    if getattr(MoE.forward, MARK, False) is not True:
        MoE._sgl_orig_forward = MoE.forward
        MoE.forward = _moe_forward_fused
        setattr(MoE.forward, MARK, True)
        stats["moe_class_patched"] = 1
    if getattr(Expert.forward, MARK, False) is not True:
        Expert._sgl_orig_forward = Expert.forward
        Expert.forward = _expert_forward_fused
        setattr(Expert.forward, MARK, True)
        stats["expert_class_patched"] = 1
    stats["moe_modules"] = sum(1 for m in model.modules() if isinstance(m, MoE))
    stats["expert_modules"] = sum(1 for m in model.modules() if isinstance(m, Expert))
    stats["enabled"] = True
    stats["backend"] = "gfx950_hip"
    print(f"[sglang-lite-amd] MoE fast armed (grouped FP8 MFMA, on-device dispatch); "
          f"moe_modules={stats['moe_modules']} expert_modules={stats['expert_modules']}")
    return stats


def detach_v4_moe_fast() -> None:
    M = sys.modules.get("model")
    if M is None:
        return
    for cls in (M.MoE, M.Expert):
        orig = cls.__dict__.get("_sgl_orig_forward")
        if orig is not None:
            cls.forward = orig
            del cls._sgl_orig_forward


__all__ = ["attach_v4_moe_fast", "detach_v4_moe_fast", "expert_table", "frag_layout_enabled",
           "moe_fast_enabled"]
