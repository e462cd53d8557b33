"""Inputs of the reference-generated MoE golden vectors (``ref_moe_*.npz``).

Every input is drawn on the CPU from a seeded ``torch.Generator`` (fp32, then
cast), so the script that writes the fixtures (``make_ref_moe.py``, run once
in a container holding the reference) and the tests that read them rebuild
the same values.  FP8 weights are quantized afterwards: by the reference's
``per_block_cast_to_fp8`` in the script, by the oracle's restatement in the
tests; a SHA-256 of the quantized bytes, stored in the fixture, shows the two
agree (and catches a change in torch's RNG stream).

Cases (the layer configuration of deepseek_infer/model.py:613-627):

* ``tiny``: T=32, hidden 256, intermediate 128, 8 experts top-2, softmax, no
  bias, route_scale 1, no SwiGLU clamp, fp32 activation and weight scales.
* ``live_fp8``: T=40, hidden 256, intermediate 256, 16 experts top-6,
  sqrtsoftplus with a selection bias, route_scale 1.5, swiglu_limit 10,
  ue8m0 activation scales and e8m0 weight scales (config.json's
  ``scale_fmt: "ue8m0"``; FP8 Linear scales are float8_e8m0fnu,
  model.py:138-142).  w1/w3 are drawn wide (std 0.5) so the clamp binds.
* ``live_fp4``: ``live_fp8`` with MXFP4 routed experts (model.py:129-137:
  packed e2m1 + e8m0 1x32 scales, codes drawn uniformly, every nibble code
  including 8 present) and the FP8 shared expert.
"""

from __future__ import annotations

import hashlib
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    "tiny": dict(seed=11, T=32, H=256, I=128, E=8, k=2, score_func="softmax", bias=False,
                 route_scale=1.0, swiglu_limit=0.0, ue8m0=False, fp4=False, std13=0.02),
    "live_fp8": dict(seed=12, T=40, H=256, I=256, E=16, k=6, score_func="sqrtsoftplus", bias=True,
                     route_scale=1.5, swiglu_limit=10.0, ue8m0=True, fp4=False, std13=0.5),
    "live_fp4": dict(seed=13, T=40, H=256, I=256, E=16, k=6, score_func="sqrtsoftplus", bias=True,
                     route_scale=1.5, swiglu_limit=10.0, ue8m0=True, fp4=True, std13=0.5),
}


def path(name: str) -> str:
    return os.path.join(HERE, f"ref_moe_{name}.npz")


def draw(name: str):
    """Raw inputs of a case: x (bf16 values as fp32), router weight (bf16
    values as fp32), bias, and per expert either fp32 weights to be
    quantized 128x128 (FP8) or packed e2m1 bytes + e8m0 scale bytes (FP4).
    The last expert entry is the shared expert (always FP8)."""
    import torch

    c = CASES[name]
    g = torch.Generator().manual_seed(c["seed"])
    T, H, I, E = c["T"], c["H"], c["I"], c["E"]
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).float().numpy()
    w_router = (torch.randn(E, H, generator=g) * (H ** -0.5)).to(torch.bfloat16).float().numpy()
    bias = (torch.randn(E, generator=g) * 0.1).numpy().astype(np.float32) if c["bias"] else None

    def fp8_expert():
        return {"w1": (torch.randn(I, H, generator=g) * c["std13"]).numpy().astype(np.float32),
                "w3": (torch.randn(I, H, generator=g) * c["std13"]).numpy().astype(np.float32),
                "w2": (torch.randn(H, I, generator=g) * 0.02).numpy().astype(np.float32)}

    def fp4_expert():
        out = {}
        for nm, (n, kk) in (("1", (I, H)), ("3", (I, H)), ("2", (H, I))):
            out["w" + nm] = torch.randint(0, 256, (n, kk // 2), generator=g, dtype=torch.uint8).numpy()
            lo = 120 if nm == "2" else 124  # w1/w3 values up to 6 * 2^-3: the clamp binds
            out["s" + nm] = torch.randint(lo - 3, lo + 1, (n, kk // 32), generator=g,
                                          dtype=torch.uint8).numpy()
        return out

    experts = [fp4_expert() if c["fp4"] else fp8_expert() for _ in range(E)]
    shared = fp8_expert()
    return {"x": x, "w_router": w_router, "bias": bias, "experts": experts, "shared": shared}


def digest(experts, shared) -> str:
    """SHA-256 over the quantized bytes and scales of every expert (w1, s1,
    w3, s3, w2, s2 in order; scales as stored: fp32 or e8m0 bytes)."""
    h = hashlib.sha256()
    for e in list(experts) + [shared]:
        for key in ("w1", "s1", "w3", "s3", "w2", "s2"):
            h.update(np.ascontiguousarray(e[key]).tobytes())
    return h.hexdigest()
