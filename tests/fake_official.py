"""A stand-in for the official DeepSeek-V4 ``model`` / ``kernel`` modules with
the attributes the drop-in reads (deepseek_infer/model.py:15-21,108-120,
123-152,546-644; kernel.py:105,257): module globals, Linear with an FP8 weight
Parameter carrying ``.scale``, Gate, Expert, MoE.  The official forwards here
raise: tests check the patched forwards against the oracle instead."""

from __future__ import annotations

import sys
import types

import torch
from torch import nn


def _unpatched(*a, **k):
    raise NotImplementedError("official TileLang kernels are not available here")


def install():
    K = types.ModuleType("kernel")
    K.act_quant = _unpatched
    K.fp8_gemm = _unpatched
    K.fp4_gemm = _unpatched
    K.sparse_attn = _unpatched
    M = types.ModuleType("model")
    M.world_size = 1
    M.rank = 0
    M.block_size = 128
    M.scale_fmt = None
    M.scale_dtype = torch.float32
    M.act_quant = K.act_quant
    M.fp8_gemm = K.fp8_gemm
    M.fp4_gemm = K.fp4_gemm
    M.sparse_attn = K.sparse_attn

    def linear(x, weight, bias=None):
        """The dispatch of model.py:108-120 on the module's (patchable) names."""
        assert bias is None
        if weight.dtype == torch.float4_e2m1fn_x2:
            xq, s = M.act_quant(x, M.block_size, M.scale_fmt, M.scale_dtype)
            return M.fp4_gemm(xq, s, weight, weight.scale, M.scale_dtype)
        if weight.dtype == torch.float8_e4m3fn:
            xq, s = M.act_quant(x, M.block_size, M.scale_fmt, M.scale_dtype)
            return M.fp8_gemm(xq, s, weight, weight.scale, M.scale_dtype)
        return torch.nn.functional.linear(x, weight)

    M.linear = linear

    class Linear(nn.Module):
        def __init__(self, w_q: torch.Tensor, s: torch.Tensor):
            super().__init__()
            self.weight = nn.Parameter(w_q, requires_grad=False)
            self.weight.scale = self.scale = nn.Parameter(s, requires_grad=False)

        def forward(self, x):
            return _unpatched()

    class Gate(nn.Module):
        def __init__(self, W, topk, score_func="softmax", route_scale=1.0, bias=None, tid2eid=None):
            super().__init__()
            self.weight = nn.Parameter(W, requires_grad=False)
            self.topk, self.score_func, self.route_scale = topk, score_func, route_scale
            self.hash = tid2eid is not None
            if self.hash:
                self.tid2eid = nn.Parameter(tid2eid, requires_grad=False)
            self.bias = None if bias is None else nn.Parameter(bias, requires_grad=False)

        def forward(self, x, input_ids=None):
            return _unpatched()

    class Expert(nn.Module):
        def __init__(self, ws, swiglu_limit=0.0):
            super().__init__()
            w1, w3, w2, s1, s3, s2 = ws
            self.w1, self.w3, self.w2 = Linear(w1, s1), Linear(w3, s3), Linear(w2, s2)
            self.swiglu_limit = swiglu_limit

        def forward(self, x, weights=None):
            return _unpatched()

    class MoE(nn.Module):
        def __init__(self, dim, gate, experts, shared):
            super().__init__()
            self.dim = dim
            self.gate = gate
            self.n_routed_experts = len(experts)
            self.experts_start_idx, self.experts_end_idx = 0, len(experts)
            self.experts = nn.ModuleList(experts)
            self.shared_experts = shared

        def forward(self, x, input_ids):
            return _unpatched()

    M.Linear, M.Gate, M.Expert, M.MoE = Linear, Gate, Expert, MoE
    saved = {n: sys.modules.get(n) for n in ("model", "kernel")}
    sys.modules["kernel"] = K
    sys.modules["model"] = M
    return M, K, saved


def uninstall(saved):
    for n, m in saved.items():
        if m is None:
            sys.modules.pop(n, None)
        else:
            sys.modules[n] = m
