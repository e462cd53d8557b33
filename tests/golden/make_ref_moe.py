"""Write the MoE golden vectors from the reference's own layer code.

Why an import: the oracle's MoE composition (oracle/moe.py expert_forward /
moe_forward) restates the reference's order of operations -- one act_quant
for gate and up, bf16 GEMM outputs upcast, the asymmetric SwiGLU clamp, the
routing weight applied before w2, bf16 h, the ascending-expert fp32 combine,
the shared expert added last -- and nothing but its own output checked it.
These vectors come from the reference's code for that composition instead.

What runs (when the fixtures are generated; the tests read only the
committed vectors):

* ``engine/vendor/deepseek_infer/model.py`` -- the official ``Gate``,
  ``Expert``, ``MoE`` and ``Linear`` / ``linear`` classes, loaded as module
  ``model`` with a stand-in ``kernel`` module (the real one imports TileLang,
  absent here, and needs an NVIDIA GPU);
* ``engine/v4_moe_fast.py`` -- ``_moe_forward_activated_only`` and
  ``_expert_forward_fused``, whose output must equal the official forward
  bit for bit;
* ``engine/vendor/deep_gemm_sm120/utils/math.py`` -- loaded by file path
  (never the package ``__init__``, which loads a compiled extension) for
  ``per_token_cast_to_fp8`` (the stand-in ``act_quant``),
  ``per_block_cast_to_fp8`` (weights) and ``_dequantize_from_fp4_e2m1``.

The stand-in ``kernel.fp8_gemm`` / ``fp4_gemm`` are dequantize-to-fp32
products: A * sa and B * sb exactly in float64, the sum over K in float64,
rounded to fp32 and then to bf16 (the model's default dtype, kernel.py:270).

Stored per case (``ref_moe_<case>.npz``, inputs in ``ref_moe_cases.py``):
router logits (F.linear(x.float(), W.float()), model.py:565) and the Gate's
indices / weights; the 1x128 quant of x (bytes, scales); per routed expert in
ascending id with its rows in token order, then the shared expert: h = the
input of w2's act_quant (bf16 bits), its quant (bytes, scales) and the
expert output (bf16 bits); the layer output y (bf16 bits); a digest of the
expert weights.

Run from the repository root:  python tests/golden/make_ref_moe.py
"""

from __future__ import annotations

import importlib.util
import os
import sys
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import ref_moe_cases as C  # noqa: E402

REF = "/root/reference/engine"


def _load(modname, rel, register=False):
    spec = importlib.util.spec_from_file_location(modname, os.path.join(REF, rel))
    mod = importlib.util.module_from_spec(spec)
    if register:
        sys.modules[modname] = mod
    spec.loader.exec_module(mod)
    return mod


def _reference():
    import torch

    dgm = _load("_ref_dg_math", "vendor/deep_gemm_sm120/utils/math.py")
    calls = []
    kernel = types.ModuleType("kernel")

    def act_quant(x, block_size=128, scale_fmt=None, scale_dtype=torch.float32, inplace=False):
        assert block_size == 128 and not inplace
        shape = x.shape
        q, s = dgm.per_token_cast_to_fp8(x.reshape(-1, shape[-1]), use_ue8m0=scale_fmt is not None)
        s = s.to(scale_dtype)
        calls.append((x.detach().clone(), q, s))
        return q.view(shape), s.view(*shape[:-1], -1)

    def _product(a, a_s, b_val):
        A = a.reshape(-1, a.shape[-1]).double() * \
            a_s.reshape(-1, a_s.shape[-1]).double().repeat_interleave(128, dim=1)
        c = (A @ b_val.double().T).float().to(torch.bfloat16)
        return c.view(*a.shape[:-1], b_val.shape[0])

    def fp8_gemm(a, a_s, b, b_s, scale_dtype=torch.float32):
        N, K = b.shape
        sb = b_s.double().repeat_interleave(128, 0).repeat_interleave(128, 1)[:N, :K]
        return _product(a.float(), a_s.float(), b.float().double() * sb)

    def fp4_gemm(a, a_s, b, b_s, scale_dtype=torch.float32):
        p = b.view(torch.uint8)
        codes = torch.empty(p.shape[0], p.shape[1] * 2, dtype=torch.int8)
        codes[:, 0::2] = (p & 0x0F).to(torch.int8)
        codes[:, 1::2] = (p >> 4).to(torch.int8)
        val = dgm._dequantize_from_fp4_e2m1(codes).double() * \
            b_s.float().double().repeat_interleave(32, dim=1)
        return _product(a.float(), a_s.float(), val)

    def _absent(*a, **k):
        raise NotImplementedError("not on the MoE path")

    kernel.act_quant, kernel.fp8_gemm, kernel.fp4_gemm = act_quant, fp8_gemm, fp4_gemm
    kernel.fp4_act_quant = kernel.sparse_attn = kernel.hc_split_sinkhorn = _absent
    sys.modules["kernel"] = kernel
    model = _load("model", "vendor/deepseek_infer/model.py", register=True)
    fast = _load("_ref_v4_moe_fast", "v4_moe_fast.py")
    return dgm, model, fast, calls


def build_layer(name, dgm, model):
    import torch
    import torch.nn as nn

    c = C.CASES[name]
    inp = C.draw(name)
    model.default_dtype = torch.float8_e4m3fn
    model.scale_fmt = "ue8m0" if c["ue8m0"] else None
    model.scale_dtype = torch.float8_e8m0fnu if c["ue8m0"] else torch.float32
    args = model.ModelArgs(dim=c["H"], moe_inter_dim=c["I"], n_routed_experts=c["E"],
                           n_activated_experts=c["k"], score_func=c["score_func"],
                           route_scale=c["route_scale"], swiglu_limit=c["swiglu_limit"],
                           n_hash_layers=0, expert_dtype="fp4" if c["fp4"] else None)
    moe = model.MoE(1, args)
    moe.gate.weight = nn.Parameter(torch.from_numpy(inp["w_router"]), requires_grad=False)
    if inp["bias"] is None:
        moe.gate.bias = None
    else:
        moe.gate.bias = nn.Parameter(torch.from_numpy(inp["bias"]), requires_grad=False)

    stored = []

    def fill_fp8(lin, w):
        q, s = dgm.per_block_cast_to_fp8(torch.from_numpy(w), use_ue8m0=c["ue8m0"])
        lin.weight = nn.Parameter(q, requires_grad=False)
        lin.weight.scale = s.to(torch.float8_e8m0fnu) if c["ue8m0"] else s
        sv = lin.weight.scale.view(torch.uint8) if c["ue8m0"] else lin.weight.scale
        return q.view(torch.uint8).numpy().copy(), sv.numpy().copy()

    def fill_fp4(lin, wb, sb):
        lin.weight = nn.Parameter(torch.from_numpy(wb.copy()).view(torch.float4_e2m1fn_x2),
                                  requires_grad=False)
        lin.weight.scale = torch.from_numpy(sb.copy()).view(torch.float8_e8m0fnu)
        return wb, sb

    for e_mod, e_in in list(zip(moe.experts, inp["experts"])) + [(moe.shared_experts, inp["shared"])]:
        rec = {}
        for nm in ("1", "3", "2"):
            lin = getattr(e_mod, "w" + nm)
            if "s" + nm in e_in:
                rec["w" + nm], rec["s" + nm] = fill_fp4(lin, e_in["w" + nm], e_in["s" + nm])
            else:
                rec["w" + nm], rec["s" + nm] = fill_fp8(lin, e_in["w" + nm])
        stored.append(rec)
    return moe, inp, stored


def run_case(name, dgm, model, fast, calls):
    import torch
    import torch.nn.functional as F

    c = C.CASES[name]
    moe, inp, stored = build_layer(name, dgm, model)
    x = torch.from_numpy(inp["x"]).to(torch.bfloat16)
    input_ids = torch.zeros(c["T"], dtype=torch.int64)
    with torch.no_grad():
        logits = F.linear(x.float(), moe.gate.weight.float())
        weights, indices = moe.gate(x, input_ids)
        y = moe(x, input_ids)
        # the reference's fast dispatch: must equal the official loop bit for bit
        orig = model.Expert.forward
        model.Expert.forward = fast._expert_forward_fused
        try:
            y_fast = fast._moe_forward_activated_only(moe, x, input_ids)
        finally:
            model.Expert.forward = orig
        assert torch.equal(y.view(torch.int16), y_fast.view(torch.int16)), f"{name}: fast != official"
        # per expert (ascending id, rows in token order) and the shared expert:
        # w2's act_quant input h, its quant, and the expert output
        h, hq, hs, out = [], [], [], []
        for e in range(c["E"] + 1):
            if e < c["E"]:
                idx, top = torch.where(indices == e)
                if idx.numel() == 0:
                    continue
                calls.clear()
                o = moe.experts[e](x[idx], weights[idx, top, None])
            else:
                calls.clear()
                o = moe.shared_experts(x)
            xin, q, s = calls[-1]  # the w2 linear's act_quant
            h.append(xin.view(torch.int16).numpy().astype(np.uint16))
            hq.append(q.view(torch.uint8).numpy())
            hs.append(s.float().numpy())
            out.append(o.view(torch.int16).numpy().astype(np.uint16))
        calls.clear()
        xq, xs = sys.modules["kernel"].act_quant(x, 128, model.scale_fmt, torch.float32)
    res = {
        "logits": logits.numpy().astype(np.float32),
        "ids": indices.numpy().astype(np.int64),
        "route_w": weights.numpy().astype(np.float32),
        "xq": xq.view(torch.uint8).numpy(),
        "xs": xs.float().numpy(),
        "h_bits": np.concatenate(h),
        "hq": np.concatenate(hq),
        "hs": np.concatenate(hs).astype(np.float32),
        "out_bits": np.concatenate(out),
        "y_bits": y.view(torch.int16).numpy().astype(np.uint16),
        "weights_sha256": np.frombuffer(C.digest(stored[:-1], stored[-1]).encode(), dtype=np.uint8),
    }
    return res


def main():
    dgm, model, fast, calls = _reference()
    for name in C.CASES:
        res = run_case(name, dgm, model, fast, calls)
        np.savez_compressed(C.path(name), **res)
        print(f"wrote {C.path(name)}: ids {res['ids'].shape}, h rows {res['h_bits'].shape[0]}")


if __name__ == "__main__":
    main()
