"""Golden fixture of the tiny MoE layer (the CPU-runnable configuration).

T=32 tokens, hidden 256, expert intermediate 128, 8 routed experts top-2
softmax, 1 shared expert, route_scale 1, no SwiGLU clamp.  Inputs are drawn
on the CPU from ``torch.Generator().manual_seed(1)`` in fp32, then cast:
x bf16 N(0,1) [32,256]; router weight N(0,1)/sqrt(256) [8,256]; per expert
w1, w3 [128,256] and w2 [256,128] N(0,0.02) quantized to e4m3 with 128x128
fp32 block scales (deep_gemm_sm120/utils/math.py:50-60), shared expert
likewise.  Router logits are torch's F.linear(x.float(), W) on the CPU
(deepseek_infer/model.py:572).

Every intermediate of the layer is computed by the oracle and stored in
tiny_moe_seed1.npz: logits, route ids and weights, the permutation (counts,
offsets, sorted_slot, slot_pos), the 1x128 activation quant (xq bytes, xs),
the gate/up output requantized (hq bytes, hs, in permuted-row order with the
shared expert's rows last), and the layer output y (bf16 bits).  A SHA-256 of
the generated weights is stored so a change in torch's RNG stream is caught
instead of silently producing different inputs.

Run from the repository root:  python tests/golden/make_tiny_moe.py
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

T, H, I, E, K_TOP, SEED = 32, 256, 128, 8, 2, 1
PATH = os.path.join(HERE, "tiny_moe_seed1.npz")


def make_inputs(seed: int = SEED):
    import torch
    import torch.nn.functional as F

    from oracle import quant as Q

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w_router = torch.randn(E, H, generator=g) * (H ** -0.5)

    def expert():
        out = {}
        for name, shape in (("1", (I, H)), ("3", (I, H)), ("2", (H, I))):
            w = (torch.randn(*shape, generator=g) * 0.02).numpy().astype(np.float32)
            q, s = Q.per_block_cast_to_fp8(w)
            out["w" + name] = q
            out["s" + name] = s
        return out

    experts = [expert() for _ in range(E)]
    shared = expert()
    logits = F.linear(x.float(), w_router).numpy().astype(np.float32)
    x_f32 = x.float().numpy()
    return {"x": x_f32, "logits": logits, "experts": experts, "shared": shared}


def weights_digest(inp) -> str:
    h = hashlib.sha256()
    for e in inp["experts"] + [inp["shared"]]:
        for key in ("w1", "s1", "w3", "s3", "w2", "s2"):
            h.update(np.ascontiguousarray(e[key]).tobytes())
    return h.hexdigest()


def compute(inp):
    from oracle import moe as OM
    from oracle import quant as Q

    x = inp["x"]
    w, ids = OM.route_topk(inp["logits"], K_TOP)
    perm = OM.permute(ids, E)
    xq, xs = Q.scale_mode_quant(x, 0, 128)
    hq_rows, hs_rows = [], []
    for e in range(E):
        tok, top = np.nonzero(ids == e)
        if tok.size == 0:
            continue
        tr = {}
        OM.expert_forward(x[tok], inp["experts"][e], w[tok, top][:, None], trace=tr)
        hq_rows.append(tr["hq"])
        hs_rows.append(tr["hs"])
    tr = {}
    OM.expert_forward(x, inp["shared"], None, trace=tr)
    hq_rows.append(tr["hq"])
    hs_rows.append(tr["hs"])
    y = OM.moe_forward(x, ids, w, inp["experts"], inp["shared"])
    return {
        "logits": inp["logits"],
        "ids": ids.astype(np.int32),
        "route_w": w.astype(np.float32),
        "counts": perm["counts"],
        "offsets": perm["offsets"],
        "sorted_slot": perm["sorted_slot"],
        "slot_pos": perm["slot_pos"],
        "xq": xq,
        "xs": xs.astype(np.float32),
        "hq": np.concatenate(hq_rows, axis=0),
        "hs": np.concatenate(hs_rows, axis=0).astype(np.float32),
        "y_bf16_bits": (y.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16),
    }


def main():
    inp = make_inputs()
    out = compute(inp)
    out["x_bf16_bits"] = (inp["x"].view(np.uint32) >> 16).astype(np.uint16)
    out["weights_sha256"] = np.frombuffer(weights_digest(inp).encode(), dtype=np.uint8)
    np.savez_compressed(PATH, **out)
    print(f"wrote {PATH}")


if __name__ == "__main__":
    main()
