"""Write the FP4 -> FP8 weight-repack golden vectors from the reference's
``cast_e2m1fn_to_e4m3fn`` (engine/vendor/deepseek_infer/convert.py:17-52).

Why an import: the oracle's repack (oracle/fp4.py fp4_to_fp8_repack) was
pinned by its value invariants, which cannot see the sign of a zero: the
e4m3 byte of e2m1 code 8 (the format's -0) is 0x00 in the converter
(FP4_TABLE[8] = +0.0, convert.py:11-14) and 0x80 under a plain OCP decode.
These vectors fix the bytes.

convert.py is loaded by file path in this container only (it imports torch,
safetensors and tqdm at module level; only the cast function is called).
Inputs (drawn from a seeded torch.Generator on the CPU): a [256, 512] FP4
weight with uniform codes and e8m0 scales spread over 2^10 (so some blocks
round), whose first 128 x 128 block is all 0x88 bytes (every nibble code 8)
and whose second block mixes code 8 with code 0.  Stored in
``ref_fp4_repack.npz``: packed bytes, scale bytes, the repacked e4m3 bytes
and the e8m0 block-scale bytes.

Run from the repository root:  python tests/golden/make_ref_fp4_repack.py
"""

from __future__ import annotations

import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "ref_fp4_repack.npz")
CONVERT = "/root/reference/engine/vendor/deepseek_infer/convert.py"
N, K, SEED = 256, 512, 21


def make_inputs():
    import torch

    g = torch.Generator().manual_seed(SEED)
    bp = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    sb = torch.randint(112, 123, (N, K // 32), generator=g, dtype=torch.uint8)
    bp[:128, :64] = 0x88
    mix = torch.randint(0, 2, (128, 64), generator=g, dtype=torch.uint8)
    bp[:128, 64:128] = mix * 0x08 + (1 - mix) * 0x80
    return bp.numpy(), sb.numpy()


def main():
    import torch

    spec = importlib.util.spec_from_file_location("_ref_convert", CONVERT)
    conv = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(conv)
    bp, sb = make_inputs()
    q, s = conv.cast_e2m1fn_to_e4m3fn(torch.from_numpy(bp).view(torch.int8),
                                      torch.from_numpy(sb).view(torch.float8_e8m0fnu))
    np.savez_compressed(PATH, bp=bp, sb=sb, q=q.view(torch.uint8).numpy(),
                        s=s.view(torch.uint8).numpy())
    print(f"wrote {PATH}")


if __name__ == "__main__":
    main()
