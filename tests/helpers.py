"""Shared test helpers: numpy <-> device tensors and the GEMM tolerance."""

from __future__ import annotations

import numpy as np
import torch

# GEMM outputs (bf16) against the dequantize-to-fp32 reference: rel-L2 <= 1e-2
# and |out - ref| <= 2e-2 + 2^-7 * |ref| elementwise (2e-2 absolute plus one
# bf16 ulp of the reference, since a bf16 output cannot hold 2e-2 absolute
# accuracy above |C| = 8).
REL_L2 = 1e-2
ATOL = 2e-2
RTOL_BF16 = 2.0 ** -7


def to_dev_u8(a: np.ndarray, dev, dtype=torch.uint8) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.uint8))
    return t.view(dtype).to(dev) if dtype != torch.uint8 else t.to(dev)


def to_dev_fp8(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).view(torch.float8_e4m3fn).to(dev)


def to_dev_f32(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def to_dev_bf16(a: np.ndarray, dev) -> torch.Tensor:
    """float32 array holding bf16 values -> exact bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(dev)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).cpu().numpy()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def assert_gemm_close(out: np.ndarray, ref: np.ndarray, what: str = "gemm") -> float:
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    denom = max(np.linalg.norm(ref), 1e-30)
    rel = float(np.linalg.norm(out - ref) / denom)
    err = np.abs(out - ref)
    bound = ATOL + RTOL_BF16 * np.abs(ref)
    bad = int(np.sum(err > bound))
    assert rel <= REL_L2, f"{what}: rel-L2 {rel:.3e} > {REL_L2}"
    assert bad == 0, f"{what}: {bad} elements beyond 2e-2 + 2^-7|ref| (max err {err.max():.3e})"
    return rel


def bf16_values(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    from oracle.quant import bf16_round

    return bf16_round((rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32))
