"""The MFMA fragment layout of expert weights (``sgl_fp8_weight_to_frag``):
the numpy restatement used as the GPU tests' reference, checked element by
element against the layout's definition in include/sglang_lite_amd.h, and
the entry point's argument checks (no GPU compute)."""

from __future__ import annotations

import numpy as np


def frag_layout_ref(w: np.ndarray) -> np.ndarray:
    """[N, K] bytes -> the fragment layout: blocks (n16, kb) in that order,
    each [j (2)][lane (64) = 16 (K quarter) + row][16 bytes]."""
    N, K = w.shape
    return np.ascontiguousarray(
        w.reshape(N // 16, 16, K // 128, 4, 2, 16).transpose(0, 2, 4, 3, 1, 5)).reshape(-1)


def test_reference_matches_definition():
    rng = np.random.default_rng(0)
    N, K = 48, 384
    w = rng.integers(0, 256, size=(N, K), dtype=np.uint8)
    out = frag_layout_ref(w)
    KB = K // 128
    for idx in range(out.size):
        blk, rem = divmod(idx, 2048)
        j, rem = divmod(rem, 1024)
        lane, b = divmod(rem, 16)
        n16, kb = divmod(blk, KB)
        n = 16 * n16 + lane % 16
        k = 128 * kb + 32 * (lane // 16) + 16 * j + b
        assert out[idx] == w[n, k], idx


def test_weight_to_frag_rejects_bad_shapes():
    from sglang_lite_amd import _lib

    lib = _lib.load()
    assert lib.sgl_fp8_weight_to_frag(None, 24, 128, None, None) != 0  # N % 16
    assert b"multiple" in lib.sgl_last_error()
    assert lib.sgl_fp8_weight_to_frag(None, 16, 100, None, None) != 0  # K % 128
    assert lib.sgl_fp8_weight_to_frag(None, 16, 128, None, None) != 0  # null
    assert b"null" in lib.sgl_last_error()
    assert lib.sgl_fp8_weight_to_frag(None, 0, 128, None, None) == 0  # empty: nothing to do
