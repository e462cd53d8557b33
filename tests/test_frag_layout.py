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


def frag_fp4_layout_ref(w: np.ndarray, s: np.ndarray):
    """Packed e2m1 [N, K/2] and e8m0 [N, K/32] bytes -> the FP4 fragment
    layout: weights blocks (n16, kb) of [lane (64) = 16 (K quarter) + row][16
    packed bytes]; scales blocks (n16, group q of four 128-deep blocks) of
    [lane][4 bytes: the lane's scale for each of the group's stages]."""
    N, KH = w.shape
    KB = 2 * KH // 128
    wf = np.ascontiguousarray(w.reshape(N // 16, 16, KB, 4, 16).transpose(0, 2, 3, 1, 4)).reshape(-1)
    sf = np.ascontiguousarray(
        s.reshape(N // 16, 16, KB // 4, 4, 4).transpose(0, 2, 4, 1, 3)).reshape(-1)
    return wf, sf


def test_fp4_reference_matches_definition():
    rng = np.random.default_rng(1)
    N, K = 32, 1024
    KB = K // 128
    w = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    s = rng.integers(0, 256, size=(N, K // 32), dtype=np.uint8)
    wf, sf = frag_fp4_layout_ref(w, s)
    for idx in range(wf.size):
        blk, rem = divmod(idx, 1024)
        lane, b = divmod(rem, 16)
        n16, kb = divmod(blk, KB)
        assert wf[idx] == w[16 * n16 + lane % 16, 64 * kb + 16 * (lane // 16) + b], idx
    for idx in range(sf.size):
        blk, rem = divmod(idx, 256)
        lane, j = divmod(rem, 4)
        n16, q = divmod(blk, KB // 4)
        assert sf[idx] == s[16 * n16 + lane % 16, 16 * q + 4 * j + lane // 16], idx


def test_fp4_weight_to_frag_rejects_bad_shapes():
    from sglang_lite_amd import _lib

    lib = _lib.load()
    assert lib.sgl_fp4_weight_to_frag(None, None, 24, 512, None, None, None) != 0  # N % 16
    assert lib.sgl_fp4_weight_to_frag(None, None, 16, 384, None, None, None) != 0  # K % 512
    assert b"multiple" in lib.sgl_last_error()
    assert lib.sgl_fp4_weight_to_frag(None, None, 16, 512, None, None, None) != 0  # null
    assert lib.sgl_fp4_weight_to_frag(None, None, 0, 512, None, None, None) == 0
