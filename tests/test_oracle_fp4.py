"""Pins of the FP4 oracle (``oracle/fp4.py``) against things other than itself:
the OCP e2m1 definition, torch's e8m0 cast, hand-worked vectors, integer
arithmetic, an element-by-element brute force and the repack's invariants."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp4 as F4
from oracle import quant as Q


def test_e2m1_table_is_the_ocp_definition():
    # sign bit 3, exponent bits 2..1 with bias 1, mantissa bit 0; exponent 0 is
    # subnormal (m * 2^-1).  Code 8 (the format's -0) is +0.0, as in the
    # converter's table (convert.py:11-14, FP4_TABLE[8] = 0.0) and
    # deep_gemm_sm120/utils/math.py `_dequantize_from_fp4_e2m1` (sign only on
    # nonzero magnitudes): the repack of code 8 must be the e4m3 byte 0x00.
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        mag = m * 0.5 if e == 0 else (1.0 + m / 2.0) * 2.0 ** (e - 1)
        want = -mag if s else mag
        got = float(F4.E2M1[c])
        assert got == want and np.signbit(got) == bool(s and mag != 0.0), (c, got, want)
    assert not np.signbit(F4.E2M1[8])
    assert sorted(set(np.abs(F4.E2M1).tolist())) == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_e8m0_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e8m0fnu).float().numpy()
    got = F4.e8m0_to_f32(codes)
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.isnan(got[255]) and np.isnan(ref[255])


def test_nibble_order_known_answer():
    # byte 0x21: low nibble 1 (0.5) is element 0, high nibble 2 (1.0) element 1
    # (convert.py:31-33 stacks low then high); 0xF8: code 8 (+0) then -6
    p = np.array([[0x21, 0xF8]], dtype=np.uint8)
    np.testing.assert_array_equal(F4.unpack_fp4(p), [[1, 2, 8, 15]])
    v = F4.e2m1_to_f32(F4.unpack_fp4(p))
    np.testing.assert_array_equal(v, np.array([[0.5, 1.0, 0.0, -6.0]], np.float32))
    assert not np.signbit(v[0, 2])
    rng = np.random.default_rng(0)
    c = rng.integers(0, 16, (5, 64), dtype=np.uint8)
    np.testing.assert_array_equal(F4.unpack_fp4(F4.pack_fp4(c)), c)


def _rand_case(rng, M, N, K, int_values=False):
    """Random e4m3 A with fp32 row scales, random e2m1 B with e8m0 scales."""
    if int_values:
        # e4m3 codes of the integers 1..8 and their negatives (exact products)
        vals = rng.integers(1, 9, (M, K)) * rng.choice([-1, 1], (M, K))
        aq = Q.f32_to_e4m3(vals.astype(np.float32))
    else:
        aq = rng.integers(0, 256, (M, K), dtype=np.uint8)
        aq[(aq & 0x7F) == 0x7F] = 0x3A  # no NaN codes
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    bp = F4.pack_fp4(codes)
    return aq, bp, codes


def test_fp4_gemm_integer_case_is_exact():
    """Unit scales and integer-valued operands: C is an integer matmul."""
    rng = np.random.default_rng(1)
    M, N, K = 9, 24, 256
    aq, bp, codes = _rand_case(rng, M, N, K, int_values=True)
    sa = np.ones((M, K // 128), np.float32)
    sb = np.full((N, K // 32), 127, np.uint8)
    a_int = Q.e4m3_to_f32(aq).astype(np.int64)
    b_twice = (2 * F4.e2m1_to_f32(codes)).astype(np.int64)  # e2m1 values are multiples of 1/2
    want = (a_int @ b_twice.T).astype(np.float64) / 2.0
    np.testing.assert_array_equal(F4.fp4_gemm(aq, sa, bp, sb, out_bf16=False), want.astype(np.float32))
    np.testing.assert_array_equal(F4.fp4_gemm_blocked(aq, sa, bp, sb), want.astype(np.float32))


def test_fp4_gemm_matches_elementwise_brute_force():
    """Distinct scales per (row, 128 K) and per (column, 32 K): a transposed
    operand, a wrong scale index or a swapped nibble changes the answer."""
    rng = np.random.default_rng(2)
    M, N, K = 3, 5, 256
    aq, bp, codes = _rand_case(rng, M, N, K)
    sa = rng.uniform(0.01, 2.0, (M, K // 128)).astype(np.float32)
    sb = rng.integers(118, 136, (N, K // 32)).astype(np.uint8)
    av = Q.e4m3_to_f32(aq).astype(np.float64)
    want = np.zeros((M, N))
    mag = np.zeros((M, N))  # sum of |terms|: bounds the fp32 roundings of the oracle
    for m in range(M):
        for n in range(N):
            acc = tot = 0.0
            for k in range(K):
                byte = int(bp[n, k // 2])
                code = (byte >> 4) if (k & 1) else (byte & 0xF)
                t = av[m, k] * float(sa[m, k // 128]) * float(F4.E2M1[code]) * 2.0 ** (int(sb[n, k // 32]) - 127)
                acc += t
                tot += abs(t)
            want[m, n] = acc
            mag[m, n] = tot
    got = F4.fp4_gemm(aq, sa, bp, sb, out_bf16=False)
    assert np.all(np.abs(got - want) <= 2.0**-22 * mag + 2.0**-24 * np.abs(want))
    blk = F4.fp4_gemm_blocked(aq, sa, bp, sb)
    assert np.all(np.abs(blk - want) <= 2.0**-20 * mag)


def test_fp4_gemm_blocked_and_dequant_agree_at_scale():
    rng = np.random.default_rng(3)
    M, N, K = 40, 64, 1024
    aq, bp, _ = _rand_case(rng, M, N, K)
    sa = rng.uniform(0.001, 0.1, (M, K // 128)).astype(np.float32)
    sb = rng.integers(115, 125, (N, K // 32)).astype(np.uint8)
    a = F4.fp4_gemm(aq, sa, bp, sb, out_bf16=False).astype(np.float64)
    b = F4.fp4_gemm_blocked(aq, sa, bp, sb).astype(np.float64)
    assert np.linalg.norm(a - b) / np.linalg.norm(a) < 1e-6


def test_repack_is_lossless_within_the_offset_range():
    """convert.py:17-52: when a block's scales span at most 2^6 the e4m3
    weight times its e8m0 block scale equals the FP4 weight exactly."""
    rng = np.random.default_rng(4)
    N, K = 256, 384
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    bp = F4.pack_fp4(codes)
    sb = rng.integers(110, 117, (N, K // 32)).astype(np.uint8)  # spread 2^6
    q, s = F4.fp4_to_fp8_repack(bp, sb)
    assert q.shape == (N, K) and s.shape == (N // 128, K // 128)
    deq8 = Q.dequant_blocks(q, F4.e8m0_to_f32(s), 128)
    np.testing.assert_array_equal(deq8, F4.dequant_fp4(bp, sb))
    # block scale = block max scale / 2^6
    blk_max = sb.reshape(N // 128, 128, K // 128, 4).max(axis=(1, 3))
    np.testing.assert_array_equal(s, blk_max - 6)
    # the largest scale's elements are e2m1 * 2^6 (at most 384 < 448)
    assert np.abs(Q.e4m3_to_f32(q)).max() <= 384.0


def test_repack_rounds_far_below_the_block_max():
    """A scale 2^20 below the block's maximum leaves e2m1 * 2^-14, below half
    the smallest e4m3 subnormal (2^-9): those elements round to zero."""
    N, K = 128, 128
    codes = np.full((N, K), 7, np.uint8)  # 6.0
    bp = F4.pack_fp4(codes)
    sb = np.full((N, K // 32), 100, np.uint8)
    sb[0, 0] = 120  # the block max
    q, s = F4.fp4_to_fp8_repack(bp, sb)
    assert int(s[0, 0]) == 114
    v = Q.e4m3_to_f32(q)
    assert np.all(v[0, :32] == 384.0)
    assert np.all(v[1:, :] == 0.0) and np.all(v[0, 32:] == 0.0)


def test_quant_fp4_weight_reconstructs_within_half_a_step():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    bp, sb = F4.quant_fp4_weight(w)
    deq = F4.dequant_fp4(bp, sb)
    scale = np.repeat(F4.e8m0_to_f32(sb), 32, axis=1)
    # nearest e2m1 value: error at most half the largest gap (1.0 between 4 and 6) times the scale
    assert np.all(np.abs(deq - w) <= 1.0 * scale + 1e-12)
    # the scale is the smallest power of two with amax / scale <= 6
    amax = np.abs(w.reshape(64, 8, 32)).max(-1)
    s = F4.e8m0_to_f32(sb)
    assert np.all(amax / s <= 6.0) and np.all(amax / (s / 2) > 6.0)


def test_repack_of_code_8_is_byte_zero():
    """Closed form: every element of an all-0x88 block (nibble code 8 = +0.0 in
    the converter's table) repacks to the e4m3 byte 0x00, whatever its scales."""
    N, K = 128, 256
    bp = np.full((N, K // 2), 0x88, np.uint8)
    sb = np.random.default_rng(7).integers(100, 130, (N, K // 32)).astype(np.uint8)
    q, s = F4.fp4_to_fp8_repack(bp, sb)
    assert np.all(q == 0x00)
    # each nibble code's byte under a unit offset: the e4m3 code of the table value
    codes = np.arange(16, dtype=np.uint8)
    want = Q.f32_to_e4m3(F4.E2M1[codes])
    assert want[8] == 0x00 and want[0] == 0x00


def test_repack_matches_reference_converter_bytes():
    """tests/golden/ref_fp4_repack.npz: convert.py cast_e2m1fn_to_e4m3fn's
    bytes (written by tests/golden/make_ref_fp4_repack.py) for uniform codes,
    an all-0x88 block and a code 8 / code 0 mix, scales spread over 2^10."""
    import os

    d = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "ref_fp4_repack.npz"))
    q, s = F4.fp4_to_fp8_repack(d["bp"], d["sb"])
    np.testing.assert_array_equal(q, d["q"])
    np.testing.assert_array_equal(s, d["s"])
    assert np.all(d["q"][:128, :128] == 0)
