"""Dense block-scaled FP8 GEMM on the GPU vs the dequantize-to-fp32 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_gemm_close, bf16_values, f32, to_dev_f32, to_dev_fp8, u8
from oracle import moe as OM
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _operands(rng, M, N, K):
    a = bf16_values(rng, (M, K))
    aq, sa = Q.per_token_cast_to_fp8(a, False, 128)
    b = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    bq, sb = Q.per_block_cast_to_fp8(b)
    return aq, sa, bq, sb


@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (16, 512, 1024), (77, 384, 768),
                                    (16, 4096, 7168), (33, 272, 1536), (64, 768, 1024), (65, 640, 896),
                                    (128, 4096, 7168),
                                    (129, 512, 2048), (300, 1040, 512),
                                    # ragged last N tile on the 32 x 64 (M <= 128), 32 x 128
                                    # (M <= 256), 128 x 128 (M <= 2048) and 128 x 256 tiles
                                    (100, 1040, 512), (200, 1040, 512), (1000, 1040, 512),
                                    (2304, 1040, 512)])
def test_fp8_gemm_matches_oracle(gpu, M, N, K):
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(M * 7 + N)
    aq, sa, bq, sb = _operands(rng, M, N, K)
    ref = OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False)
    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.bfloat16)
        c = K_.fp8_gemm(to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), to_dev_fp8(bq, gpu),
                        to_dev_f32(sb, gpu))
    finally:
        torch.set_default_dtype(prev)
    assert c.dtype == torch.bfloat16 and c.shape == (M, N)
    assert_gemm_close(f32(c), ref, f"fp8_gemm {M}x{N}x{K}")


def test_fp8_gemm_fp32_out_tracks_promotion_structure(gpu):
    """fp32 output vs the exact per-128-K promotion emulation of kernel.py:238-250."""
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(11)
    M, N, K = 64, 256, 1024
    aq, sa, bq, sb = _operands(rng, M, N, K)
    ref = OM.fp8_gemm_promoted(aq, sa, bq, sb)
    c = K_.fp8_gemm(to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), to_dev_fp8(bq, gpu),
                    to_dev_f32(sb, gpu))
    assert c.dtype == torch.float32
    got = f32(c)
    # The MFMA's 128-deep fp8 partial is not an IEEE-exact fp32 sum (observed
    # ~1e-5 relative to the output scale); a wrong scale index or block would
    # be off by O(1).
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


def test_fp8_gemm_e8m0_scales(gpu):
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(12)
    M, N, K = 48, 256, 512
    a = bf16_values(rng, (M, K))
    aq, sa = Q.per_token_cast_to_fp8(a, True, 128)
    b = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    bq, sb = Q.per_block_cast_to_fp8(b, True)
    ref = OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False)
    sa_e = torch.from_numpy(Q.e8m0_byte(sa)).view(torch.float8_e8m0fnu).to(gpu)
    sb_e = torch.from_numpy(Q.e8m0_byte(sb)).view(torch.float8_e8m0fnu).to(gpu)
    c = K_.fp8_gemm(to_dev_fp8(aq, gpu), sa_e, to_dev_fp8(bq, gpu), sb_e)
    assert_gemm_close(f32(c), ref, "fp8_gemm e8m0")


@pytest.mark.parametrize("M,N,K", [(16, 256, 1024), (40, 4096, 7168), (128, 384, 1024),
                                   (300, 256, 1024), (1024, 512, 2048), (2100, 512, 1024)])
def test_fp8_gemm_reads_e8m0_activation_scales_as_bytes(gpu, M, N, K):
    """The live format (model.py:138-142,777-778: act_quant with ue8m0 e8m0
    scales, e8m0 weight scales) without a conversion launch.  Every dense
    kernel (skinny M <= 16, split-K 16 < M <= 64, 32 x 64 / 32 x 128 /
    64 x 128 / 128 x 128 tiles, 256 x 256 tiles above M = 2048) reads the
    activation scale bytes itself.  With fp32 weight scales the split-K and
    tiled kernels put the row scale's exponent into the MFMA and promote by
    the weight scale alone: the output equals the all-fp32 call bit for bit
    (a power-of-two scale inside the MFMA rounds as the promotion does).
    With e8m0 weight scales too, the tiled kernels apply both inside the
    MFMA (no promotion; a different rounding of the same sum), within the
    GEMM bound of the oracle."""
    from sglang_lite_amd import kernel as K_

    print(f"fp8_gemm e8m0 activations M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + 7 * N)
    a = bf16_values(rng, (M, K))
    aq, sa = Q.per_token_cast_to_fp8(a, True, 128)
    b = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    bq, sb = Q.per_block_cast_to_fp8(b, True)
    sa_e = torch.from_numpy(Q.e8m0_byte(sa)).view(torch.float8_e8m0fnu).to(gpu)
    sb_e = torch.from_numpy(Q.e8m0_byte(sb)).view(torch.float8_e8m0fnu).to(gpu)
    aqd, bqd = to_dev_fp8(aq, gpu), to_dev_fp8(bq, gpu)
    sb32 = torch.from_numpy(sb).to(gpu)
    c8 = K_.fp8_gemm(aqd, sa_e, bqd, sb32)
    c32 = K_.fp8_gemm(aqd, torch.from_numpy(sa).to(gpu), bqd, sb32)
    c88 = K_.fp8_gemm(aqd, sa_e, bqd, sb_e)
    torch.cuda.synchronize()
    assert torch.equal(c8, c32)
    ref = OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False)
    assert_gemm_close(f32(c8), ref, f"fp8_gemm e8m0 a {M}")
    assert_gemm_close(f32(c88), ref, f"fp8_gemm e8m0 a and b {M}")


def test_fp8_gemm_end_to_end_from_bf16(gpu):
    """act_quant -> fp8_gemm (model.py:116-118 linear()) against the oracle of
    the same pipeline, at the dense config's K and N."""
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(13)
    M, N, K = 16, 4096, 7168
    x = bf16_values(rng, (M, K))
    b = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    bq, sb = Q.per_block_cast_to_fp8(b)
    aq, sa = Q.per_token_cast_to_fp8(x, False, 128)
    ref = OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False)
    xq, xs = K_.act_quant(torch.from_numpy(x).to(torch.bfloat16).to(gpu))
    np.testing.assert_array_equal(u8(xq), aq)
    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.bfloat16)
        c = K_.fp8_gemm(xq, xs, to_dev_fp8(bq, gpu), to_dev_f32(sb, gpu))
    finally:
        torch.set_default_dtype(prev)
    assert_gemm_close(f32(c), ref, "linear")


# The split-K kernel (16 < M <= 64, N % 128 == 0; 32-row tiles up to M = 32,
# 64-row tiles above): N/128 column tiles x S K ranges of KS <= 8 blocks, the
# partials summed in split order by a second kernel.  Shapes beside it take
# the unsplit kernels.
@pytest.mark.parametrize("M,N,K", [
    (33, 1024, 1152),   # 8 tiles, KB = 9: S = 5, ragged last split; 31 rows past M
    (48, 4096, 896),    # 32 tiles, one block per split
    (64, 384, 2048),    # 3 tiles
    (40, 4096, 7168),   # the dense config's N and K: 8 splits of 7 blocks
    (64, 2048, 4096),
    (32, 1024, 1152),   # 32-row tiles
    (17, 4096, 7168),   # 32-row tiles, 15 rows past M, the dense config's N and K
    (16, 1024, 1152),   # M <= 16 and M > 64: the unsplit kernels
    (65, 1024, 1152),
])
def test_fp8_gemm_splitk_matches_oracle(gpu, M, N, K):
    from sglang_lite_amd import kernel as K_

    print(f"splitk {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    aq, sa, bq, sb = _operands(rng, M, N, K)
    ref = OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False)
    args = (to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), to_dev_fp8(bq, gpu), to_dev_f32(sb, gpu))
    c32 = K_.fp8_gemm(*args)  # default dtype fp32: fp32 output
    assert c32.dtype == torch.float32
    np.testing.assert_allclose(f32(c32), OM.fp8_gemm_promoted(aq, sa, bq, sb), rtol=1e-4,
                               atol=1e-4 * np.abs(ref).max())
    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.bfloat16)
        c = K_.fp8_gemm(*args)
        c2 = K_.fp8_gemm(*args)
    finally:
        torch.set_default_dtype(prev)
    assert_gemm_close(f32(c), ref, f"fp8_gemm split-K {M}x{N}x{K}")
    # the partials are summed in split order: the same bytes on every call
    np.testing.assert_array_equal(u8(c), u8(c2))


def test_fp8_gemm_splitk_e8m0_weight_scales(gpu):
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(21)
    M, N, K = 50, 2048, 7168
    a = bf16_values(rng, (M, K))
    aq, sa = Q.per_token_cast_to_fp8(a, True, 128)
    bq, sb = Q.per_block_cast_to_fp8(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02),
                                     True)
    ref = OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False)
    sb_e = torch.from_numpy(Q.e8m0_byte(sb)).view(torch.float8_e8m0fnu).to(gpu)
    c = K_.fp8_gemm(to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), to_dev_fp8(bq, gpu), sb_e)
    assert_gemm_close(f32(c), ref, "fp8_gemm split-K e8m0")


def test_fp8_gemm_splitk_concurrent_streams(gpu):
    """Each call's split-K partials live in a workspace the shim allocates on
    the calling stream, so GEMMs overlapping on two streams stay exact."""
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(22)
    M, N, K = 48, 4096, 7168
    ops = [_operands(rng, M, N, K) for _ in range(2)]
    dev_ops = [(to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), to_dev_fp8(bq, gpu), to_dev_f32(sb, gpu))
               for aq, sa, bq, sb in ops]
    refs = [OM.fp8_gemm(*o, out_bf16=False) for o in ops]
    eager = [K_.fp8_gemm(*d) for d in dev_ops]
    torch.cuda.synchronize()
    for e, r in zip(eager, refs):
        assert_gemm_close(f32(e), r, "split-K eager")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.empty(M, N, dtype=torch.float32, device=gpu) for _ in range(2)]
    for _ in range(3):
        for st, d, o in zip(streams, dev_ops, outs):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                for _ in range(4):
                    K_.fp8_gemm(*d, out=o)
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            np.testing.assert_array_equal(f32(o).view(np.uint32), f32(e).view(np.uint32))


@pytest.mark.parametrize("M", [17, 40, 64])
def test_fp8_gemm_captured_equals_eager_bit_for_bit(gpu, M):
    """The split decision is a function of the shape and the workspace comes
    from torch (the graph's pool inside a capture), so a GEMM captured first
    on a fresh stream -- no eager call before it -- replays the eager bytes,
    with eager GEMMs of other sizes (their own workspaces) between replays."""
    from sglang_lite_amd import kernel as K_

    print(f"captured split-K M={M}", flush=True)
    rng = np.random.default_rng(24 + M)
    N, K = 4096, 7168
    ops = _operands(rng, M, N, K)
    other = _operands(rng, 64 if M != 64 else 33, N, K)
    d = (to_dev_fp8(ops[0], gpu), to_dev_f32(ops[1], gpu), to_dev_fp8(ops[2], gpu), to_dev_f32(ops[3], gpu))
    d2 = (to_dev_fp8(other[0], gpu), to_dev_f32(other[1], gpu), to_dev_fp8(other[2], gpu),
          to_dev_f32(other[3], gpu))
    g = torch.cuda.CUDAGraph()
    gout = torch.empty(M, N, dtype=torch.float32, device=gpu)
    fresh = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=fresh):
        K_.fp8_gemm(*d, out=gout)
    eager = K_.fp8_gemm(*d)
    eager2 = K_.fp8_gemm(*d2)
    torch.cuda.synchronize()
    assert_gemm_close(f32(eager), OM.fp8_gemm(*ops, out_bf16=False), f"split-K M={M}")
    e_bits, e2_bits = f32(eager).view(np.uint32), f32(eager2).view(np.uint32)
    for _ in range(3):
        gout.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(f32(gout).view(np.uint32), e_bits)
        np.testing.assert_array_equal(f32(K_.fp8_gemm(*d2)).view(np.uint32), e2_bits)


def test_hbm_stream_copies_and_reads(gpu):
    """sgl_hbm_stream (the bandwidth measurement kernel): the copy is exact and
    the read leaves the XOR of each 1/2048 slice."""
    from sglang_lite_amd import _lib

    rng = np.random.default_rng(30)
    n = 2048 * 64 * 16  # 2 MiB
    host = rng.integers(0, 256, n, dtype=np.uint8)
    src = torch.from_numpy(host).to(gpu)
    dst = torch.zeros_like(src)
    sums = torch.zeros(2048, dtype=torch.int32, device=gpu)
    _lib.call("sgl_hbm_stream", src.data_ptr(), dst.data_ptr(), n, sums.data_ptr(), _lib.stream_of(src))
    _lib.call("sgl_hbm_stream", src.data_ptr(), None, n, sums.data_ptr(), _lib.stream_of(src))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dst.cpu().numpy(), host)
    words = host.view(np.uint32).reshape(2048, -1)
    np.testing.assert_array_equal(sums.cpu().numpy().view(np.uint32),
                                  np.bitwise_xor.reduce(words, axis=1))


def test_mfma_mix_measurement_kernel(gpu):
    """sgl_mfma_mix (the MFMA-rate measurement kernel) runs both instruction
    mixes on every CU and its per-thread sums are exact multiples of one
    round (the e4m3 operands have at most 4 significant bits, so every block
    partial and its promotion by 1, 1.25, 1.5 or 1.75 is exact in fp32)."""
    from sglang_lite_amd import _lib

    n = _lib.load().sgl_mfma_mix_threads()
    assert n > 0 and n % 256 == 0
    outs = {}
    for v in (0, 1):
        for it in (1, 2, 4):
            o = torch.empty(n, dtype=torch.float32, device=gpu)
            _lib.call("sgl_mfma_mix", v, o.data_ptr(), it, _lib.stream_of(o))
            outs[v, it] = f32(o)
    for v in (0, 1):
        assert np.all(np.isfinite(outs[v, 1])) and np.any(outs[v, 1] != 0)
        np.testing.assert_array_equal(outs[v, 2], 2 * outs[v, 1])
        np.testing.assert_array_equal(outs[v, 4], 4 * outs[v, 1])
    assert not np.array_equal(outs[0, 1], outs[1, 1])  # the promotion scales differ from 1


# The 256 x 256 tiles (M > 2048): a partial last M tile whose rows end inside
# a wavefront's 64 (3000 = 11 x 256 + 184), a last row tile of 8 rows
# (2056), ragged N (a 16-column last tile: chunks past N are not loaded),
# one 256-deep K range (two stages), and fp32 output against the exact
# per-128-K promotion emulation.
@pytest.mark.parametrize("M,N,K,f32_out", [(3000, 1040, 1024, True), (2056, 512, 256, True),
                                           (2304, 4096, 7168, False), (4100, 272, 640, False)])
def test_fp8_gemm_wide_tiles(gpu, M, N, K, f32_out):
    from sglang_lite_amd import kernel as K_

    print(f"wide {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K)
    aq, sa, bq, sb = _operands(rng, M, N, K)
    args = (to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), to_dev_fp8(bq, gpu), to_dev_f32(sb, gpu))
    if f32_out:
        c = K_.fp8_gemm(*args)
        assert c.dtype == torch.float32
        ref = OM.fp8_gemm_promoted(aq, sa, bq, sb)
        np.testing.assert_allclose(f32(c), ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    else:
        prev = torch.get_default_dtype()
        try:
            torch.set_default_dtype(torch.bfloat16)
            c = K_.fp8_gemm(*args)
        finally:
            torch.set_default_dtype(prev)
        assert_gemm_close(f32(c), OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False), f"wide {M}x{N}x{K}")


def test_fp8_gemm_wide_tiles_e8m0_weight_scales(gpu):
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(23)
    M, N, K = 2500, 768, 1536
    a = bf16_values(rng, (M, K))
    aq, sa = Q.per_token_cast_to_fp8(a, True, 128)
    bq, sb = Q.per_block_cast_to_fp8(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02),
                                     True)
    ref = OM.fp8_gemm(aq, sa, bq, sb, out_bf16=False)
    sb_e = torch.from_numpy(Q.e8m0_byte(sb)).view(torch.float8_e8m0fnu).to(gpu)
    c = K_.fp8_gemm(to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), to_dev_fp8(bq, gpu), sb_e)
    assert_gemm_close(f32(c), ref, "fp8_gemm wide e8m0")
