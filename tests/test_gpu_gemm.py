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
