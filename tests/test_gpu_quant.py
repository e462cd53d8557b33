"""act_quant / weight quant on the GPU vs the oracle: e4m3 bytes and scales bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (assert_e4m3_equal_nan_signless, bf16_values, nan_inf_rows, to_dev_bf16, to_dev_f32,
                     u8)
from oracle import quant as Q

pytestmark = pytest.mark.gpu

MODES = [0, 1, 2, 3, 4]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("shape", [(1, 128), (37, 512), (256, 7168)])
def test_act_quant_bit_exact(gpu, mode, group, shape):
    from sglang_lite_amd import kernel as K

    M, Kd = shape
    if Kd % group:
        pytest.skip("shape not divisible")
    rng = np.random.default_rng(hash((mode, group, shape)) % 2**32)
    x = bf16_values(rng, shape) * np.exp(rng.uniform(-8, 8, (M, 1))).astype(np.float32)
    x = Q.bf16_round(x.astype(np.float32))
    if M > 3:
        x[1, :group] = 0.0                      # all-zero group
        x[2, :group] = np.float32(448.0 * 4)    # constant group
    q_ref, s_ref = Q.scale_mode_quant(x, mode, group)
    xd = to_dev_bf16(x, gpu)
    y, s = K.act_quant(xd, group, None, torch.float32, False, scale_mode=mode)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u8(y), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("group", [64, 128])
def test_act_quant_nan_and_inf_groups(gpu, mode, group):
    """Groups holding NaN or Inf: the scale (NaN, Inf or the mode's clamp of
    them) bit-exact, the e4m3 bytes exact up to the sign of NaN codes."""
    from sglang_lite_amd import kernel as K

    x = nan_inf_rows(np.random.default_rng(mode * 7 + group), 512)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        q_ref, s_ref = Q.scale_mode_quant(x, mode, group)
    y, s = K.act_quant(to_dev_bf16(x, gpu), group, None, torch.float32, False, scale_mode=mode)
    torch.cuda.synchronize()
    assert_e4m3_equal_nan_signless(u8(y), q_ref, f"act_quant mode {mode} group {group}")
    s_dev = s.cpu().numpy()
    both_nan = np.isnan(s_dev) & np.isnan(s_ref)
    np.testing.assert_array_equal(np.where(both_nan, 0, s_dev.view(np.uint32)),
                                  np.where(both_nan, 0, s_ref.view(np.uint32)))


def test_act_quant_default_formula_is_torch_per_token(gpu):
    from sglang_lite_amd import kernel as K

    rng = np.random.default_rng(7)
    x = bf16_values(rng, (64, 7168))
    q_ref, s_ref = Q.per_token_cast_to_fp8(x, False, 128)
    y, s = K.per_token_cast_to_fp8(to_dev_bf16(x, gpu), False)
    np.testing.assert_array_equal(u8(y), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    y2, s2 = K.act_quant(to_dev_bf16(x, gpu))  # scale_fmt None -> same formula by default
    np.testing.assert_array_equal(u8(y2), q_ref)
    np.testing.assert_array_equal(s2.cpu().numpy(), s_ref)


def test_act_quant_e8m0_scales_and_inplace(gpu):
    from sglang_lite_amd import kernel as K

    rng = np.random.default_rng(8)
    x = bf16_values(rng, (33, 448))
    q_ref, s_ref = Q.act_quant_tilelang(x, 64, round_scale=True)
    y, s = K.act_quant(to_dev_bf16(x, gpu), 64, "ue8m0", torch.float8_e8m0fnu, False,
                       scale_mode=3)
    assert s.dtype == torch.float8_e8m0fnu and s.shape == (33, 7)
    np.testing.assert_array_equal(u8(y), q_ref)
    np.testing.assert_array_equal(u8(s), Q.e8m0_byte(s_ref))
    # inplace QAT: bf16(fp32(e4m3) * s), written back into x (kernel.py:84-91,122-124)
    xd = to_dev_bf16(x, gpu)
    ret = K.act_quant(xd, 64, "ue8m0", torch.float32, True, scale_mode=3)
    assert ret is xd
    ref_inp, _ = Q.act_quant_inplace_tilelang(x, 64, round_scale=True)
    np.testing.assert_array_equal(xd.float().cpu().numpy().view(np.uint32), ref_inp.view(np.uint32))


@pytest.mark.parametrize("shape", [(128, 128), (300, 200), (4096, 7168)])
@pytest.mark.parametrize("ue8m0", [False, True])
def test_weight_quant_bit_exact(gpu, shape, ue8m0):
    from sglang_lite_amd import kernel as K

    rng = np.random.default_rng(shape[0] + ue8m0)
    w = (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    q_ref, s_ref = Q.per_block_cast_to_fp8(w, ue8m0)
    q, s = K.per_block_cast_to_fp8(to_dev_f32(w, gpu), ue8m0)
    np.testing.assert_array_equal(u8(q), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


def test_e8m0_to_f32(gpu):
    from sglang_lite_amd import kernel as K

    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e8m0fnu).float().numpy()
    got = K.e8m0_to_f32(codes.to(gpu).view(torch.float8_e8m0fnu)).cpu().numpy()
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.all(np.isnan(got[~ok]))


def test_hardware_conversions_match_software_rules_exhaustively(gpu):
    """v_cvt_pk_fp8_f32 / v_cvt_pk_bf16_f32 (+ NaN fix-up), used by the GEMM
    epilogues and the quant kernels, equal the bit-level rounding rules of
    f32_to_e4m3 / f32_to_bf16 for all 2^32 fp32 inputs."""
    from sglang_lite_amd import _lib

    counts = torch.zeros(5, dtype=torch.int64, device=gpu)
    _lib.call("sgl_check_conversions", counts.data_ptr(), _lib.stream_of(counts))
    torch.cuda.synchronize()
    assert counts.cpu().tolist() == [0, 0, 0, 0, 0]
