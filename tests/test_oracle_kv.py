"""Pins the oracle's KV layouts on the CPU against independent decodes.

Layout B (a [T, 576] latent+rope row packed to 656 bytes) has no producer in
the reference, so its bytes are rebuilt here from torch's own ops --
``per_token_cast_to_fp8``'s formula (deep_gemm_sm120/utils/math.py:25-37)
written with torch tensors, torch's bf16 storage for the rope bytes, and
numpy's explicit little-endian float32 for the scales -- and compared with
``oracle.kv.pack_layout_b``; the decode is checked by a round trip.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import kv as OK
from oracle import quant as Q


def _torch_per_token(x: torch.Tensor):
    """utils/math.py:25-37 with torch ops: amax over 1x128 groups clamped at
    1e-4, sf = amax / 448, q = e4m3(x * (1 / sf))."""
    m, n = x.shape
    v = x.float().view(m, n // 128, 128)
    amax = v.abs().float().amax(dim=2).clamp(1e-4)
    sf = amax / 448.0
    q = (v * (1.0 / sf.unsqueeze(2))).to(torch.float8_e4m3fn).view(m, n)
    return q, sf


def _case(T=300, seed=21):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(T, 512, generator=g).to(torch.bfloat16)
    rope = torch.randn(T, 64, generator=g).to(torch.bfloat16)
    lat[5, :128] = 0  # an all-zero group: sf = fp32(1e-4) / 448
    lat[6, 128:256] *= 1000  # a group with a large amax
    return lat, rope


def test_layout_b_bytes_decode_field_by_field():
    lat, rope = _case()
    T = lat.shape[0]
    rows = OK.pack_layout_b(lat.float().numpy(), rope.view(torch.uint8).numpy())
    assert rows.shape == (T, 656) and rows.dtype == np.uint8
    q, sf = _torch_per_token(lat)
    # [0:512): the e4m3 codes of the latent, group g at bytes [128 g, 128 g + 128)
    np.testing.assert_array_equal(rows[:, :512], q.view(torch.uint8).numpy())
    # [512:640): the 64 rope values' bf16 bytes verbatim, element j at 512 + 2 j (low byte first)
    rb = rope.view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    np.testing.assert_array_equal(rows[:, 512:640:2], (rb & 0xFF).astype(np.uint8))
    np.testing.assert_array_equal(rows[:, 513:640:2], (rb >> 8).astype(np.uint8))
    # [640:656): the four fp32 scales, little endian, group g at 640 + 4 g
    sb = sf.numpy().view(np.uint32).astype(np.int64)
    for g in range(4):
        for byte in range(4):
            np.testing.assert_array_equal(rows[:, 640 + 4 * g + byte],
                                          ((sb[:, g] >> (8 * byte)) & 0xFF).astype(np.uint8))
    assert sf[5, 0].item() == np.float32(np.float32(1e-4) / np.float32(448.0))
    assert not rows[5, :128].any()


def test_layout_b_round_trip_within_half_an_e4m3_step():
    """dequant_row_b(pack(x)): each latent value within half an e4m3 step of x
    (2^-4 relative, or half the subnormal step sf * 2^-10) plus the bf16
    rounding of the product (2^-8 relative); the rope part exact."""
    lat, rope = _case(T=512, seed=22)
    x = lat.float().numpy()
    rows = OK.pack_layout_b(x, rope.view(torch.uint8).numpy())
    deq = OK.dequant_row_b(rows)
    assert deq.shape == (512, 576)
    sf = np.ascontiguousarray(rows[:, 640:656]).view("<f4").reshape(512, 4)
    step = np.maximum(np.abs(x) * 2.0**-4, np.repeat(sf, 128, axis=1) * 2.0**-10)
    err = np.abs(deq[:, :512] - x)
    assert np.all(err <= step + np.abs(deq[:, :512]) * 2.0**-8)
    np.testing.assert_array_equal(deq[:, 512:], rope.float().numpy())


def test_layout_b_gather_equals_row_decode_with_minus_one_rows_zero():
    lat, rope = _case(T=64, seed=23)
    rows = OK.pack_layout_b(lat.float().numpy(), rope.view(torch.uint8).numpy())
    idx = np.array([[3, -1, 63, 0], [64, 7, 7, -1]], np.int32)
    out = OK.gather_dequant(rows, idx, "B")
    deq = OK.dequant_row_b(rows)
    np.testing.assert_array_equal(out[0, 0], deq[3])
    np.testing.assert_array_equal(out[0, 2], deq[63])
    np.testing.assert_array_equal(out[1, 1], deq[7])
    for q, i in ((0, 1), (1, 0), (1, 3)):  # -1 and past-the-end indices give zero rows
        assert not out[q, i].any()


def test_layout_a_round_trip_matches_qat_quant_dequant():
    """Layout A decode equals the reference's inplace quant-dequant
    (kernel.py:84-91) with the injected ue8m0 quantizer (mode 3), and the
    torch fallback's scales (mode 4) are powers of two bracketing amax/448."""
    g = torch.Generator().manual_seed(24)
    kv = torch.randn(200, 512, generator=g).to(torch.bfloat16)
    x = kv.float().numpy()
    rope = kv[:, 448:].contiguous().view(torch.uint8).numpy()
    rows3 = OK.pack_layout_a(x, rope, 3)
    qat, _ = Q.act_quant_inplace_tilelang(x[:, :448], 64, round_scale=True)
    np.testing.assert_array_equal(OK.dequant_row_a(rows3)[:, :448], qat)
    rows4 = OK.pack_layout_a(x, rope, 4)
    s = np.ldexp(1.0, rows4[:, 576:583].astype(np.int32) - 127)
    amax = np.abs(x[:, :448].reshape(200, 7, 64)).max(-1)
    assert np.all(s >= amax / 448 * (1 - 2.0**-20)) and np.all(s < 2 * amax / 448)
    assert not rows4[:, 583].any()
