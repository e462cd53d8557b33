"""FP8 x MXFP4 on the GPU vs the oracle: the dense ``fp4_gemm``, the FP4 -> FP8
weight repack (bit-exact) and the MoE layer with FP4 routed experts."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (assert_gemm_close, bf16_values, f32, to_dev_bf16, to_dev_f32, to_dev_fp8,
                     u8)
from oracle import fp4 as F4
from oracle import moe as OM
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def dev_fp4(bp: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bp, dtype=np.uint8)).to(dev).view(torch.float4_e2m1fn_x2)


def dev_e8m0(sb: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(sb, dtype=np.uint8)).to(dev).view(torch.float8_e8m0fnu)


def _operands(rng, M, N, K, pow2):
    a = bf16_values(rng, (M, K))
    aq, sa = Q.per_token_cast_to_fp8(a, pow2, 128)
    bp, sb = F4.make_fp4_weight(rng, N, K)
    return aq, sa, bp, sb


def _gemm(gpu, aq, sa, bp, sb, out_dtype=torch.bfloat16, **kw):
    from sglang_lite_amd import kernel as K_

    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(out_dtype)
        c = K_.fp4_gemm(to_dev_fp8(aq, gpu), sa if isinstance(sa, torch.Tensor) else to_dev_f32(sa, gpu),
                        dev_fp4(bp, gpu), sb if isinstance(sb, torch.Tensor) else dev_e8m0(sb, gpu), **kw)
    finally:
        torch.set_default_dtype(prev)
    return c


# skinny (M <= 64), 64 x 128 tiles (M <= 2048) and 128 x 256 tiles
@pytest.mark.parametrize("M,N,K", [(1, 256, 256), (16, 512, 1024), (33, 272, 1536), (64, 768, 1024),
                                    (65, 640, 512), (300, 1040, 768), (128, 4096, 7168),
                                    (200, 1040, 512), (1000, 1040, 512), (2100, 512, 512),
                                    (2100, 1040, 512)])
@pytest.mark.parametrize("pow2", [False, True])
def test_fp4_gemm_matches_oracle(gpu, M, N, K, pow2):
    print(f"fp4_gemm M={M} N={N} K={K} pow2={pow2}", flush=True)
    rng = np.random.default_rng(M * 7 + N + pow2)
    aq, sa, bp, sb = _operands(rng, M, N, K, pow2)
    ref = F4.fp4_gemm(aq, sa, bp, sb, out_bf16=False)
    c = _gemm(gpu, aq, sa, bp, sb, a_scale_pow2=pow2)
    assert c.dtype == torch.bfloat16 and c.shape == (M, N)
    assert_gemm_close(f32(c), ref, f"fp4_gemm {M}x{N}x{K} pow2={pow2}")


@pytest.mark.parametrize("M", [8, 40, 200, 600, 2100])
def test_fp4_gemm_fp32_out_tracks_the_blocked_structure(gpu, M):
    """fp32 output against the reference kernel's own accumulation order
    (kernel.py:485-513) with e8m0 activation scales (the live scale_dtype):
    a wrong scale index or K block would be off by O(1)."""
    rng = np.random.default_rng(20 + M)
    N, K = 256, 1024
    aq, sa, bp, sb = _operands(rng, M, N, K, True)
    ref = F4.fp4_gemm_blocked(aq, sa, bp, sb)
    sa_e8m0 = dev_e8m0(Q.e8m0_byte(sa), gpu)
    c = _gemm(gpu, aq, sa_e8m0, bp, sb, out_dtype=torch.float32)
    assert c.dtype == torch.float32
    np.testing.assert_allclose(f32(c), ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    # the e8m0 bytes, read by the kernel itself, give what the same powers of
    # two given as fp32 give
    c32 = _gemm(gpu, aq, to_dev_f32(sa, gpu), bp, sb, out_dtype=torch.float32, a_scale_pow2=True)
    assert torch.equal(c, c32)


def test_fp4_gemm_accepts_fp32_weight_scales_and_3d_input(gpu):
    rng = np.random.default_rng(31)
    M, N, K = 48, 384, 512
    aq, sa, bp, sb = _operands(rng, M, N, K, False)
    ref = F4.fp4_gemm(aq, sa, bp, sb, out_bf16=False)
    sb32 = to_dev_f32(F4.e8m0_to_f32(sb), gpu)
    from sglang_lite_amd import kernel as K_

    prev = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.bfloat16)
        a3 = to_dev_fp8(aq, gpu).view(2, M // 2, K)
        s3 = to_dev_f32(sa, gpu).view(2, M // 2, K // 128)
        c = K_.fp4_gemm(a3, s3, dev_fp4(bp, gpu), sb32)
    finally:
        torch.set_default_dtype(prev)
    assert c.shape == (2, M // 2, N)
    assert_gemm_close(f32(c).reshape(M, N), ref, "fp4_gemm 3-d")


def test_fp4_gemm_rejects_bad_shapes(gpu):
    from sglang_lite_amd import kernel as K_

    a = torch.zeros(4, 384, dtype=torch.float8_e4m3fn, device=gpu)
    s = torch.ones(4, 3, dtype=torch.float32, device=gpu)
    b = torch.zeros(64, 192, dtype=torch.uint8, device=gpu)
    sb = torch.full((64, 12), 127, dtype=torch.uint8, device=gpu).view(torch.float8_e8m0fnu)
    with pytest.raises(ValueError, match="multiple of 256"):
        K_.fp4_gemm(a, s, b, sb)


@pytest.mark.parametrize("N,K,spread", [(128, 128, 6), (256, 512, 6), (384, 256, 12)])
def test_fp4_to_fp8_repack_bit_exact(gpu, N, K, spread):
    """convert.py:17-52 on the device: e4m3 bytes and e8m0 block scales equal
    the oracle's; with a spread above 2^6 the small-scale elements round."""
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(N + K + spread)
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    bp = F4.pack_fp4(codes)
    sb = rng.integers(120 - spread, 121, (N, K // 32)).astype(np.uint8)
    q_ref, s_ref = F4.fp4_to_fp8_repack(bp, sb)
    q, s = K_.cast_e2m1fn_to_e4m3fn(dev_fp4(bp, gpu).view(torch.int8), dev_e8m0(sb, gpu))
    assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float8_e8m0fnu
    np.testing.assert_array_equal(u8(s), s_ref)
    np.testing.assert_array_equal(u8(q), q_ref)


def test_fp4_to_fp8_repack_reference_bytes(gpu):
    """The repack on the device against the reference converter's bytes
    (tests/golden/ref_fp4_repack.npz from convert.py cast_e2m1fn_to_e4m3fn):
    an all-0x88 block (nibble code 8 -> e4m3 0x00), a code 8 / code 0 mix and
    uniform codes with scales spread over 2^10."""
    import os

    from sglang_lite_amd import kernel as K_

    d = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "ref_fp4_repack.npz"))
    q, s = K_.cast_e2m1fn_to_e4m3fn(dev_fp4(d["bp"], gpu).view(torch.int8), dev_e8m0(d["sb"], gpu))
    np.testing.assert_array_equal(u8(q), d["q"])
    np.testing.assert_array_equal(u8(s), d["s"])


def test_repacked_fp8_gemm_equals_fp4_gemm(gpu):
    """The lossless repack feeds the FP8 path: fp8_gemm on the repacked weight
    and fp4_gemm on the original agree to fp32 summation order."""
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(41)
    M, N, K = 96, 256, 1024
    aq, sa, bp, sb = _operands(rng, M, N, K, False)
    q, s = K_.cast_e2m1fn_to_e4m3fn(dev_fp4(bp, gpu), dev_e8m0(sb, gpu))
    c8 = K_.fp8_gemm(to_dev_fp8(aq, gpu), to_dev_f32(sa, gpu), q, s)
    c4 = _gemm(gpu, aq, sa, bp, sb, out_dtype=torch.float32)
    ref = F4.fp4_gemm(aq, sa, bp, sb, out_bf16=False)
    np.testing.assert_allclose(f32(c8), f32(c4), rtol=1e-4, atol=1e-4 * np.abs(ref).max())


def fp4_table(experts, shared, dev):
    from sglang_lite_amd import moe as M

    def ent4(e):
        return (dev_fp4(e["w1"], dev), dev_fp4(e["w3"], dev), dev_fp4(e["w2"], dev),
                dev_e8m0(e["s1"], dev), dev_e8m0(e["s3"], dev), dev_e8m0(e["s2"], dev))

    def ent8(e):
        return (to_dev_fp8(e["w1"], dev), to_dev_fp8(e["w3"], dev), to_dev_fp8(e["w2"], dev),
                to_dev_f32(e["s1"], dev), to_dev_f32(e["s3"], dev), to_dev_f32(e["s2"], dev))

    return M.ExpertTable.build([ent4(e) for e in experts], ent8(shared) if shared else None)


@pytest.mark.parametrize("T,H,I,E,k,shared,lim,mode", [
    (32, 256, 256, 8, 2, True, 0.0, 0),
    (100, 512, 256, 16, 4, True, 10.0, 1),
    (64, 1024, 512, 32, 8, True, 0.0, 3),
    (7, 512, 256, 5, 3, False, 0.5, 2),
    (512, 512, 512, 8, 2, True, 0.0, 3),   # >= 64 rows per expert: 128-row tiles
    (600, 256, 512, 4, 2, False, 0.0, 0),
])
def test_moe_forward_fp4_experts_matches_oracle(gpu, T, H, I, E, k, shared, lim, mode):
    """The reference's live expert format (model.py:623-626): FP4 routed
    experts, FP8 shared expert, one act_quant per projection."""
    from sglang_lite_amd import _lib
    from sglang_lite_amd import moe as M

    print(f"moe fp4 T={T} H={H} I={I} E={E} k={k} mode={mode}", flush=True)
    rng = np.random.default_rng(T * H + E + mode)
    x = bf16_values(rng, (T, H))
    logits = (rng.standard_normal((T, E)) * 2.0).astype(np.float32)
    w, ids = OM.route_topk(logits, k)
    experts = [OM.make_fp4_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I) if shared else None
    table = fp4_table(experts, sh, gpu)
    assert table.fmt & ~_lib.EXPERT_POW2_SCALES == _lib.EXPERT_FP4_E2M1
    y = M.moe_forward(to_dev_bf16(x, gpu), torch.from_numpy(ids).to(gpu), to_dev_f32(w, gpu), table,
                      swiglu_limit=lim, scale_mode=mode)
    y_ref = OM.moe_forward(x, ids, w, experts, sh, swiglu_limit=lim, mode=mode)
    assert_gemm_close(f32(y), y_ref, f"moe fp4 T={T} H={H} I={I} E={E} k={k} mode={mode}")


@pytest.mark.parametrize("mode", [0, 3])
def test_moe_fp4_group_sizes_at_block_edges(gpu, mode):
    """FP4 decode tiles (32 rows) compute only the 16-row blocks a group
    fills: group sizes 0, 1, 15, 16, 17, 31, 32, 33, 47 ... against the oracle."""
    from sglang_lite_amd import moe as M
    from helpers import EDGE_COUNTS_SHORT, ids_with_counts

    rng = np.random.default_rng(1234 + mode)
    H, I, E, k = 512, 256, len(EDGE_COUNTS_SHORT), 2
    ids = ids_with_counts(rng, EDGE_COUNTS_SHORT, k)
    T = ids.shape[0]
    print(f"moe fp4 block edges T={T} E={E} mode={mode}", flush=True)
    x = bf16_values(rng, (T, H))
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    experts = [OM.make_fp4_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    table = fp4_table(experts, sh, gpu)
    y = M.moe_forward(to_dev_bf16(x, gpu), torch.from_numpy(ids).to(gpu), to_dev_f32(w, gpu), table,
                      scale_mode=mode)
    y_ref = OM.moe_forward(x, ids, w, experts, sh, mode=mode)
    assert_gemm_close(f32(y), y_ref, f"moe fp4 block edges mode={mode}")


def test_moe_fp4_stages_match_oracle(gpu):
    """gate_up / down with FP4 routed experts, stage by stage: the routed and
    the shared rows of h, and the expert outputs."""
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    rng = np.random.default_rng(77)
    T, H, I, E, k = 48, 512, 256, 8, 2
    x = bf16_values(rng, (T, H))
    w, ids = OM.route_topk((rng.standard_normal((T, E)) * 2.0).astype(np.float32), k)
    experts = [OM.make_fp4_expert(rng, H, I) for _ in range(E)]
    sh = OM.make_expert(rng, H, I)
    table = fp4_table(experts, sh, gpu)
    xq, xs = K.act_quant(to_dev_bf16(x, gpu))
    idd = torch.from_numpy(ids).to(gpu)
    counts, offsets, sorted_slot, _ = M.permute(idd, E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, to_dev_f32(w, gpu).reshape(-1), table, k)
    out = M.down(hq, hs, offsets, sorted_slot, table, T, k)
    torch.cuda.synchronize()
    perm = OM.permute(ids, E)
    hq_n, hs_n, out_n = u8(hq), f32(hs), f32(out)
    for e in range(E):
        rows = perm["sorted_slot"][perm["offsets"][e]:perm["offsets"][e + 1]]
        if rows.size == 0:
            continue
        tok, top = rows // k, rows % k
        tr = {}
        ref_out = OM.expert_forward(x[tok], experts[e], w[tok, top][:, None], trace=tr)
        p0, p1 = perm["offsets"][e], perm["offsets"][e + 1]
        assert_gemm_close(Q.dequant_rows(hq_n[p0:p1], hs_n[p0:p1]), Q.dequant_rows(tr["hq"], tr["hs"]),
                          f"h expert {e}")
        assert_gemm_close(out_n[tok, top], ref_out, f"out expert {e}")
    tr = {}
    ref_sh = OM.expert_forward(x, sh, None, trace=tr)
    p0 = T * k
    assert_gemm_close(Q.dequant_rows(hq_n[p0:], hs_n[p0:]), Q.dequant_rows(tr["hq"], tr["hs"]), "h shared")
    assert_gemm_close(out_n[:, k], ref_sh, "shared")
