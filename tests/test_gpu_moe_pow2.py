"""FP8 experts whose block scales are powers of two (the float8_e8m0fnu scales
of deepseek_infer/model.py:138-142) with power-of-two activation scales
(scale_fmt "ue8m0", model.py:777-778): the grouped GEMMs apply both scales as
e8m0 exponents inside the MFMA.  The layer, and each GEMM on the device's own
inputs, against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (assert_gemm_close, assert_layer_close, assert_requant_close, bf16_values,
                     f32, to_dev_bf16, to_dev_f32, u8)
from oracle import moe as OM
from test_gpu_moe import logits_without_near_ties, table_from, zipf_logits

pytestmark = pytest.mark.gpu


def _case(rng, T, H, I, E, k, zipf):
    x = bf16_values(rng, (T, H))
    logits = zipf_logits(rng, T, E) if zipf else logits_without_near_ties(rng, T, E, k)
    w, ids = OM.route_topk(logits, k)
    experts = [OM.make_expert(rng, H, I, ue8m0=True) for _ in range(E)]
    sh = OM.make_expert(rng, H, I, ue8m0=True)
    return x, w, ids, experts, sh


@pytest.mark.parametrize("T,H,I,E,k,lim,zipf,mode", [
    # >= 64 rows per expert: the pipelined kernels, five / four K stages, a
    # partial last column tile in down, skewed routing
    (300, 640, 512, 12, 3, 7.0, True, 3),
    (300, 640, 512, 12, 3, 0.0, False, 1),
    # fewer rows per expert: the other kernels promote in fp32 (exact for
    # these scales too)
    (40, 512, 256, 16, 2, 0.0, False, 3),
])
def test_moe_forward_pow2_scales(gpu, T, H, I, E, k, lim, zipf, mode):
    from sglang_lite_amd import _lib
    from sglang_lite_amd import moe as M

    print(f"pow2 layer T={T} H={H} I={I} E={E} k={k} mode={mode}", flush=True)
    rng = np.random.default_rng(T + H + mode)
    x, w, ids, experts, sh = _case(rng, T, H, I, E, k, zipf)
    table = table_from(experts, sh, gpu)
    assert table.fmt == _lib.EXPERT_FP8_BLOCK128 | _lib.EXPERT_POW2_SCALES
    y = M.moe_forward(to_dev_bf16(x, gpu), torch.from_numpy(ids).to(gpu), to_dev_f32(w, gpu), table,
                      swiglu_limit=lim, scale_mode=mode)
    y_ref = OM.moe_forward(x, ids, w, experts, sh, swiglu_limit=lim, mode=mode)
    assert_layer_close(f32(y), y_ref, f"pow2 layer T={T} mode={mode}")


def test_pow2_stages_at_expert_shapes(gpu):
    """H = 4096, I = 2048 (32 and 16 K stages): each GEMM of each expert on
    the device's own inputs, within the GEMM tolerance of the oracle; the
    in-MFMA scaled results also within it of the fp32-promoted kernel's."""
    from sglang_lite_amd import _lib
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    T, H, I, E, k, mode = 512, 4096, 2048, 8, 2, 3
    print(f"pow2 stages T={T} H={H} I={I} E={E} k={k}", flush=True)
    rng = np.random.default_rng(4096)
    x, w, ids, experts, sh = _case(rng, T, H, I, E, k, False)
    table = table_from(experts, sh, gpu)
    assert table.fmt & _lib.EXPERT_POW2_SCALES
    xd = to_dev_bf16(x, gpu)
    idd = torch.from_numpy(ids).to(gpu)
    wd = to_dev_f32(w, gpu).reshape(-1)
    xq, xs = K.act_quant(xd, scale_mode=mode)
    counts, offsets, sorted_slot, _ = M.permute(idd, E)
    hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, wd, table, k, scale_mode=mode)
    out = M.down(hq, hs, offsets, sorted_slot, table, T, k, scale_mode=mode)
    # the same layer with the flag cleared: fp32 promotion of the same scales
    plain = M.ExpertTable(table.ptrs, table.E, table.H, table.I, table.has_shared, table.keep,
                          _lib.EXPERT_FP8_BLOCK128)
    hq_p, hs_p = M.gate_up(xq, xs, offsets, sorted_slot, wd, plain, k, scale_mode=mode)
    out_p = M.down(hq_p, hs_p, offsets, sorted_slot, plain, T, k, scale_mode=mode)
    torch.cuda.synchronize()
    xq_n, xs_n = u8(xq), f32(xs)
    hq_n, hs_n, out_n = u8(hq), f32(hs), f32(out)
    off = offsets.cpu().numpy()
    slots = sorted_slot.cpu().numpy()
    for e in range(E + 1):
        ex = sh if e == E else experts[e]
        if e == E:
            p0, p1 = int(off[E]), int(off[E]) + T
            tok, top, wr = np.arange(T), np.full(T, k), None
        else:
            p0, p1 = int(off[e]), int(off[e + 1])
            sl = slots[p0:p1]
            tok, top = sl // k, sl % k
            wr = w[tok, top][:, None]
        if p1 == p0:
            continue
        tr = {}
        OM.expert_forward(x[tok], ex, wr, mode=mode, trace=tr)
        # the device's x quant is the oracle's (bit-exact), so h is compared
        # with the oracle's h of the same rows
        np.testing.assert_array_equal(xq_n[tok], tr["xq"])
        assert_requant_close(hq_n[p0:p1], hs_n[p0:p1], tr["hq"], tr["hs"], f"h expert {e}",
                             pow2=True)
        ref = OM.fp8_gemm(hq_n[p0:p1], hs_n[p0:p1], ex["w2"], ex["s2"])
        assert_gemm_close(out_n[tok, top], ref, f"down expert {e} on the device's h")
    # the two paths' h agree to rounding; their down rows to the layer bound
    assert_requant_close(hq_n, hs_n, u8(hq_p), f32(hs_p), "h in-MFMA vs fp32-promoted", pow2=True)
    P = T * (k + 1)
    assert_layer_close(out_n.reshape(P, H), f32(out_p).reshape(P, H), "in-MFMA vs fp32-promoted rows")
