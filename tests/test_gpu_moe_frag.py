"""Expert weights in the MFMA fragment layout (``ExpertTable(frag_layout=True)``).

* ``fp8_weight_to_frag`` against the layout's definition
  (``frag_layout_ref``, itself checked element by element in
  tests/test_frag_layout.py).
* The register-fed grouped GEMMs (gemm_rb_kernel: gate/up with the SwiGLU +
  1x128 requant epilogue, and down) against the LDS-staged kernels (the
  pipelined prefill kernel, the 32-row decode kernel), which the other MoE
  tests hold to the oracle.  They run the same arithmetic (the same MFMA
  fragments, the per-128-K fp32 promotion in the same order, the same
  epilogue), so hq, hs, the expert rows and the layer output are compared
  bit for bit: at the prefill shape (T = 8192, H = 4096, I = 2048, E = 256
  top-8 + shared, uniform routing), at decode batches (T = 64 and 512, Zipf
  load) and at ragged shapes
  (Zipf load with empty, one-row and remainder M tiles, a down N that is
  not a multiple of the 256-column tile, gate/up N of 10 column tiles),
  with fp32 block scales and with power-of-two scales (e8m0 weight scales,
  ue8m0 activation scales: both applied inside the MFMA).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_values, to_dev_bf16, to_dev_f32, u8
from test_frag_layout import frag_fp4_layout_ref, frag_layout_ref

pytestmark = pytest.mark.gpu


def test_weight_to_frag_matches_layout(gpu):
    from sglang_lite_amd import kernel as K

    rng = np.random.default_rng(3)
    for N, K_ in ((16, 128), (48, 384), (2048, 4096)):
        w = rng.integers(0, 256, size=(N, K_), dtype=np.uint8)
        wd = torch.from_numpy(w).to(gpu).view(torch.float8_e4m3fn)
        out = K.fp8_weight_to_frag(wd)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), frag_layout_ref(w), err_msg=f"{N}x{K_}")


def test_fp4_weight_to_frag_matches_layout(gpu):
    from sglang_lite_amd import kernel as K

    rng = np.random.default_rng(4)
    for N, K_ in ((16, 512), (48, 1024), (2048, 4096)):
        w = rng.integers(0, 256, size=(N, K_ // 2), dtype=np.uint8)
        sc = rng.integers(0, 256, size=(N, K_ // 32), dtype=np.uint8)
        ow, os_ = K.fp4_weight_to_frag(torch.from_numpy(w).to(gpu),
                                       torch.from_numpy(sc).to(gpu).view(torch.float8_e8m0fnu))
        torch.cuda.synchronize()
        wf, sf = frag_fp4_layout_ref(w, sc)
        np.testing.assert_array_equal(ow.cpu().numpy(), wf, err_msg=f"weights {N}x{K_}")
        np.testing.assert_array_equal(os_.cpu().numpy(), sf, err_msg=f"scales {N}x{K_}")


def _fp4_experts(dev, E, H, I, seed):
    """MXFP4 routed experts as the reference's live format stores them:
    packed e2m1 codes drawn uniformly, e8m0 1 x 32 scales in [2^-9, 2^-5]."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    u8_, e8 = torch.uint8, torch.float8_e8m0fnu
    ent = []
    for _ in range(E):
        w1 = torch.randint(0, 256, (I, H // 2), dtype=u8_, device=dev, generator=g)
        w3 = torch.randint(0, 256, (I, H // 2), dtype=u8_, device=dev, generator=g)
        w2 = torch.randint(0, 256, (H, I // 2), dtype=u8_, device=dev, generator=g)
        s1 = torch.randint(118, 123, (I, H // 32), dtype=u8_, device=dev, generator=g).view(e8)
        s3 = torch.randint(118, 123, (I, H // 32), dtype=u8_, device=dev, generator=g).view(e8)
        s2 = torch.randint(118, 123, (H, I // 32), dtype=u8_, device=dev, generator=g).view(e8)
        ent.append((w1, w3, w2, s1, s3, s2))
    return ent


def _experts(dev, n, H, I, seed, ue8m0=False):
    from sglang_lite_amd import kernel as K

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    ent = []
    for _ in range(n):
        row = []
        for shape in ((I, H), (I, H), (H, I)):
            q, s = K.per_block_cast_to_fp8(torch.randn(*shape, generator=g, device=dev) * 0.02, ue8m0)
            row.append((q, s))
        ent.append((row[0][0], row[1][0], row[2][0], row[0][1], row[1][1], row[2][1]))
    return ent


def _zipf_ids(rng, T, E, k, s=1.1):
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = rng.permutation(E)
    logits = (np.log(p)[np.argsort(perm)][None, :] + rng.gumbel(size=(T, E))).astype(np.float32)
    return logits


def _compare(gpu, x, logits, ent, E, k, swiglu_limit=0.0, mode=0, pow2_flag=None):
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    T = x.shape[0]
    rows = M.ExpertTable.build(ent[:E], ent[E])
    frag = M.ExpertTable.build(ent[:E], ent[E], frag_layout=True)
    assert frag.fmt & 4 and frag.ptrs.shape[0] == 2 * (E + 1)
    # power-of-two scales: both scales in the MFMA
    assert bool(rows.fmt & 2) == ((mode == 1) if pow2_flag is None else pow2_flag)
    w, ids = M.route_topk(to_dev_f32(logits, gpu), k)
    xd = to_dev_bf16(x, gpu)
    xq, xs = K.act_quant(xd, scale_mode=mode)
    counts, offsets, sorted_slot, _ = M.permute(ids, E)
    res = {}
    for name, table in (("rows", rows), ("frag", frag)):
        hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), table, k,
                           swiglu_limit=swiglu_limit, scale_mode=mode)
        out = M.down(hq, hs, offsets, sorted_slot, table, T, k, scale_mode=mode)
        y = M.moe_forward(xd, ids, w, table, swiglu_limit=swiglu_limit, scale_mode=mode)
        torch.cuda.synchronize()
        res[name] = (u8(hq), u8(hs), u8(out), u8(y))
    for i, what in enumerate(("hq", "hs", "expert rows", "layer")):
        np.testing.assert_array_equal(res["frag"][i], res["rows"][i], err_msg=what)
    return counts.cpu().numpy()


@pytest.mark.parametrize("pow2", [False, True])
def test_prefill_shape_bit_identical(gpu, pow2):
    H, I, E, k, T = 4096, 2048, 256, 8, 8192
    print(f"frag prefill T={T} pow2={pow2}", flush=True)
    rng = np.random.default_rng(11)
    ent = _experts(gpu, E + 1, H, I, seed=5, ue8m0=pow2)
    x = bf16_values(rng, (T, H))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    counts = _compare(gpu, x, logits, ent, E, k, mode=1 if pow2 else 0)
    assert counts.sum() == T * k


@pytest.mark.parametrize("T", [64, 512])
def test_decode_shape_bit_identical(gpu, T):
    """Decode batches (Zipf(1.1) expert load, most experts with a few rows)
    against the LDS-staged decode kernel."""
    H, I, E, k = 4096, 2048, 256, 8
    print(f"frag decode T={T}", flush=True)
    rng = np.random.default_rng(T + 1)
    ent = _experts(gpu, E + 1, H, I, seed=6)
    x = bf16_values(rng, (T, H))
    logits = _zipf_ids(rng, T, E, k)
    counts = _compare(gpu, x, logits, ent, E, k)
    assert (counts > 0).sum() > E // 2


@pytest.mark.parametrize("H,I,pow2", [(2176, 2048, False), (2048, 1280, False), (2176, 2048, True)])
def test_ragged_shapes_bit_identical(gpu, H, I, pow2):
    E, k, T = 16, 4, 600
    print(f"frag ragged H={H} I={I} pow2={pow2}", flush=True)
    rng = np.random.default_rng(H + I)
    ent = _experts(gpu, E + 1, H, I, seed=H, ue8m0=pow2)
    x = bf16_values(rng, (T, H))
    logits = _zipf_ids(rng, T, E, k)
    counts = _compare(gpu, x, logits, ent, E, k, swiglu_limit=7.0, mode=1 if pow2 else 0)
    assert (counts % 128 != 0).any()  # remainder M tiles were exercised


@pytest.mark.parametrize("T,mode", [(64, 3), (64, 0), (8192, 3), (8192, 0)])
def test_fp4_experts_bit_identical(gpu, T, mode):
    """FP4 routed experts (the live format) with the FP8 shared expert: the
    register-fed fp4 kernels (weight scales in the MFMA; row scales in the
    MFMA in the ue8m0 mode 3, promoted in fp32 in mode 0) against the
    LDS-staged FP4 kernels, at decode (Zipf) and prefill (uniform) batches."""
    H, I, E, k = 4096, 2048, 256, 8
    print(f"frag fp4 T={T} mode={mode}", flush=True)
    rng = np.random.default_rng(T + mode)
    ent = _fp4_experts(gpu, E, H, I, seed=9) + _experts(gpu, 1, H, I, seed=10, ue8m0=(mode == 3))
    x = bf16_values(rng, (T, H))
    logits = _zipf_ids(rng, T, E, k) if T <= 512 else rng.standard_normal((T, E)).astype(np.float32)
    counts = _compare(gpu, x, logits, ent, E, k, mode=mode, pow2_flag=(mode == 3))
    assert counts.sum() == T * k


@pytest.mark.parametrize("frag", [False, True])
def test_fp4_layer_in_a_graph_replays_equal_eager(gpu, frag):
    """The FP4 layer at a decode batch (routed FP4 launch, then the FP8 shared
    expert's launch) captured into a HIP graph on the caller's stream: every
    replay, with eager layers and synchronizations between them, equals the
    eager layer bit for bit."""
    from sglang_lite_amd import moe as M

    H, I, E, k, T = 4096, 2048, 256, 8, 64
    print(f"fp4 graph frag={frag}", flush=True)
    rng = np.random.default_rng(21)
    ent = _fp4_experts(gpu, E, H, I, seed=12) + _experts(gpu, 1, H, I, seed=13, ue8m0=True)
    table = M.ExpertTable.build(ent[:E], ent[E], frag_layout=frag)
    x = to_dev_bf16(bf16_values(rng, (T, H)), gpu)
    w, ids = M.route_topk(to_dev_f32(_zipf_ids(rng, T, E, k), gpu), k)
    x2 = to_dev_bf16(bf16_values(rng, (T, H)), gpu)
    ws = M.MoEWorkspace()
    y = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    M.moe_forward(x, ids, w, table, workspace=ws, out=y, scale_mode=3)
    torch.cuda.synchronize()
    eager = u8(y).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        M.moe_forward(x, ids, w, table, workspace=ws, out=y, scale_mode=3)
    for i in range(4):
        y.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(u8(y), eager, err_msg=f"replay {i}")
        # eager work between replays, on its own workspace
        M.moe_forward(x2, ids, w, table, scale_mode=3)
        torch.cuda.synchronize()
