"""Sparse MLA attention on the GPU against the oracle: bf16 KV (the official
kernel.sparse_attn contract), and the packed FP8 cache (layout A rows and
footer pages) read directly."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_gemm_close, bf16_values, f32, to_dev_bf16, to_dev_f32
from oracle import attn as OA
from oracle import kv as OK

pytestmark = pytest.mark.gpu


def _case(rng, B, S, H, n, K, pad=0.1):
    q = bf16_values(rng, (B, S, H, 512))
    kv = bf16_values(rng, (B, n, 512))
    sink = (rng.standard_normal(H) * 2).astype(np.float32)
    idx = np.stack([np.stack([rng.permutation(n)[:K] for _ in range(S)]) for _ in range(B)]).astype(np.int32)
    idx[rng.random(idx.shape) < pad] = -1
    return q, kv, sink, idx


# small batches split their rows over workgroups (partials + merge); the
# 256-query case fills the device with one workgroup per query and runs unsplit
@pytest.mark.parametrize("B,S,H,n,K", [(1, 1, 64, 300, 128), (2, 3, 16, 700, 640), (1, 4, 8, 100, 70),
                                        (3, 1, 64, 2048, 512), (1, 2, 128, 256, 200),
                                        (1, 256, 64, 600, 192), (1, 1, 64, 5000, 4096)])
def test_sparse_attn_bf16_matches_oracle(gpu, B, S, H, n, K):
    from sglang_lite_amd import v4_sparse_mla as SA

    print(f"sparse_attn bf16 B={B} S={S} H={H} n={n} K={K}", flush=True)
    rng = np.random.default_rng(B * 100 + S * 10 + H + K)
    q, kv, sink, idx = _case(rng, B, S, H, n, K)
    scale = 512 ** -0.5
    o = SA.sparse_attn(to_dev_bf16(q, gpu), to_dev_bf16(kv, gpu), to_dev_f32(sink, gpu),
                       torch.from_numpy(idx).to(gpu), scale)
    assert o.dtype == torch.bfloat16 and o.shape == (B, S, H, 512)
    got = f32(o)
    assert_gemm_close(got, OA.sparse_attn_blocked(q, kv, sink, idx, scale), "vs blocked oracle")
    assert_gemm_close(got, OA.sparse_attn_exact(q, kv, sink, idx, scale), "vs exact softmax")


def test_sparse_attn_masked_rows_and_all_masked_query(gpu):
    from sglang_lite_amd import v4_sparse_mla as SA

    rng = np.random.default_rng(7)
    B, S, H, n, K = 1, 2, 16, 50, 100
    q, kv, sink, idx = _case(rng, B, S, H, n, K, pad=0.0)
    idx[0, 0, :] = -1            # every row masked: output zero
    idx[0, 1, ::3] = n + 5       # out of range rows are masked like -1
    idx[0, 1, :64] = -1          # a whole 64-row block (one split) masked
    o = f32(SA.sparse_attn(to_dev_bf16(q, gpu), to_dev_bf16(kv, gpu), to_dev_f32(sink, gpu),
                           torch.from_numpy(idx).to(gpu), 0.05))
    assert np.all(o[0, 0] == 0)
    assert_gemm_close(o, OA.sparse_attn_blocked(q, kv, sink, idx, 0.05), "masked")


@pytest.mark.parametrize("paged", [False, True])
def test_sparse_attn_packed_cache_matches_oracle(gpu, paged):
    """The fused consumer: attention straight off the layout A cache equals the
    attention over the cache's dequantized rows (the reference's pack ->
    FlashInfer path, v4_sparse_mla.py:34-122, without the pack)."""
    from sglang_lite_amd import dsv4_kv_pack as KVP
    from sglang_lite_amd import v4_sparse_mla as SA

    rng = np.random.default_rng(11 + paged)
    B, S, H, n, K = 2, 2, 64, 333, 256
    q, kv, sink, idx = _case(rng, B, S, H, n, K)
    kvd = to_dev_bf16(kv, gpu)
    if paged:
        cache = torch.stack([KVP.pack_dsv4_kv_paged(kvd[i], 64) for i in range(B)])
    else:
        cache = KVP.pack_dsv4_kv_bf16(kvd)
    # dequantized rows of the packed cache (the gather-dequant oracle's rows)
    rows = np.stack([OK.dequant_row_a(KVP.pack_dsv4_kv_bf16(kvd[i]).cpu().numpy()) for i in range(B)])
    o = SA.sparse_attn_packed(to_dev_bf16(q, gpu), cache, to_dev_f32(sink, gpu),
                              torch.from_numpy(idx).to(gpu), 512 ** -0.5, n_rows=n)
    got = f32(o)
    assert_gemm_close(got, OA.sparse_attn_blocked(q, rows, sink, idx, 512 ** -0.5), "packed vs blocked")
    # and the packed path equals the bf16 path over the dequantized rows
    o2 = SA.sparse_attn(to_dev_bf16(q, gpu), to_dev_bf16(rows, gpu), to_dev_f32(sink, gpu),
                        torch.from_numpy(idx).to(gpu), 512 ** -0.5)
    np.testing.assert_array_equal(o.view(torch.int16).cpu().numpy(), o2.view(torch.int16).cpu().numpy())


def test_attach_patches_official_sparse_attn(gpu, monkeypatch):
    """attach_v4_sparse_mla replaces kernel.sparse_attn / model.sparse_attn
    (v4_sparse_mla.py:144-250); SGLANG_LITE_V4_SPARSE=official keeps them."""
    import fake_official
    from sglang_lite_amd import v4_sparse_mla as SA

    M, K, saved = fake_official.install()
    try:
        monkeypatch.setenv("SGLANG_LITE_V4_SPARSE", "official")
        assert SA.attach_v4_sparse_mla(None) is False and K.sparse_attn is M.sparse_attn
        monkeypatch.setenv("SGLANG_LITE_V4_SPARSE", "auto")
        assert SA.attach_v4_sparse_mla(None) is True
        assert getattr(K.sparse_attn, SA.MARK, False) and M.sparse_attn is K.sparse_attn
        rng = np.random.default_rng(3)
        q, kv, sink, idx = _case(rng, 1, 1, 64, 200, 160)
        o = M.sparse_attn(to_dev_bf16(q, gpu), to_dev_bf16(kv, gpu), to_dev_f32(sink, gpu),
                          torch.from_numpy(idx).to(gpu), 0.04)
        assert_gemm_close(f32(o), OA.sparse_attn_blocked(q, kv, sink, idx, 0.04), "patched sparse_attn")
        SA.detach_v4_sparse_mla()
        assert not getattr(K.sparse_attn, SA.MARK, False)
    finally:
        fake_official.uninstall(saved)


def test_sparse_attn_workspace_contract(gpu):
    """Small batches need the split workspace; a too-small one is refused."""
    from sglang_lite_amd import _lib

    lib = _lib.load()
    assert lib.sgl_sparse_attn_workspace_size(1, 1, 64, 640) > 0
    assert lib.sgl_sparse_attn_workspace_size(1, 1, 64, 64) == 0      # one block: no split
    assert lib.sgl_sparse_attn_workspace_size(4, 1024, 64, 2048) == 0  # device already full
    rng = np.random.default_rng(5)
    q, kv, sink, idx = _case(rng, 1, 1, 64, 300, 256)
    qd, kvd = to_dev_bf16(q, gpu), to_dev_bf16(kv, gpu)
    sd, idd = to_dev_f32(sink, gpu), torch.from_numpy(idx).to(gpu)
    o = torch.empty_like(qd)
    need = lib.sgl_sparse_attn_workspace_size(1, 1, 64, 256)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    rc = lib.sgl_sparse_attn(qd.data_ptr(), 1, 1, 64, kvd.data_ptr(), _lib.ATTN_KV_BF16, 0, 300,
                             kvd.stride(0) * 2, 512, sd.data_ptr(), idd.data_ptr(), 256, 0.04,
                             o.data_ptr(), ws.data_ptr(), need - 16, _lib.stream_of(qd))
    assert rc == _lib.SGL_ERR_WORKSPACE and "workspace" in _lib.last_error()


def test_sparse_attn_without_indices_gives_zero_output(gpu):
    """K = 0 (no selected rows, null index pointer): the kernel reads no index
    and the output is the sink-only softmax's zero (the oracle's closed form
    with no gathered rows)."""
    from sglang_lite_amd import _lib

    lib = _lib.load()
    print("sparse_attn K=0 B=1 S=2 H=64 n=300", flush=True)
    rng = np.random.default_rng(6)
    q, kv, sink, _ = _case(rng, 1, 2, 64, 300, 64)
    qd, kvd = to_dev_bf16(q, gpu), to_dev_bf16(kv, gpu)
    sd = to_dev_f32(sink, gpu)
    o = torch.full_like(qd, 7.0)
    assert lib.sgl_sparse_attn_workspace_size(1, 2, 64, 0) == 0
    rc = lib.sgl_sparse_attn(qd.data_ptr(), 1, 2, 64, kvd.data_ptr(), _lib.ATTN_KV_BF16, 0, 300,
                             kvd.stride(0) * 2, 512, sd.data_ptr(), None, 0, 0.04,
                             o.data_ptr(), None, 0, _lib.stream_of(qd))
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(o).item() == 0
