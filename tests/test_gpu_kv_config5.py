"""The FP8 KV pack and the sparse-MLA gather-dequant at the benchmarked size,
bit-exact against the oracle: a 65,536-token cache of 576-dim rows (512-dim
latent + 64-dim rope, bf16 N(0, 1), seed 5), packed as 656-byte rows
(layout B: e4m3 latent with 4 fp32 per-128 scales, rope bf16) and as the
reference's 584-byte rows in footer pages of 64 (layout A,
engine/dsv4_kv_pack.py:40-146), then 128 queries each gathering 2048
distinct uniformly random rows (torch.randperm) from each cache
(engine/v4_sparse_torch.py:77-83 semantics)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv as OK
from oracle import quant as Q

pytestmark = pytest.mark.gpu

T, NQ, NSEL = 65536, 128, 2048


@pytest.fixture(scope="module")
def cache(gpu):
    g = torch.Generator().manual_seed(5)
    kv = torch.randn(T, 576, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(T, generator=g)[:NSEL] for _ in range(NQ)]).to(torch.int32)
    return kv, idx


def _bf16_bits(a: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_layout_b_pack_and_gather_65536_rows(gpu, cache):
    from sglang_lite_amd import dsv4_kv_pack as KVP

    kv, idx = cache
    print(f"layout B pack T={T}, gather {NQ}x{NSEL}", flush=True)
    x = kv.float().numpy()
    rows_ref = OK.pack_layout_b(x[:, :512], kv[:, 512:].contiguous().view(torch.uint8).numpy())
    rows = KVP.pack_kv_latent_rope(kv.to(gpu))
    got_rows = rows.cpu().numpy()
    assert got_rows.shape == (T, 656)
    np.testing.assert_array_equal(got_rows, rows_ref)
    d_idx = idx.to(gpu)
    out = KVP.gather_dequant(rows, d_idx, layout="B")
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert got.shape == (NQ, NSEL, 576)
    deq = _bf16_bits(OK.dequant_row_b(rows_ref))
    np.testing.assert_array_equal(got, deq[idx.numpy()])
    # every row of the cache is the row's own dequant: spot check the decode
    # against the input (half an e4m3 step plus the bf16 rounding, 2^-8 relative)
    sf = np.ascontiguousarray(rows_ref[:, 640:656]).view("<f4").reshape(T, 4)
    dv = OK.dequant_row_b(rows_ref)[:, :512]
    step = np.maximum(np.abs(x[:, :512]) * 2.0**-4, np.repeat(sf, 128, axis=1) * 2.0**-10)
    assert np.all(np.abs(dv - x[:, :512]) <= step + np.abs(dv) * 2.0**-8)


def test_layout_a_paged_pack_and_gather_65536_rows(gpu, cache):
    from sglang_lite_amd import dsv4_kv_pack as KVP

    kv, idx = cache
    print(f"layout A paged pack T={T}, gather {NQ}x{NSEL}", flush=True)
    a = kv[:, :512].contiguous()
    xv = a.float().numpy()
    rope = a[:, 448:].contiguous().view(torch.uint8).numpy()
    rows_ref = OK.pack_layout_a(xv, rope, 4)
    pages_ref = OK.to_paged_hnd(rows_ref, 64)
    pages = KVP.pack_dsv4_kv_paged(a.to(gpu), 64)
    np.testing.assert_array_equal(pages.cpu().numpy(), pages_ref)
    d_idx = idx.to(gpu)
    out = KVP.gather_dequant(pages, d_idx, layout="A", page_size=64)
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert got.shape == (NQ, NSEL, 512)
    deq = _bf16_bits(OK.dequant_row_a(rows_ref))
    np.testing.assert_array_equal(got, deq[idx.numpy()])
    # the rows gathered from the logical [T, 584] rows are the same
    flat = KVP.pack_dsv4_kv_bf16(a.to(gpu))
    np.testing.assert_array_equal(flat.cpu().numpy(), rows_ref)
    out2 = KVP.gather_dequant(flat, d_idx[:8], layout="A")
    assert torch.equal(out2, out[:8])
