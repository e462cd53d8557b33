"""FP8 KV pack / paging / gather-dequant / index split on the GPU: bit-exact
against the oracle, plus the reference's own KV tests run on the device
(tests/test_dsv4_kv_pack.py:16-65, tests/test_v4_dual_pool.py:57-75)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_e4m3_equal_nan_signless, bf16_values, nan_inf_rows, u8
from oracle import kv as OK
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _official_act_quant():
    """Stand-in for the official TileLang ``kernel.act_quant`` (identified by
    module and name): the pack kernels compute its ue8m0 formula themselves,
    so it is never called."""
    def act_quant(*a, **k):
        raise AssertionError("the official act_quant's formula runs in the fused kernel")
    act_quant.__module__ = "kernel"
    return act_quant


def _kv(rng, T, dim, dtype):
    x = bf16_values(rng, (T, dim))
    t = torch.from_numpy(x).to(dtype)
    return t.float().numpy(), t


def _quantizer(mode):
    """The act_quant_fn whose formula is scale mode ``mode``: None (the torch
    fallback), the official TileLang act_quant, or this package's act_quant
    with its default torch formula."""
    from sglang_lite_amd import kernel as HK

    return {4: None, 3: _official_act_quant(), 1: HK.act_quant}[mode]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", [4, 3, 1])
@pytest.mark.parametrize("T", [1, 70, 4096])
def test_pack_layout_a_bit_exact(gpu, dtype, mode, T, monkeypatch):
    from sglang_lite_amd import dsv4_kv_pack as KVP

    monkeypatch.delenv("SGLANG_LITE_AMD_ACT_QUANT", raising=False)
    rng = np.random.default_rng(T + mode)
    xv, xt = _kv(rng, T, 512, dtype)
    if T > 2:
        xt[1, :64] = 0.0
        xv[1, :64] = 0.0
    rope = xt[:, 448:].contiguous().view(torch.uint8).numpy()
    ref = OK.pack_layout_a(xv, rope, mode)
    d = xt.to(gpu)
    out = KVP.pack_dsv4_kv_bf16(d, act_quant_fn=_quantizer(mode))
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    pages = KVP.pack_dsv4_kv_paged(d, 64, act_quant_fn=_quantizer(mode))
    np.testing.assert_array_equal(pages.cpu().numpy(), OK.to_paged_hnd(ref, 64))
    pages2 = KVP.to_paged_hnd(out, 64)
    np.testing.assert_array_equal(pages2.cpu().numpy(), OK.to_paged_hnd(ref, 64))


@pytest.mark.parametrize("mode", [4, 3, 1])
def test_pack_layout_a_nan_and_inf_rows(gpu, mode, monkeypatch):
    """Rows with NaN / Inf values: scale bytes and RoPE bytes exact, the e4m3
    bytes exact up to the sign of NaN codes, plain and footer-paged."""
    from sglang_lite_amd import dsv4_kv_pack as KVP

    monkeypatch.delenv("SGLANG_LITE_AMD_ACT_QUANT", raising=False)
    x = nan_inf_rows(np.random.default_rng(mode), 512)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    rope = xt[:, 448:].contiguous().view(torch.uint8).numpy()
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        ref = OK.pack_layout_a(x, rope, mode)
    d = xt.to(gpu)
    for got, want, what in ((KVP.pack_dsv4_kv_bf16(d, act_quant_fn=_quantizer(mode)), ref, "rows"),
                            (KVP.to_paged_hnd(KVP.pack_dsv4_kv_bf16(d, act_quant_fn=_quantizer(mode)), 64),
                             OK.to_paged_hnd(ref, 64), "pages")):
        g = got.cpu().numpy()
        if what == "pages":
            g, want = OK.unpage(g, 64)[:6], OK.unpage(want, 64)[:6]
        assert_e4m3_equal_nan_signless(g[:, :448], want[:, :448], f"layout A mode {mode} {what} e4m3")
        np.testing.assert_array_equal(g[:, 448:], want[:, 448:])
    pages = KVP.pack_dsv4_kv_paged(d, 64, act_quant_fn=_quantizer(mode)).cpu().numpy()
    g, want = OK.unpage(pages, 64)[:6], ref
    assert_e4m3_equal_nan_signless(g[:, :448], want[:, :448], f"layout A mode {mode} paged e4m3")
    np.testing.assert_array_equal(g[:, 448:], want[:, 448:])


@pytest.mark.parametrize("page,T", [(16, 100), (48, 97), (40, 90), (64, 128), (128, 300), (7, 30),
                                    (2, 5)])
def test_pack_paged_page_sizes_and_strided_rows(gpu, page, T):
    """Footer pages at several page sizes (odd ones among them), a ragged
    last page, and input rows that are a view of a wider [T, 576] buffer (row
    stride 576)."""
    from sglang_lite_amd import dsv4_kv_pack as KVP

    print(f"paged pack page={page} T={T}", flush=True)
    rng = np.random.default_rng(page * 1000 + T)
    wide = bf16_values(rng, (T, 576))
    wt = torch.from_numpy(wide).to(torch.bfloat16)
    xt = wt[:, :512]
    xv = xt.float().numpy()
    rope = xt[:, 448:].contiguous().view(torch.uint8).numpy()
    ref = OK.to_paged_hnd(OK.pack_layout_a(xv, rope, 4), page)
    pages = KVP.pack_dsv4_kv_paged(wt.to(gpu)[:, :512], page)
    np.testing.assert_array_equal(pages.cpu().numpy(), ref)


def test_pack_calls_an_injected_quantizer(gpu):
    """dsv4_kv_pack.py:58-61: a quantizer other than the official act_quant is
    called on the NoPE part as (nope, 64, "ue8m0", float8_e8m0fnu, False) and
    its bytes are packed: with the KV formula it reproduces the default pack,
    with a constant quantizer its bytes land in place (rows and pages)."""
    import functools

    from sglang_lite_amd import dsv4_kv_pack as KVP
    from sglang_lite_amd import kernel as K_

    rng = np.random.default_rng(31)
    xv, xt = _kv(rng, 130, 512, torch.bfloat16)
    d = xt.to(gpu)
    calls = []

    def kv_formula(x, block, fmt, sdtype, inplace):
        calls.append((tuple(x.shape), block, fmt, sdtype, inplace))
        return K_.act_quant(x, block, fmt, sdtype, inplace, scale_mode=4)

    got = KVP.pack_dsv4_kv_bf16(d, act_quant_fn=kv_formula)
    assert calls == [((130, 448), 64, "ue8m0", torch.float8_e8m0fnu, False)]
    np.testing.assert_array_equal(got.cpu().numpy(), KVP.pack_dsv4_kv_bf16(d).cpu().numpy())

    def const(x, block, fmt, sdtype, inplace):
        y = torch.full(x.shape, 0x3C, dtype=torch.uint8, device=x.device).view(torch.float8_e4m3fn)
        s = torch.full((*x.shape[:-1], x.shape[-1] // block), 0x7A, dtype=torch.uint8,
                       device=x.device).view(torch.float8_e8m0fnu)
        return y, s

    rows = KVP.pack_dsv4_kv_bf16(d, act_quant_fn=const).cpu().numpy()
    assert np.all(rows[:, :448] == 0x3C) and np.all(rows[:, 576:583] == 0x7A)
    assert np.all(rows[:, 583] == 0)
    np.testing.assert_array_equal(rows[:, 448:576], xt[:, 448:].contiguous().view(torch.uint8).numpy())
    pages = KVP.pack_dsv4_kv_paged(d, 64, act_quant_fn=functools.partial(const)).cpu().numpy()
    np.testing.assert_array_equal(pages, OK.to_paged_hnd(rows, 64))
    pool = torch.zeros(1, 4, 1, 64, 584, dtype=torch.uint8, device=gpu)
    with pytest.raises(TypeError, match="act_quant_fn"):
        KVP.write_packed_kv_bf16(pool, [0, 1, 2], 0, d, act_quant_fn=const)


def test_reference_pack_shape_and_rope_bytes(gpu):
    """tests/test_dsv4_kv_pack.py:16-25 on the device."""
    from sglang_lite_amd.dsv4_kv_pack import DSV4_PACKED_BYTES, pack_dsv4_kv_bf16

    kv = torch.randn(3, 512, dtype=torch.bfloat16)
    kv[:, 448:] = torch.arange(64, dtype=torch.bfloat16)
    packed = pack_dsv4_kv_bf16(kv.to(gpu)).cpu()
    assert packed.shape == (3, DSV4_PACKED_BYTES)
    assert packed.dtype == torch.uint8
    rope_u8 = kv[:, 448:].contiguous().view(torch.uint8).view(3, 128)
    assert torch.equal(packed[:, 448:576], rope_u8)
    assert (packed[:, 583] == 0).all()


def test_reference_paging(gpu):
    """tests/test_dsv4_kv_pack.py:28-54 on the device."""
    from sglang_lite_amd.dsv4_kv_pack import (DSV4_DATA_BYTES, DSV4_PACKED_BYTES, DSV4_PAGE_SIZE,
                                              DSV4_SCALE_STRIDE, to_paged_hnd)

    pages = to_paged_hnd(torch.zeros(10, DSV4_PACKED_BYTES, dtype=torch.uint8, device=gpu),
                         page_size=DSV4_PAGE_SIZE)
    assert pages.shape == (1, 1, DSV4_PAGE_SIZE, DSV4_PACKED_BYTES)
    packed = torch.arange(70 * DSV4_PACKED_BYTES, dtype=torch.int64).to(torch.uint8)
    packed = packed.view(70, DSV4_PACKED_BYTES).clone()
    packed[0, :DSV4_DATA_BYTES] = 11
    packed[0, DSV4_DATA_BYTES:] = 22
    packed[1, :DSV4_DATA_BYTES] = 33
    packed[1, DSV4_DATA_BYTES:] = 44
    pages = to_paged_hnd(packed.to(gpu), page_size=DSV4_PAGE_SIZE).cpu()
    flat = pages.view(2, -1)[0]
    assert (flat[0:DSV4_DATA_BYTES] == 11).all()
    assert (flat[DSV4_DATA_BYTES: 2 * DSV4_DATA_BYTES] == 33).all()
    scale0 = DSV4_PAGE_SIZE * DSV4_DATA_BYTES
    assert (flat[scale0: scale0 + DSV4_SCALE_STRIDE] == 22).all()
    assert (flat[scale0 + DSV4_SCALE_STRIDE: scale0 + 2 * DSV4_SCALE_STRIDE] == 44).all()
    # page round trip is byte-identical (tests/test_v4_dual_pool.py:57-75)
    np.testing.assert_array_equal(OK.unpage(pages.numpy(), 64)[:70], packed.numpy())
    assert not OK.unpage(pages.numpy(), 64)[70:].any()


def test_reference_split_indices(gpu):
    """tests/test_dsv4_kv_pack.py:56-65 on the device, plus random int64 input."""
    from sglang_lite_amd.dsv4_kv_pack import split_swa_compress_indices

    topk = torch.tensor([[[0, 1, 2, -1, 4, 5]]], dtype=torch.int32, device=gpu)
    swa, swa_l, comp, comp_l = split_swa_compress_indices(topk, window_size=4)
    assert swa.shape == (1, 4)
    assert int(swa_l[0]) == 3
    assert torch.equal(comp[0].cpu(), torch.tensor([0, 1], dtype=torch.int32))
    assert int(comp_l[0]) == 2
    rng = np.random.default_rng(0)
    for (b, s, k, win) in [(2, 3, 200, 128), (4, 1, 100, 128), (1, 5, 640, 128), (3, 2, 0, 4)]:
        t = rng.integers(-1, 70000, (b, s, k)).astype(np.int64)
        ref = OK.split_swa_compress_indices(t, win)
        got = split_swa_compress_indices(torch.from_numpy(t).to(gpu), win)
        for r, g in zip(ref, got):
            np.testing.assert_array_equal(g.cpu().numpy(), r)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_pack_layout_b_bit_exact(gpu, dtype):
    from sglang_lite_amd import dsv4_kv_pack as KVP

    rng = np.random.default_rng(21)
    T = 333
    xv, xt = _kv(rng, T, 576, dtype)
    if dtype == torch.float32:
        rope = xt[:, 512:].to(torch.bfloat16).contiguous().view(torch.uint8).numpy()
    else:
        rope = xt[:, 512:].contiguous().view(torch.uint8).numpy()
    ref = OK.pack_layout_b(xv[:, :512], rope)
    out = KVP.pack_kv_latent_rope(xt.to(gpu))
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


def test_gather_dequant_bit_exact(gpu):
    from sglang_lite_amd import dsv4_kv_pack as KVP

    rng = np.random.default_rng(22)
    T = 1000
    xv, xt = _kv(rng, T, 512, torch.bfloat16)
    rope = xt[:, 448:].contiguous().view(torch.uint8).numpy()
    rows_a = OK.pack_layout_a(xv, rope, 4)
    idx = rng.integers(0, T, (8, 300)).astype(np.int32)
    idx[:, -5:] = -1
    idx[0, :3] = [0, T - 1, -1]
    ref = OK.gather_dequant(rows_a, idx, "A")
    d_rows = torch.from_numpy(rows_a).to(gpu)
    d_idx = torch.from_numpy(idx).to(gpu)
    got = KVP.gather_dequant(d_rows, d_idx, layout="A").float().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    pages = KVP.to_paged_hnd(d_rows, 64)
    got_p = KVP.gather_dequant(pages, d_idx, layout="A", page_size=64).float().cpu().numpy()
    np.testing.assert_array_equal(got_p.view(np.uint32), ref.view(np.uint32))
    # layout B
    xb, xbt = _kv(rng, T, 576, torch.bfloat16)
    rows_b = OK.pack_layout_b(xb[:, :512], xbt[:, 512:].contiguous().view(torch.uint8).numpy())
    ref_b = OK.gather_dequant(rows_b, idx, "B")
    got_b = KVP.gather_dequant(torch.from_numpy(rows_b).to(gpu), d_idx, layout="B")
    np.testing.assert_array_equal(got_b.float().cpu().numpy().view(np.uint32), ref_b.view(np.uint32))


def test_gather_dequant_rows_with_nan_codes_and_scales(gpu):
    """Rows holding e4m3 NaN codes or NaN scales (packed from NaN / Inf
    values, plus one NaN code planted in a finite row) beside plain rows:
    NaN where the oracle has NaN (the device writes the canonical bf16 NaN),
    every other value bit-exact, layouts A (plain and footer pages) and B."""
    from sglang_lite_amd import dsv4_kv_pack as KVP

    rng = np.random.default_rng(24)
    x = np.concatenate([nan_inf_rows(rng, 576), bf16_values(rng, (58, 576))])
    xt = torch.from_numpy(x).to(torch.bfloat16)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        rows_a = OK.pack_layout_a(x[:, :512], xt[:, 448:512].contiguous().view(torch.uint8).numpy(), 4)
        rows_b = OK.pack_layout_b(x[:, :512], xt[:, 512:].contiguous().view(torch.uint8).numpy())
    rows_a[7, 100] = 0x7F  # a NaN code in a finite row
    rows_b[8, 200] = 0xFF
    idx = rng.integers(0, 64, (4, 96)).astype(np.int32)
    idx[:, :8] = np.arange(8)
    idx[1, 8:16] = np.arange(8)
    d_idx = torch.from_numpy(idx).to(gpu)

    def check(got, ref, what):
        got = got.float().cpu().numpy()
        nan = np.isnan(ref)
        assert nan.any(), what
        assert np.array_equal(np.isnan(got), nan), f"{what}: NaN positions differ"
        assert np.all(got.view(np.uint32)[nan] == 0x7FC00000), f"{what}: NaN not canonical"
        np.testing.assert_array_equal(got.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])

    with np.errstate(invalid="ignore", over="ignore"):
        ref_a = OK.gather_dequant(rows_a, idx, "A")
        ref_b = OK.gather_dequant(rows_b, idx, "B")
    d_rows = torch.from_numpy(rows_a).to(gpu)
    check(KVP.gather_dequant(d_rows, d_idx, layout="A"), ref_a, "layout A")
    check(KVP.gather_dequant(KVP.to_paged_hnd(d_rows, 64), d_idx, layout="A", page_size=64), ref_a,
          "layout A pages")
    check(KVP.gather_dequant(torch.from_numpy(rows_b).to(gpu), d_idx, layout="B"), ref_b, "layout B")


def test_layout_a_dequant_equals_qat_inplace(gpu):
    """Layout A gather = the official QAT quant-dequant (kernel.py:84-91) of the
    NoPE part with the injected act_quant formula."""
    from sglang_lite_amd import dsv4_kv_pack as KVP

    rng = np.random.default_rng(23)
    xv, xt = _kv(rng, 200, 512, torch.bfloat16)
    d = xt.to(gpu)
    rows = KVP.pack_dsv4_kv_bf16(d, act_quant_fn=_official_act_quant())
    idx = torch.arange(200, dtype=torch.int32, device=gpu)[None]
    deq = KVP.gather_dequant(rows, idx, layout="A")[0].float().cpu().numpy()
    qat, _ = Q.act_quant_inplace_tilelang(xv[:, :448], 64, round_scale=True)
    np.testing.assert_array_equal(deq[:, :448], qat)
    np.testing.assert_array_equal(deq[:, 448:], xv[:, 448:])


@pytest.mark.parametrize("table_on_device", [False, True])
def test_packed_page_writer_bit_exact(gpu, table_on_device):
    """write_packed_kv_bf16 = pack_dsv4_kv_bf16 + RadixCache.write_packed_kv
    (kv_cache.py:340-390) in one kernel: the whole pool, untouched blocks and
    layers included, equals the oracle's page write of the packed rows."""
    from sglang_lite_amd import dsv4_kv_pack as KVP

    rng = np.random.default_rng(12 + table_on_device)
    L, NB, page, T, start = 3, 10, 64, 150, 37
    xv, xt = _kv(rng, T, 512, torch.bfloat16)
    rope = xt[:, 448:].contiguous().view(torch.uint8).numpy()
    rows = OK.pack_layout_a(xv, rope, 4)
    table = [7, 2, 9, 0]
    init = rng.integers(0, 256, (L, NB, 1, page, 584), dtype=np.uint8)
    pool = torch.from_numpy(init).to(gpu)
    bt = torch.tensor(table, dtype=torch.int32, device=gpu) if table_on_device else table
    KVP.write_packed_kv_bf16(pool, bt, start, xt.to(gpu), layer_idx=1)
    want = OK.write_packed_pages(init, table, start, rows, 1)
    np.testing.assert_array_equal(pool.cpu().numpy(), want)


def test_packed_page_writer_errors(gpu):
    from sglang_lite_amd import dsv4_kv_pack as KVP

    pool = torch.zeros(2, 4, 1, 64, 584, dtype=torch.uint8, device=gpu)
    kv = torch.zeros(100, 512, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="block_table too short"):
        KVP.write_packed_kv_bf16(pool, [0], 10, kv)
    with pytest.raises(RuntimeError, match="out of range"):
        KVP.write_packed_kv_bf16(pool, [0, 4], 0, kv)
    with pytest.raises(ValueError, match="layer_idx"):
        KVP.write_packed_kv_bf16(pool, [0, 1], 0, kv, layer_idx=2)
    with pytest.raises(ValueError, match="requires block_table"):
        KVP.write_packed_kv_bf16(pool, [], 0, kv)


def test_gather_dequant_ragged_steps_out_of_range_and_empty_cache(gpu):
    """Indices past the cache give zero rows; a gather whose row count is not
    a multiple of the rows per step (3 x 301) ends cleanly; an empty cache
    gives all-zero rows without reading it (layouts A, A pages, B)."""
    from sglang_lite_amd import dsv4_kv_pack as KVP

    print("gather ragged / out of range / empty cache", flush=True)
    rng = np.random.default_rng(23)
    T = 128
    xv, xt = _kv(rng, T, 512, torch.bfloat16)
    rows_a = OK.pack_layout_a(xv, xt[:, 448:].contiguous().view(torch.uint8).numpy(), 4)
    idx = rng.integers(0, T, (3, 301)).astype(np.int32)
    idx[0, :4] = [T, T + 7, 2 ** 30, -5]
    idx[2, -1] = T - 1
    d_idx = torch.from_numpy(idx).to(gpu)
    ref = OK.gather_dequant(rows_a, idx, "A")
    d_rows = torch.from_numpy(rows_a).to(gpu)
    got = KVP.gather_dequant(d_rows, d_idx, layout="A").float().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    pages = KVP.to_paged_hnd(d_rows, 64)
    got_p = KVP.gather_dequant(pages, d_idx, layout="A", page_size=64).float().cpu().numpy()
    np.testing.assert_array_equal(got_p.view(np.uint32), ref.view(np.uint32))
    xb, xbt = _kv(rng, T, 576, torch.bfloat16)
    rows_b = OK.pack_layout_b(xb[:, :512], xbt[:, 512:].contiguous().view(torch.uint8).numpy())
    ref_b = OK.gather_dequant(rows_b, idx, "B")
    got_b = KVP.gather_dequant(torch.from_numpy(rows_b).to(gpu), d_idx, layout="B")
    np.testing.assert_array_equal(got_b.float().cpu().numpy().view(np.uint32), ref_b.view(np.uint32))
    for layout, width in (("A", 584), ("B", 656)):
        empty = torch.zeros(0, width, dtype=torch.uint8, device=gpu)
        z = KVP.gather_dequant(empty, d_idx, layout=layout)
        assert torch.count_nonzero(z).item() == 0
