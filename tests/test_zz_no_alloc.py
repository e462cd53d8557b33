"""sgl_moe_forward_noalloc (the layer's workspace in a static device array)
against sgl_moe_forward with a caller-allocated workspace, through the C ABI:
bit-identical outputs on consecutive calls, the second with fewer tokens
than the first (the array keeps the first call's contents), at the decode
expert shapes (hidden 4096, intermediate 2048, 256 experts top-8 + shared);
a token count whose workspace exceeds the array is refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_values, to_dev_bf16, u8

pytestmark = pytest.mark.gpu

H, I, E, K_TOP = 4096, 2048, 256, 8


def _experts(dev):
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    g = torch.Generator(device=dev)
    g.manual_seed(17)
    n = E + 1
    w13 = torch.empty(n, 2, I, H, dtype=torch.float8_e4m3fn, device=dev)
    s13 = torch.empty(n, 2, I // 128, H // 128, dtype=torch.float32, device=dev)
    w2 = torch.empty(n, H, I, dtype=torch.float8_e4m3fn, device=dev)
    s2 = torch.empty(n, H // 128, I // 128, dtype=torch.float32, device=dev)
    for e in range(n):
        for j in range(2):
            q, s = K.per_block_cast_to_fp8(torch.randn(I, H, generator=g, device=dev) * 0.02, False)
            w13[e, j].copy_(q)
            s13[e, j].copy_(s)
        q, s = K.per_block_cast_to_fp8(torch.randn(H, I, generator=g, device=dev) * 0.02, False)
        w2[e].copy_(q)
        s2[e].copy_(s)
    ent = [(w13[e, 0], w13[e, 1], w2[e], s13[e, 0], s13[e, 1], s2[e]) for e in range(n)]
    return M.ExpertTable.build(ent[:E], ent[E])


def _inputs(rng, T, dev):
    from sglang_lite_amd import moe as M

    x = to_dev_bf16(bf16_values(rng, (T, H)), dev)
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    w, ids = M.route_topk(logits, K_TOP)
    return x, ids, w


def _noalloc(x, ids, w, table, y, lim=0.0, mode=0):
    from sglang_lite_amd import _lib

    T = x.shape[0]
    _lib.call("sgl_moe_forward_noalloc", x.data_ptr(), T, H, I, E, K_TOP, ids.data_ptr(),
              w.data_ptr(), table.ptrs.data_ptr(), int(table.has_shared), table.fmt, float(lim),
              int(mode), y.data_ptr(), _lib.stream_of(x))


def _with_workspace(x, ids, w, table, y, lim=0.0, mode=0):
    from sglang_lite_amd import _lib
    from sglang_lite_amd import moe as M

    T = x.shape[0]
    nbytes = M.workspace_size(T, H, I, E, K_TOP, True)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    _lib.call("sgl_moe_forward", x.data_ptr(), T, H, I, E, K_TOP, ids.data_ptr(), w.data_ptr(),
              table.ptrs.data_ptr(), int(table.has_shared), table.fmt, float(lim), int(mode),
              ws.data_ptr(), ws.numel(), y.data_ptr(), _lib.stream_of(x))


def test_noalloc_matches_the_workspace_entry_point(gpu):
    from sglang_lite_amd import _lib

    print("noalloc MoE: T=512 then T=64, fp32 and ue8m0 scale modes", flush=True)
    assert _lib.load().sgl_moe_workspace_size(512, H, I, E, K_TOP, 1) <= 64 << 20
    table = _experts(gpu)
    rng = np.random.default_rng(77)
    for T, lim, mode in ((512, 0.0, 0), (64, 0.0, 0), (512, 10.0, 1), (37, 0.0, 1)):
        x, ids, w = _inputs(rng, T, gpu)
        y0 = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
        y1 = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
        _with_workspace(x, ids, w, table, y0, lim, mode)
        _noalloc(x, ids, w, table, y1, lim, mode)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(u8(y1), u8(y0), err_msg=f"T={T} lim={lim} mode={mode}")
        assert bool(torch.isfinite(y1.float()).all())


def test_noalloc_refuses_tokens_beyond_the_static_workspace(gpu):
    from sglang_lite_amd import _lib

    T = 1024  # ~99 MB of workspace at these shapes, above the 64 MiB array
    need = _lib.load().sgl_moe_workspace_size(T, H, I, E, K_TOP, 1)
    assert need > 64 << 20
    x = torch.zeros(8, H, dtype=torch.bfloat16, device=gpu)
    y = torch.zeros(8, H, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(_lib.SglError) as ei:
        _lib.call("sgl_moe_forward_noalloc", x.data_ptr(), T, H, I, E, K_TOP, None, None, None, 1,
                  0, 0.0, 0, y.data_ptr(), _lib.stream_of(x))
    assert ei.value.status == _lib.SGL_ERR_WORKSPACE
    assert "static" in ei.value.message
    torch.cuda.synchronize()
    assert bool((y == 0).all())
