#!/usr/bin/env python3
"""Benchmark: the FP8 MoE layer (DeepSeek-V4-Flash expert shapes) on one MI355X.

Headline workload (one "step"): MoE prefill of T=8192 bf16 tokens, hidden 4096,
expert intermediate 2048, 256 routed experts top-8 (softmax over uniform N(0,1)
router logits) + 1 shared expert, FP8 e4m3 weights with fp32 128x128 scales:
route -> 1x128 act quant -> permute -> grouped gate/up (+SiLU*mul*w, requant)
-> grouped down -> ordered combine.  Inputs and weights are resident in HBM
before the timed region.  Also measured (reported under "extra"): the decode
configs (T = 64/256/512, Zipf(1.1) expert load), the dense FP8 GEMM
(M = 16..4096, N = 4096, K = 7168), the FP8 x MXFP4 variants, the power-of-two
(e8m0) weight-scale format with both scales applied in the MFMA, the router gate,
the FP8 KV pack (65536 rows, 656-byte layout) + sparse-MLA gather-dequant
(128 queries x 2048 rows), and the sparse attention straight off the packed
FP8 pages (64 heads; 128 queries x 2048 rows, and a 32-sequence decode batch
with 640 rows each).

Prints ONE JSON line.  ``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "sglang-lite_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "FP8 MoE layer tokens/s + % FP8 MFMA peak (prefill) / % HBM BW (decode), 1 GPU"
PEAK_FP8_TFLOPS = 5000.0   # MI355X dense FP8 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
H, I, E, K_TOP = 4096, 2048, 256, 8
SCALE_BYTES_PER_EXPERT = 4 * (2 * (I // 128) * (H // 128) + (H // 128) * (I // 128))  # 6144
W_BYTES_PER_EXPERT = 3 * H * I


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-extra", action="store_true", help="headline prefill line only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-kernels", nargs="?", const="fp8",
                    choices=("fp8", "fp4", "small", "frag", "fp4frag", "attn"),
                    help="for rocprofv3 runs: only 3 prefill steps (fp8: FP8 experts; fp4: FP4 "
                         "routed experts in the ue8m0 scale mode; frag / fp4frag: the same with "
                         "fragment-layout weight copies, then 3 decode steps at T = 64/256/512; "
                         "small: the short kernels; attn: the sparse attention off packed pages "
                         "at 128 x 2048 and decode 32 x 640, 5 calls each) plus a "
                         "counter-calibration kernel; prints no JSON")
    return ap.parse_args()


# ------------------------------------------------------------------ weights


def make_weights(torch, M, dev, seed=4, ue8m0=False):
    """256 routed + 1 shared FP8 experts: N(0, 0.02) fp32 drawn on the GPU from a
    seeded generator, quantized 128x128 by the library's weight-quant kernel
    (``ue8m0``: power-of-two scales, the e8m0 form of deepseek_infer/model.py:138-142)."""
    from sglang_lite_amd import kernel as K

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    n = E + 1
    w13 = torch.empty(n, 2, I, H, dtype=torch.float8_e4m3fn, device=dev)
    s13 = torch.empty(n, 2, I // 128, H // 128, dtype=torch.float32, device=dev)
    w2 = torch.empty(n, H, I, dtype=torch.float8_e4m3fn, device=dev)
    s2 = torch.empty(n, H // 128, I // 128, dtype=torch.float32, device=dev)
    for e in range(n):
        for j in range(2):
            q, s = K.per_block_cast_to_fp8(torch.randn(I, H, generator=g, device=dev) * 0.02, ue8m0)
            w13[e, j].copy_(q)
            s13[e, j].copy_(s)
        q, s = K.per_block_cast_to_fp8(torch.randn(H, I, generator=g, device=dev) * 0.02, ue8m0)
        w2[e].copy_(q)
        s2[e].copy_(s)
    experts = [(w13[e, 0], w13[e, 1], w2[e], s13[e, 0], s13[e, 1], s2[e]) for e in range(E)]
    shared = (w13[E, 0], w13[E, 1], w2[E], s13[E, 0], s13[E, 1], s2[E])
    table = M.ExpertTable.build(experts, shared)
    return table, (w13, s13, w2, s2)


def frag_table(M, weights):
    """The same 257 FP8 experts with fragment-layout copies of their weights
    (ExpertTable frag_layout: the register-fed prefill GEMMs)."""
    w13, s13, w2, s2 = weights
    experts = [(w13[e, 0], w13[e, 1], w2[e], s13[e, 0], s13[e, 1], s2[e]) for e in range(E)]
    shared = (w13[E, 0], w13[E, 1], w2[E], s13[E, 0], s13[E, 1], s2[E])
    return M.ExpertTable.build(experts, shared, frag_layout=True)


def make_fp4_weights(torch, M, dev, shared, seed=6, frag_layout=False):
    """256 routed MXFP4 experts (the reference's live routed format: packed
    e2m1 codes drawn uniformly, e8m0 1x32 scales in [2^-9, 2^-5]) plus the
    given FP8 shared expert; with frag_layout the table also carries
    fragment-layout copies (the register-fed GEMMs)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    u8 = torch.uint8
    w13 = torch.randint(0, 256, (E, 2, I, H // 2), dtype=u8, device=dev, generator=g)
    s13 = torch.randint(118, 123, (E, 2, I, H // 32), dtype=u8, device=dev, generator=g)
    w2 = torch.randint(0, 256, (E, H, I // 2), dtype=u8, device=dev, generator=g)
    s2 = torch.randint(118, 123, (E, H, I // 32), dtype=u8, device=dev, generator=g)
    e8 = torch.float8_e8m0fnu
    experts = [(w13[e, 0], w13[e, 1], w2[e], s13[e, 0].view(e8), s13[e, 1].view(e8), s2[e].view(e8))
               for e in range(E)]
    return M.ExpertTable.build(experts, shared, frag_layout=frag_layout)


def zipf_logits(torch, T, seed, s=1.1):
    g = torch.Generator().manual_seed(seed)
    p = torch.arange(1, E + 1, dtype=torch.float64) ** -s
    p /= p.sum()
    perm = torch.randperm(E, generator=g)
    logp = torch.log(p)[torch.argsort(perm)]
    u = torch.rand(T, E, generator=g, dtype=torch.float64).clamp_min(1e-300)
    gumbel = -torch.log(-torch.log(u))
    return (logp[None, :] + gumbel).float()


# ------------------------------------------------------------------- timing


def time_steps(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def event_avg_ms(torch, fn, iters, flush=None):
    """Average duration of fn on torch's current stream (the stream the
    library launches on), timed with HIP events, optional cache flush between.
    One untimed call first, so an output the allocator has to map for the
    first call is not inside the average."""
    fn()
    torch.cuda.synchronize()
    tot = 0.0
    for _ in range(iters):
        if flush is not None:
            flush()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        tot += a.elapsed_time(b)
    return tot / iters


def graph_ms(torch, fn, iters=20, warmup=3):
    """Device time per call of ``fn`` captured into a HIP graph and replayed
    back to back between two events: the launch-bound decode path as a
    serving loop runs it (the reference's decode runner captures the model the
    same way, engine/v4_runner/cuda_graph.py:98-137), without the Python and
    ctypes launch overhead that paces an eager loop."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        g.replay()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / iters


def replay_ms(torch, calls, reps=8):
    """Device time per call of ``calls`` run back to back, captured into one
    HIP graph and replayed ``reps`` times between two events: a serving loop's
    view of a short kernel, free of the ~12 us an event pair around a single
    small launch measures even for an empty kernel.  ``calls`` rotate input
    sets larger together than the 256 MB memory-side cache, so each call reads
    its inputs from HBM."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fn in calls:  # allocations and per-stream workspaces before capture
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for fn in calls:
            fn()
    g.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / (reps * len(calls))


class Prefill:
    """The staged prefill pipeline with events around each stage."""

    def __init__(self, torch, M, K, table, T, dev, seed, mode=0):
        self.torch, self.M, self.K, self.table, self.T = torch, M, K, table, T
        self.mode = mode  # sgl_scale_mode of the activation quant
        g = torch.Generator().manual_seed(seed)
        self.x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
        self.logits = torch.randn(T, E, generator=g).to(dev)
        self.ws = M.MoEWorkspace()
        self.y = torch.empty(T, H, dtype=torch.bfloat16, device=dev)

    def step(self):
        w, ids = self.M.route_topk(self.logits, K_TOP)
        self.M.moe_forward(self.x, ids, w, self.table, workspace=self.ws, out=self.y,
                           scale_mode=self.mode)
        return ids

    def staged(self, iters):
        torch, M, K = self.torch, self.M, self.K
        names = ["route", "act_quant", "permute", "gate_up", "down", "combine"]
        tot = {n: 0.0 for n in names}
        for _ in range(iters):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
            ev[0].record()
            w, ids = M.route_topk(self.logits, K_TOP)
            ev[1].record()
            xq, xs = K.act_quant(self.x, scale_mode=self.mode)
            ev[2].record()
            _, offsets, sorted_slot, _ = M.permute(ids, E)
            ev[3].record()
            hq, hs = M.gate_up(xq, xs, offsets, sorted_slot, w.reshape(-1), self.table, K_TOP,
                               scale_mode=self.mode)
            ev[4].record()
            out = M.down(hq, hs, offsets, sorted_slot, self.table, self.T, K_TOP,
                         scale_mode=self.mode)
            ev[5].record()
            M.combine(out, ids, True)
            ev[6].record()
            ev[6].synchronize()
            for i, n in enumerate(names):
                tot[n] += ev[i].elapsed_time(ev[i + 1])
        return {n: v / iters for n, v in tot.items()}


def hbm_ceiling(torch, dev):
    """HBM rates a plain streaming kernel reaches on this GPU (sgl_hbm_stream:
    16-byte accesses, four in flight per lane, 2048 x 512 threads), beside the
    8 TB/s nominal the fractions are quoted against: a copy (read + write) and
    a read of 2 GiB, and a read of 29.4 MB (the dense GEMM's weight) rotating
    over 12 buffers, each graph-replayed back to back."""
    from sglang_lite_amd import _lib

    out = {}
    sums = torch.empty(2048, dtype=torch.int32, device=dev)

    def stream(src, dst):
        _lib.call("sgl_hbm_stream", src.data_ptr(), dst.data_ptr() if dst is not None else None,
                  src.numel(), sums.data_ptr(), _lib.stream_of(src))

    a = torch.ones(1 << 31, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    ms = replay_ms(torch, [lambda: stream(a, b)] * 3, reps=4)
    out["copy_2GiB_gbs"] = round(2 * a.numel() / ms / 1e6, 1)
    ms = replay_ms(torch, [lambda: stream(a, None)] * 3, reps=4)
    out["read_2GiB_gbs"] = round(a.numel() / ms / 1e6, 1)
    del a, b
    bufs = [torch.ones(4096 * 7168, dtype=torch.uint8, device=dev) for _ in range(12)]
    ms = replay_ms(torch, [lambda x=x: stream(x, None) for x in bufs], reps=8)
    out["read_29MB_gbs"] = round(4096 * 7168 / ms / 1e6, 1)
    out["read_29MB_us"] = round(ms * 1e3, 2)
    return out


def mfma_ceiling(torch, dev, iters=2000):
    """MFMA rates of the GEMMs' inner-loop instruction mix on this GPU
    (sgl_mfma_mix: 4 x 4 blocks of 16x16x128 FP8 MFMAs per wavefront from
    registers, two wavefronts per SIMD on every CU), beside the 5.0 PF/s
    nominal: accumulating in the MFMA (the power-of-two-scale path) and with
    each block partial promoted by 4 fp32 FMAs (the fp32-scale path)."""
    from sglang_lite_amd import _lib

    threads = _lib.load().sgl_mfma_mix_threads()
    out = torch.empty(threads, dtype=torch.float32, device=dev)
    res = {}
    for v, name in ((0, "mfma_only_tflops"), (1, "mfma_plus_fp32_promotion_tflops")):
        run = lambda n, v=v: _lib.call("sgl_mfma_mix", v, out.data_ptr(), n, _lib.stream_of(out))  # noqa: E731
        run(10)
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        run(iters)
        b.record()
        b.synchronize()
        flops = (threads // 64) * iters * 16 * 65536.0
        res[name] = round(flops / a.elapsed_time(b) / 1e9, 1)
    return res


def profile_attn(torch, KVP, dev):
    """The sparse attention of the bench extras, 5 calls per shape, for kernel
    traces: 128 query tokens x 2048 rows of one 65536-row packed cache, then
    32 sequences x 640 rows, each of its own 32768-row cache (64 heads)."""
    from sglang_lite_amd import v4_sparse_mla as SA

    ga = torch.Generator().manual_seed(6)
    kva = torch.randn(65536, 512, generator=ga).to(torch.bfloat16).to(dev)
    pages_a = KVP.pack_dsv4_kv_paged(kva, 64).unsqueeze(0)
    del kva
    qa = torch.randn(1, 128, 64, 512, generator=ga).to(torch.bfloat16).to(dev)
    ia = torch.stack([torch.randperm(65536, generator=ga)[:2048] for _ in range(128)]).to(
        torch.int32).view(1, 128, 2048).to(dev)
    sink = torch.randn(64, generator=ga).to(dev)
    for _ in range(5):
        SA.sparse_attn_packed(qa, pages_a, sink, ia, 512 ** -0.5)
    torch.cuda.synchronize()
    del pages_a, qa, ia
    Bd, NRd, Kd = 32, 32768, 640
    kvd = torch.randn(Bd * NRd, 512, generator=ga).to(torch.bfloat16).to(dev)
    pages_d = KVP.pack_dsv4_kv_paged(kvd, 64).view(Bd, NRd // 64, 1, 64, 584)
    del kvd
    qd = torch.randn(Bd, 1, 64, 512, generator=ga).to(torch.bfloat16).to(dev)
    idd = torch.randint(0, NRd, (Bd, 1, Kd), generator=ga).to(torch.int32).to(dev)
    for _ in range(5):
        SA.sparse_attn_packed(qd, pages_d, sink, idd, 512 ** -0.5)
    torch.cuda.synchronize()


def profile_small(torch, M, K, table, dev):
    """The short kernels for a profiler run (--profile-kernels small), three
    launches each: the decode layers (T = 64 / 256 / 512, Zipf(1.1) load), the
    dense GEMM at M = 16 / 32 / 64 / 128 (N = 4096, K = 7168) over 12 rotating
    weight copies (three rounds; M = 4096 one round), the same GEMM in the
    live format (e8m0 weight and activation scales) at M = 128 / 1024 / 4096
    (one round), act_quant 4096 x 7168, the KV packs (65536 rows), and the
    router gate (projection + sqrtsoftplus/bias top-k, E = 256) at T = 64 /
    512 / 2048 / 8192."""
    from sglang_lite_amd import dsv4_kv_pack as KVP

    for Td, seed in ((64, 31), (256, 32), (512, 33)):
        logits = zipf_logits(torch, Td, seed).to(dev)
        xd = torch.randn(Td, H, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(dev)
        ws = M.MoEWorkspace()
        for _ in range(3):
            w, ids = M.route_topk(logits, K_TOP)
            M.moe_forward(xd, ids, w, table, workspace=ws)
    torch.cuda.synchronize()
    gg = torch.Generator(device=dev).manual_seed(8)
    wr = (torch.randn(E, H, generator=gg, device=dev) * H ** -0.5).to(torch.bfloat16)
    br = torch.randn(E, generator=gg, device=dev) * 0.05
    for Tg in (64, 512, 2048, 8192):
        xg = torch.randn(Tg, H, generator=gg, device=dev).to(torch.bfloat16)
        lg = torch.empty(Tg, E, dtype=torch.float32, device=dev)
        for _ in range(3):
            M.gate(xg, wr, K_TOP, "sqrtsoftplus", br, 1.5, logits=lg)
    torch.cuda.synchronize()
    gw = torch.Generator(device=dev).manual_seed(2)
    bq, bs = K.per_block_cast_to_fp8(torch.randn(4096, 7168, generator=gw, device=dev) * 0.02, False)
    wsets = [(bq.clone(), bs.clone()) for _ in range(12)]
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        for Md in (16, 32, 64, 128, 4096):
            aq, as_ = K.act_quant(torch.randn(Md, 7168, generator=gw, device=dev).to(torch.bfloat16))
            c = torch.empty(Md, 4096, dtype=torch.bfloat16, device=dev)
            for i in range(3 * len(wsets) if Md <= 128 else len(wsets)):
                K.fp8_gemm(aq, as_, wsets[i % 12][0], wsets[i % 12][1], out=c)
        # the live format: e8m0 weight scales and ue8m0 activation scales as e8m0
        # bytes, M = 128 / 1024 / 4096, 12 calls each over 12 weight copies
        del wsets
        bq8, bs8f = K.per_block_cast_to_fp8(torch.randn(4096, 7168, generator=gw, device=dev) * 0.02, True)
        bs8 = (bs8f.view(torch.int32) >> 23).to(torch.uint8).view(torch.float8_e8m0fnu)
        wsets = [(bq8.clone(), bs8.clone()) for _ in range(12)]
        for Md in (128, 1024, 4096):
            aq, as8 = K.act_quant(torch.randn(Md, 7168, generator=gw, device=dev).to(torch.bfloat16), 128,
                                  "ue8m0", torch.float8_e8m0fnu)
            c = torch.empty(Md, 4096, dtype=torch.bfloat16, device=dev)
            for i in range(len(wsets)):
                K.fp8_gemm(aq, as8, wsets[i][0], wsets[i][1], out=c)
        xs = [torch.randn(4096, 7168, generator=gw, device=dev).to(torch.bfloat16) for _ in range(3)]
        for x in xs:
            K.act_quant(x)
    finally:
        torch.set_default_dtype(prev)
    gk = torch.Generator().manual_seed(5)
    kvb = [torch.randn(65536, 576, generator=gk).to(torch.bfloat16).to(dev) for _ in range(3)]
    kva = [torch.randn(65536, 512, generator=gk).to(torch.bfloat16).to(dev) for _ in range(3)]
    for x in kvb:
        KVP.pack_kv_latent_rope(x)
    for x in kva:
        KVP.pack_dsv4_kv_paged(x, 64)
    torch.cuda.synchronize()


def prefill_entry(torch, M, K, table, dev, args, mode):
    """The prefill layer (T = 8192) with ``table``: whole-step time and the
    staged gate/up and down rates."""
    T = 8192
    rows = T * K_TOP + T
    pre = Prefill(torch, M, K, table, T, dev, seed=4, mode=mode)
    ms = time_steps(torch, pre.step, args.steps, args.warmup)
    st = pre.staged(max(3, min(args.steps, 10)))
    gu = rows * 4.0 * H * I / (st["gate_up"] / 1e3) / 1e12
    dn = rows * 2.0 * H * I / (st["down"] / 1e3) / 1e12
    return {"tokens": T, "ms": round(ms, 4), "tokens_per_s": round(T / ms * 1e3, 1),
            "layer_tflops": round(moe_flops(rows) / (ms / 1e3) / 1e12, 2),
            "mfma_frac": round(moe_flops(rows) / (ms / 1e3) / 1e12 / PEAK_FP8_TFLOPS, 4),
            "gate_up_tflops": round(gu, 1), "down_tflops": round(dn, 1),
            "stages_ms": {k_: round(v, 4) for k_, v in st.items()}}


def pow2_extra(torch, M, K, dev, args):
    """The reference's live FP8 scale format: power-of-two (e8m0) 128x128
    weight scales (deepseek_infer/model.py:138-142) with ue8m0 activation
    scales (mode 3), both applied inside the MFMA with no fp32 promotion: the
    prefill layer with FP8 routed experts, and with FP4 routed experts beside
    the FP8 shared expert in that format (model.py:623-626)."""
    from sglang_lite_amd import _lib

    log("generating power-of-two-scaled FP8 expert weights on the device")
    table2, (w13, s13, w2, s2) = make_weights(torch, M, dev, seed=4, ue8m0=True)
    assert table2.fmt & _lib.EXPERT_POW2_SCALES
    out = {"fp8_prefill_mode3": prefill_entry(torch, M, K, table2, dev, args, 3)}
    log(f"pow2 fp8 prefill mode 3: {out['fp8_prefill_mode3']['ms']:.3f} ms")
    del table2
    # the same experts with fragment-layout weight copies (register-fed GEMMs)
    tf = frag_table(M, (w13, s13, w2, s2))
    out["fp8_prefill_mode3_frag_layout"] = prefill_entry(torch, M, K, tf, dev, args, 3)
    log(f"pow2 fp8 prefill mode 3, fragment layout: {out['fp8_prefill_mode3_frag_layout']['ms']:.3f} ms")
    del tf
    shared = (w13[E, 0], w13[E, 1], w2[E], s13[E, 0], s13[E, 1], s2[E])
    table4 = make_fp4_weights(torch, M, dev, shared)
    assert table4.fmt & _lib.EXPERT_POW2_SCALES
    out["fp4_prefill_mode3"] = prefill_entry(torch, M, K, table4, dev, args, 3)
    log(f"pow2 fp4 prefill mode 3: {out['fp4_prefill_mode3']['ms']:.3f} ms")
    return out


def fp4_extra(torch, M, K, weights, dev, args, flush):
    """FP8 x MXFP4 (the reference's live routed-expert format): the MoE layer
    at the prefill and decode shapes with FP4 routed experts and the FP8
    shared expert, in fp32-scale mode 0 and the live ue8m0 mode 3 (scales
    applied inside the MFMA), and the dense FP8 x FP4 GEMM (N=4096, K=7168)."""
    w13, s13, w2, s2 = weights
    shared = (w13[E, 0], w13[E, 1], w2[E], s13[E, 0], s13[E, 1], s2[E])
    log("generating FP4 expert weights on the device")
    table4 = make_fp4_weights(torch, M, dev, shared)
    out = {"flops_note": "mixed fp8 x fp4 MFMA runs at the fp8 rate: peak 5.0 PF dense"}
    T = 8192
    rows = T * K_TOP + T
    for mode in (0, 3):
        pre = Prefill(torch, M, K, table4, T, dev, seed=4, mode=mode)
        ms = time_steps(torch, pre.step, args.steps, args.warmup)
        st = pre.staged(max(3, min(args.steps, 10)))
        gu = rows * 4.0 * H * I / (st["gate_up"] / 1e3) / 1e12
        dn = rows * 2.0 * H * I / (st["down"] / 1e3) / 1e12
        out[f"prefill_mode{mode}"] = {
            "tokens": T, "ms": round(ms, 4), "tokens_per_s": round(T / ms * 1e3, 1),
            "layer_tflops": round(moe_flops(rows) / (ms / 1e3) / 1e12, 2),
            "mfma_frac": round(moe_flops(rows) / (ms / 1e3) / 1e12 / PEAK_FP8_TFLOPS, 4),
            "gate_up_tflops": round(gu, 1), "down_tflops": round(dn, 1),
            "stages_ms": {k_: round(v, 4) for k_, v in st.items()}}
        if mode == 3:
            out["prefill_mode3"]["gate_up_traffic_bytes"] = read_traffic("moe_fp4_gate_up_prefill")
        log(f"fp4 prefill mode {mode}: {ms:.3f} ms, gate_up {gu:.0f} TF, down {dn:.0f} TF")
    wb = 3 * I * H // 2 + 3 * I * H // 32  # packed e2m1 + e8m0 bytes per routed expert
    sb_ = 3 * I * H + 3 * 4 * (I // 128) * (H // 128)  # the FP8 shared expert

    def decode_lines(tab, what):
        dec = []
        for Td, seed in ((64, 31), (256, 32), (512, 33)):
            logits = zipf_logits(torch, Td, seed).to(dev)
            xd = torch.randn(Td, H, generator=torch.Generator().manual_seed(seed)).to(
                torch.bfloat16).to(dev)
            ws = M.MoEWorkspace()
            yd = torch.empty(Td, H, dtype=torch.bfloat16, device=dev)

            def dstep():
                w, ids = M.route_topk(logits, K_TOP)
                M.moe_forward(xd, ids, w, tab, workspace=ws, out=yd, scale_mode=3)

            msd = time_steps(torch, dstep, max(args.steps, 10), args.warmup)
            msg_d = graph_ms(torch, dstep, max(args.steps, 10))
            _, ids = M.route_topk(logits, K_TOP)
            touched = int(torch.unique(ids).numel())
            by = touched * wb + sb_ + 4 * Td * H + 4 * Td * E
            dec.append({"tokens": Td, "ms": round(msd, 4), "tokens_per_s": round(Td / msd * 1e3, 1),
                        "experts_touched": touched, "bytes": by, "gbs": round(by / msd / 1e6, 1),
                        "hbm_frac": round(by / msd / 1e6 / PEAK_HBM_GBS, 4),
                        "graph_ms": round(msg_d, 4),
                        "graph_hbm_frac": round(by / msg_d / 1e6 / PEAK_HBM_GBS, 4)})
            log(f"fp4 decode{what} T={Td}: {msd:.3f} ms, graph {msg_d:.3f} ms, "
                f"{by / msg_d / 1e6:.0f} GB/s")
        return dec

    dec = decode_lines(table4, "")
    out["decode_mode3"] = dec
    # the same routed experts with fragment-layout copies (register-fed GEMMs)
    del table4
    table4f = make_fp4_weights(torch, M, dev, shared, frag_layout=True)
    pre = Prefill(torch, M, K, table4f, T, dev, seed=4, mode=3)
    ms = time_steps(torch, pre.step, args.steps, args.warmup)
    st = pre.staged(max(3, min(args.steps, 10)))
    out["prefill_mode3_frag_layout"] = {
        "tokens": T, "ms": round(ms, 4), "tokens_per_s": round(T / ms * 1e3, 1),
        "stages_ms": {k_: round(v, 4) for k_, v in st.items()}}
    log(f"fp4 prefill mode 3 with fragment-layout copies: {ms:.3f} ms")
    out["decode_mode3_frag_layout"] = decode_lines(table4f, " (fragment layout)")
    del table4f
    gw = torch.Generator(device=dev).manual_seed(7)
    bq = torch.randint(0, 256, (4096, 3584), dtype=torch.uint8, device=dev, generator=gw)
    bs = torch.randint(118, 123, (4096, 224), dtype=torch.uint8, device=dev,
                       generator=gw).view(torch.float8_e8m0fnu)
    # 20 copies of the weight (311 MB): each back-to-back call streams a cold B
    wsets = [(bq.clone(), bs.clone()) for _ in range(20)]
    dense = []
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        for Md in (16, 128, 1024, 4096):
            a = torch.randn(Md, 7168, generator=gw, device=dev).to(torch.bfloat16)
            for pow2 in (False, True):
                aq, as_ = K.act_quant(a, scale_mode=3 if pow2 else 0)
                c = torch.empty(Md, 4096, dtype=torch.bfloat16, device=dev)
                fn = lambda: K.fp4_gemm(aq, as_, bq, bs, out=c, a_scale_pow2=pow2)  # noqa: E731
                for _ in range(2):
                    fn()
                msg = replay_ms(torch, [lambda w=w, pow2=pow2: K.fp4_gemm(aq, as_, w[0], w[1], out=c,
                                                                             a_scale_pow2=pow2)
                                        for w in wsets])
                fl = 2.0 * Md * 4096 * 7168
                byt = Md * 7168 + 4 * Md * 56 + 4096 * 3584 + 4096 * 224 + 2 * Md * 4096
                dense.append({"M": Md, "N": 4096, "K": 7168, "a_scale_pow2": pow2,
                              "ms": round(msg, 5), "tflops": round(fl / msg / 1e9, 2),
                              "mfma_frac": round(fl / msg / 1e9 / PEAK_FP8_TFLOPS, 4),
                              "gbs": round(byt / msg / 1e6, 1),
                              "hbm_frac": round(byt / msg / 1e6 / PEAK_HBM_GBS, 4)})
                log(f"fp4 dense M={Md} pow2={pow2}: {msg * 1e3:.1f} us")
    finally:
        torch.set_default_dtype(prev)
    del wsets
    out["dense_gemm"] = dense
    return out


def moe_flops(rows):
    return rows * 6.0 * H * I  # gate+up (4HI) + down (2HI) per routed/shared row


def read_traffic(kernel_tag):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(ROOT, "profiles", f"{kernel_tag}_pmc.txt")
    if not os.path.isfile(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1].split()[0])
    return None


# ------------------------------------------------------------- cpu baseline


def cpu_model() -> str:
    """The host CPU's model string (/proc/cpuinfo), else what platform reports."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(torch, weights, pre, workers=None):
    """The oracle (numpy restatement of the reference MoE layer) timed on the
    host over the WHOLE prefill layer of the GPU workload: softmax top-8 routing
    of the same logits (oracle.moe.route_topk), then oracle.moe.moe_forward --
    per activated expert the row gather, 1x128 act quant, dequantize-to-fp32
    gate/up GEMMs (float64 BLAS), SwiGLU x routing weight, 1x128 requant and
    down GEMM, for all 256 routed experts and the shared one, and the
    ascending-expert fp32 combine.  Experts run on ``workers`` threads with one
    BLAS thread each; the weights are on the host before the clock starts
    (as they are in HBM for the GPU)."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import moe as OM

    w13, s13, w2, s2 = weights
    torch.cuda.synchronize()
    workers = workers or max(1, min(os.cpu_count() or 1, 16))
    logits = pre.logits.cpu().numpy()
    x_np = pre.x.float().cpu().numpy()

    def expert_np(e):
        return {"w1": w13[e, 0].view(torch.uint8).cpu().numpy(),
                "w3": w13[e, 1].view(torch.uint8).cpu().numpy(),
                "w2": w2[e].view(torch.uint8).cpu().numpy(),
                "s1": s13[e, 0].cpu().numpy(), "s3": s13[e, 1].cpu().numpy(),
                "s2": s2[e].cpu().numpy()}

    experts = [expert_np(e) for e in range(E)]
    shared = expert_np(E)
    blas = [f"{i['internal_api']}" for i in threadpool_info() if i.get("user_api") == "blas"]
    runs = []
    with threadpool_limits(limits=1, user_api="blas"):
        for _ in range(3):
            t0 = time.perf_counter()
            w, ids = OM.route_topk(logits, K_TOP)
            y = OM.moe_forward(x_np, ids, w, experts, shared, workers=workers)
            runs.append(time.perf_counter() - t0)
    dt = sorted(runs)[1]  # the median of three runs
    # cross-check: the host layer against the device layer of the same inputs
    y_dev = pre.y.float().cpu().numpy()
    rel = float(np.linalg.norm(y_dev - y) / max(np.linalg.norm(y), 1e-30))
    del experts, shared
    return {
        "value": round(pre.T / dt, 3),
        "unit": "tokens/s",
        "cores": workers,
        "kind": "port",
        "sample": (f"the whole T={pre.T} prefill layer, median of three runs "
                   f"({', '.join(f'{r:.1f}' for r in runs)} s): the oracle -- a numpy restatement "
                   f"of the reference's torch path, not the reference itself -- route_topk + "
                   f"moe_forward over all {E} routed experts and the shared one (gather, act "
                   f"quant, dequantize-to-fp32 GEMMs in float64 BLAS, SwiGLU, requant, ascending "
                   f"fp32 combine), experts on {workers} threads x 1 BLAS thread"),
        "seconds": round(dt, 2),
        "seconds_runs": [round(r, 2) for r in runs],
        "host_cpu": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "blas": blas,
        "blas_threads_per_worker": 1,
        "rel_l2_vs_gpu_layer": round(rel, 6),
    }


# --------------------------------------------------------------------- main


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    import sglang_lite_amd
    from sglang_lite_amd import dsv4_kv_pack as KVP
    from sglang_lite_amd import kernel as K
    from sglang_lite_amd import moe as M

    info = sglang_lite_amd.probe()
    if not info["ok"]:
        raise SystemExit(f"sglang_lite_amd probe failed: {info}")
    dev = torch.device("cuda:0")
    log("generating FP8 expert weights on the device")
    table, weights = make_weights(torch, M, dev)
    T = 8192
    pre = Prefill(torch, M, K, table, T, dev, seed=4)

    if args.profile_kernels:
        if args.profile_kernels == "fp4":
            w13, s13, w2, s2 = weights
            shared = (w13[E, 0], w13[E, 1], w2[E], s13[E, 0], s13[E, 1], s2[E])
            pre = Prefill(torch, M, K, make_fp4_weights(torch, M, dev, shared), T, dev, seed=4,
                          mode=3)
        if args.profile_kernels == "fp4frag":
            # FP4 routed experts with fragment-layout copies, ue8m0 mode 3: 3
            # prefill steps, then 3 decode steps each at T = 64 / 256 / 512
            w13, s13, w2, s2 = weights
            shared = (w13[E, 0], w13[E, 1], w2[E], s13[E, 0], s13[E, 1], s2[E])
            tf = make_fp4_weights(torch, M, dev, shared, frag_layout=True)
            pre = Prefill(torch, M, K, tf, T, dev, seed=4, mode=3)
            for _ in range(3):
                pre.step()
            for Td, seed in ((64, 31), (256, 32), (512, 33)):
                logits = zipf_logits(torch, Td, seed).to(dev)
                xd = torch.randn(Td, H, generator=torch.Generator().manual_seed(seed)).to(
                    torch.bfloat16).to(dev)
                for _ in range(3):
                    w, ids = M.route_topk(logits, K_TOP)
                    M.moe_forward(xd, ids, w, tf, scale_mode=3)
        elif args.profile_kernels == "frag":
            # fragment-layout weight copies: 3 prefill steps, then 3 decode
            # steps each at T = 64 / 256 / 512 (Zipf load)
            tf = frag_table(M, weights)
            pre = Prefill(torch, M, K, tf, T, dev, seed=4)
            for _ in range(3):
                pre.step()
            for Td, seed in ((64, 31), (256, 32), (512, 33)):
                logits = zipf_logits(torch, Td, seed).to(dev)
                xd = torch.randn(Td, H, generator=torch.Generator().manual_seed(seed)).to(
                    torch.bfloat16).to(dev)
                for _ in range(3):
                    w, ids = M.route_topk(logits, K_TOP)
                    M.moe_forward(xd, ids, w, tf)
        elif args.profile_kernels == "small":
            profile_small(torch, M, K, table, dev)
        elif args.profile_kernels == "attn":
            profile_attn(torch, KVP, dev)
        else:
            for _ in range(3):
                pre.step()
        # counter calibration: e8m0_to_f32 over 64 MiB reads 64 MiB, writes 256 MiB
        src = torch.full((64 << 20,), 127, dtype=torch.uint8, device=dev).view(torch.float8_e8m0fnu)
        for _ in range(3):
            K.e8m0_to_f32(src)
        torch.cuda.synchronize()
        log("profile-kernels run done")
        return

    log(f"prefill T={T}: warmup {args.warmup}, timed {args.steps}")
    ms = time_steps(torch, pre.step, args.steps, args.warmup)
    stages = pre.staged(max(3, min(args.steps, 10)))
    mix = mfma_ceiling(torch, dev)
    log(f"MFMA instruction-mix ceilings: {mix}")
    rows = T * K_TOP + T
    flops = moe_flops(rows)
    gu_flops = rows * 4.0 * H * I
    gu_ms = stages["gate_up"]
    n_experts_touched = E
    layer_bytes = (n_experts_touched + 1) * (W_BYTES_PER_EXPERT + SCALE_BYTES_PER_EXPERT) + \
        4 * T * H + 4 * T * E
    tok_s = T / (ms / 1e3)
    traffic = read_traffic("moe_gate_up_prefill")
    # algorithmic bytes of one gate/up launch: every expert's w1 | w3 and
    # scales, the quantized activations and scales, h and its scales written
    n_mt = H // 128
    gu_bytes = (E + 1) * (2 * I * H + 2 * (I // 128) * n_mt * 4) + T * H + T * n_mt * 4 + \
        rows * I + rows * (I // 128) * 4
    t_mfma = gu_flops / (PEAK_FP8_TFLOPS * 1e12)
    t_hbm = gu_bytes / (PEAK_HBM_GBS * 1e9)
    bound = "hbm" if t_hbm >= t_mfma else "mfma"
    gu_tflops = gu_flops / (gu_ms / 1e3) / 1e12
    gu_gbs = gu_bytes / (gu_ms / 1e3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic (seeded N(0,1) bf16 activations and router logits; N(0,0.02) weights "
                "drawn on the GPU and quantized 128x128)",
        "config": {"workload": "moe_prefill_T8192_H4096_I2048_E256_top8_shared1",
                   "tokens": T, "hidden": H, "expert_inter": I, "experts": E, "topk": K_TOP,
                   "shared_experts": 1, "router": "softmax over N(0,1) logits",
                   "parallelism": "none (1 GPU)"},
        "layer": {"tflops": round(flops / (ms / 1e3) / 1e12, 2),
                  "mfma_frac": round(flops / (ms / 1e3) / 1e12 / PEAK_FP8_TFLOPS, 4),
                  "hbm_gbs_algorithmic": round(layer_bytes / (ms / 1e3) / 1e9, 1),
                  "hbm_frac": round(layer_bytes / (ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
                  "stages_ms": {k_: round(v, 4) for k_, v in stages.items()}},
        # the bound is whichever roof the launch's algorithmic work reaches
        # later: bytes / 8 TB/s or FLOPs / 5 PF/s
        "roofline": {"kernel": "gemm_pipe_kernel<gate_up> (grouped gate/up + SwiGLU + requant)",
                     "bound": bound,
                     "achieved": round(gu_gbs, 1) if bound == "hbm" else round(gu_tflops, 2),
                     "peak": PEAK_HBM_GBS if bound == "hbm" else PEAK_FP8_TFLOPS,
                     "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
                     "frac": round(gu_gbs / PEAK_HBM_GBS if bound == "hbm" else
                                   gu_tflops / PEAK_FP8_TFLOPS, 4),
                     "traffic": traffic,
                     "algorithmic_bytes_per_launch": gu_bytes, "flops_per_launch": gu_flops,
                     "hbm_frac": round(gu_gbs / PEAK_HBM_GBS, 4),
                     "mfma_frac": round(gu_tflops / PEAK_FP8_TFLOPS, 4),
                     "roof_us": {"hbm": round(t_hbm * 1e6, 1), "mfma": round(t_mfma * 1e6, 1)},
                     "avg_launch_ms": round(gu_ms, 4),
                     # the same launch against what this GPU's MFMAs reach with the
                     # fp32-scale promotion in the instruction stream (measured now)
                     "mix_ceiling": {**mix, "frac_of_fp32_promotion_ceiling": round(
                         gu_tflops / mix["mfma_plus_fp32_promotion_tflops"], 4)}},
    }
    log(f"prefill {ms:.3f} ms/step -> {tok_s:.0f} tok/s; stages {stages}")

    if not args.no_extra:
        extra = {}
        # ---- decode configs: the row-major expert table, and the same experts
        # with fragment-layout weight copies (register-fed GEMMs)
        def decode_lines(tab):
            dec = []
            for Td, seed in ((64, 31), (256, 32), (512, 33)):
                logits = zipf_logits(torch, Td, seed).to(dev)
                xd = torch.randn(Td, H, generator=torch.Generator().manual_seed(seed)).to(
                    torch.bfloat16).to(dev)
                ws = M.MoEWorkspace()
                yd = torch.empty(Td, H, dtype=torch.bfloat16, device=dev)

                def dstep():
                    w, ids = M.route_topk(logits, K_TOP)
                    M.moe_forward(xd, ids, w, tab, workspace=ws, out=yd)

                msd = time_steps(torch, dstep, max(args.steps, 10), args.warmup)
                msg_d = graph_ms(torch, dstep, max(args.steps, 10))
                _, ids = M.route_topk(logits, K_TOP)
                touched = int(torch.unique(ids).numel())
                by = (touched + 1) * (W_BYTES_PER_EXPERT + SCALE_BYTES_PER_EXPERT) + 4 * Td * H + \
                    4 * Td * E
                dec.append({"tokens": Td, "ms": round(msd, 4), "tokens_per_s": round(Td / msd * 1e3, 1),
                            "experts_touched": touched, "bytes": by,
                            "gbs": round(by / msd / 1e6, 1),
                            "hbm_frac": round(by / msd / 1e6 / PEAK_HBM_GBS, 4),
                            "graph_ms": round(msg_d, 4),
                            "graph_hbm_frac": round(by / msg_d / 1e6 / PEAK_HBM_GBS, 4)})
                log(f"decode T={Td}: {msd:.3f} ms eager, {msg_d:.3f} ms graph, touched {touched}, "
                    f"{by / msg_d / 1e6:.0f} GB/s (graph)")
            return dec

        extra["decode"] = decode_lines(table)
        tf = frag_table(M, weights)
        extra["decode_frag_layout"] = decode_lines(tf)
        del tf
        # ---- fused gate (router projection on bf16 MFMA + score + top-k), model.py:564-584
        gate = []
        gg = torch.Generator(device=dev).manual_seed(8)
        Wr = (torch.randn(E, H, generator=gg, device=dev) * H ** -0.5).to(torch.bfloat16)
        br = torch.randn(E, generator=gg, device=dev) * 0.05
        for Tg in (64, 512, 8192):
            xg = torch.randn(Tg, H, generator=gg, device=dev).to(torch.bfloat16)
            lg = torch.empty(Tg, E, dtype=torch.float32, device=dev)
            fn = lambda: M.gate(xg, Wr, K_TOP, "sqrtsoftplus", br, 1.5, logits=lg)  # noqa: E731
            msg = graph_ms(torch, fn, 20)
            byt = E * H * 2 + Tg * H * 2 + Tg * E * 4 + Tg * K_TOP * 8
            gate.append({"tokens": Tg, "graph_ms": round(msg, 5), "gbs": round(byt / msg / 1e6, 1),
                         "tflops": round(2.0 * Tg * H * E / msg / 1e9, 1)})
            log(f"gate T={Tg}: {msg * 1e3:.1f} us")
        extra["gate_sqrtsoftplus_bias"] = gate
        # ---- dense GEMM
        # cold-cache timing: read 512 MiB between runs so neither L2 nor the
        # memory-side cache holds the inputs.  A read, not a fill: a fill
        # leaves 512 MiB of dirty lines whose write-back would land inside
        # the next timed kernel.
        flush_buf = torch.ones(128 << 20, dtype=torch.float32, device=dev)
        flush_sink = torch.empty((), dtype=torch.float32, device=dev)

        def flush():
            torch.sum(flush_buf, dim=0, out=flush_sink)

        gw = torch.Generator(device=dev).manual_seed(2)
        bq, bs = K.per_block_cast_to_fp8(torch.randn(4096, 7168, generator=gw, device=dev) * 0.02,
                                         False)
        # 12 copies of the weight (353 MB): each back-to-back call streams a
        # cold B, as the 72-odd linears of a decode step do
        wsets = [(bq.clone(), bs.clone()) for _ in range(12)]
        dense = []
        prev = torch.get_default_dtype()
        torch.set_default_dtype(torch.bfloat16)
        try:
            for Md in (16, 32, 64, 128, 1024, 4096):
                a = torch.randn(Md, 7168, generator=gw, device=dev).to(torch.bfloat16)
                aq, as_ = K.act_quant(a)
                c = torch.empty(Md, 4096, dtype=torch.bfloat16, device=dev)
                for _ in range(2):
                    K.fp8_gemm(aq, as_, bq, bs, out=c)
                msg = replay_ms(torch, [lambda w=w: K.fp8_gemm(aq, as_, w[0], w[1], out=c) for w in wsets])
                mse = event_avg_ms(torch, lambda: K.fp8_gemm(aq, as_, bq, bs, out=c), 10, flush)
                fl = 2.0 * Md * 4096 * 7168
                byt = Md * 7168 + 4 * Md * 56 + 4096 * 7168 + 4 * 32 * 56 + 2 * Md * 4096
                dense.append({"M": Md, "N": 4096, "K": 7168, "ms": round(msg, 5),
                              "ms_single_call_events": round(mse, 5),
                              "tflops": round(fl / msg / 1e9, 2),
                              "mfma_frac": round(fl / msg / 1e9 / PEAK_FP8_TFLOPS, 4),
                              "gbs": round(byt / msg / 1e6, 1),
                              "hbm_frac": round(byt / msg / 1e6 / PEAK_HBM_GBS, 4)})
                log(f"dense M={Md}: {msg * 1e3:.1f} us back to back ({mse * 1e3:.1f} us single call)")
            del wsets
            # the live format (model.py:138-142,777-778): e8m0 weight scales and
            # ue8m0 act_quant scales as e8m0 bytes, read by the GEMM as they are;
            # the tiled kernels apply both inside the MFMA
            bq8, bs8f = K.per_block_cast_to_fp8(torch.randn(4096, 7168, generator=gw, device=dev) * 0.02,
                                                True)
            bs8 = (bs8f.view(torch.int32) >> 23).to(torch.uint8).view(torch.float8_e8m0fnu)
            wsets = [(bq8.clone(), bs8.clone()) for _ in range(12)]
            live = []
            for Md in (16, 128, 1024, 4096):
                a = torch.randn(Md, 7168, generator=gw, device=dev).to(torch.bfloat16)
                aq, as8 = K.act_quant(a, 128, "ue8m0", torch.float8_e8m0fnu)
                c = torch.empty(Md, 4096, dtype=torch.bfloat16, device=dev)
                for _ in range(2):
                    K.fp8_gemm(aq, as8, bq8, bs8, out=c)
                msg = replay_ms(torch, [lambda w=w: K.fp8_gemm(aq, as8, w[0], w[1], out=c) for w in wsets])
                fl = 2.0 * Md * 4096 * 7168
                byt = Md * 7168 + Md * 56 + 4096 * 7168 + 32 * 56 + 2 * Md * 4096
                live.append({"M": Md, "N": 4096, "K": 7168, "ms": round(msg, 5),
                             "tflops": round(fl / msg / 1e9, 2),
                             "mfma_frac": round(fl / msg / 1e9 / PEAK_FP8_TFLOPS, 4),
                             "gbs": round(byt / msg / 1e6, 1),
                             "hbm_frac": round(byt / msg / 1e6 / PEAK_HBM_GBS, 4)})
                log(f"dense e8m0 scales M={Md}: {msg * 1e3:.1f} us back to back")
            del wsets
            extra["dense_gemm_live_e8m0"] = live
            # act_quant alone at the largest dense shape, 6 rotating inputs (352 MB)
            xs6 = [torch.randn(4096, 7168, generator=gw, device=dev).to(torch.bfloat16) for _ in range(6)]
            msq = replay_ms(torch, [lambda x=x: K.act_quant(x) for x in xs6])
            del xs6
            qb = 3 * 4096 * 7168 + 4 * 4096 * 56
            extra["act_quant_4096x7168"] = {"ms": round(msq, 5), "gbs": round(qb / msq / 1e6, 1),
                                            "hbm_frac": round(qb / msq / 1e6 / PEAK_HBM_GBS, 4)}
        finally:
            torch.set_default_dtype(prev)
        extra["dense_gemm"] = dense
        # ---- KV pack (layout B, 65536 rows) + gather-dequant (128 x 2048)
        gk = torch.Generator().manual_seed(5)
        kv = torch.randn(65536, 576, generator=gk).to(torch.bfloat16).to(dev)
        packed = KVP.pack_kv_latent_rope(kv)
        kvs = [kv] + [kv.clone() for _ in range(3)]  # 4 x (75 + 43) MB through the pack
        msp = replay_ms(torch, [lambda x=x: KVP.pack_kv_latent_rope(x) for x in kvs])
        del kvs
        pb = 65536 * (1152 + 656)
        idx = torch.stack([torch.randperm(65536, generator=gk)[:2048] for _ in range(128)]).to(
            torch.int32).to(dev)
        out = torch.empty(128, 2048, 576, dtype=torch.bfloat16, device=dev)
        msg_ = replay_ms(torch, [lambda: KVP.gather_dequant(packed, idx, layout="B", out=out)] * 4)
        gb = 128 * 2048 * (656 + 1152)
        kva = torch.randn(65536, 512, generator=gk).to(torch.bfloat16).to(dev)
        kvas = [kva] + [kva.clone() for _ in range(3)]
        msa = replay_ms(torch, [lambda x=x: KVP.pack_dsv4_kv_paged(x, 64) for x in kvas])
        del kvas
        ab = 65536 * (1024 + 584)
        # gather-dequant of the same 128 x 2048 indices from layout A footer pages
        pages_ga = KVP.pack_dsv4_kv_paged(kva, 64)
        out_a = torch.empty(128, 2048, 512, dtype=torch.bfloat16, device=dev)
        msga = replay_ms(torch, [lambda: KVP.gather_dequant(pages_ga, idx, layout="A", page_size=64,
                                                             out=out_a)] * 4)
        gab = 128 * 2048 * (584 + 1024)
        extra["kv"] = {
            "pack_layout_b_65536": {"ms": round(msp, 5), "gbs": round(pb / msp / 1e6, 1),
                                    "hbm_frac": round(pb / msp / 1e6 / PEAK_HBM_GBS, 4)},
            "gather_dequant_128x2048": {"ms": round(msg_, 5), "gbs": round(gb / msg_ / 1e6, 1),
                                        "hbm_frac": round(gb / msg_ / 1e6 / PEAK_HBM_GBS, 4)},
            "pack_layout_a_paged_65536": {"ms": round(msa, 5), "gbs": round(ab / msa / 1e6, 1),
                                          "hbm_frac": round(ab / msa / 1e6 / PEAK_HBM_GBS, 4)},
            "gather_dequant_a_paged_128x2048": {"ms": round(msga, 5), "gbs": round(gab / msga / 1e6, 1),
                                                "hbm_frac": round(gab / msga / 1e6 / PEAK_HBM_GBS, 4)},
        }
        log(f"kv pack {msp * 1e3:.1f} us, gather {msg_ * 1e3:.1f} us, pack A paged {msa * 1e3:.1f} us")
        # ---- sparse MLA attention straight off the packed FP8 pages (64 heads,
        # 128 query tokens x 2048 gathered rows of the 65536-row cache)
        from sglang_lite_amd import v4_sparse_mla as SA
        ga = torch.Generator().manual_seed(6)
        qa = torch.randn(1, 128, 64, 512, generator=ga).to(torch.bfloat16).to(dev)
        pages_a = KVP.pack_dsv4_kv_paged(kva, 64).unsqueeze(0)
        ia = torch.stack([torch.randperm(65536, generator=ga)[:2048] for _ in range(128)]).to(
            torch.int32).view(1, 128, 2048).to(dev)
        sink_a = torch.randn(64, generator=ga).to(dev)
        fa = lambda: SA.sparse_attn_packed(qa, pages_a, sink_a, ia, 512 ** -0.5)  # noqa: E731
        fa()
        msa_ = event_avg_ms(torch, fa, 10, flush)
        gsa_ = graph_ms(torch, fa)
        ab_ = 128 * 2048 * 584 + 2 * 128 * 64 * 512 * 2 + 128 * 2048 * 4
        afl = 4.0 * 128 * 64 * 2048 * 512
        extra["sparse_attn_packed_128x2048_h64"] = {
            "ms": round(msa_, 5), "graph_ms": round(gsa_, 5), "gbs": round(ab_ / gsa_ / 1e6, 1),
            "hbm_frac": round(ab_ / gsa_ / 1e6 / PEAK_HBM_GBS, 4),
            "tflops": round(afl / gsa_ / 1e9, 1),
            "mfma_frac_bf16": round(afl / gsa_ / 1e9 / 2500.0, 4)}
        log(f"sparse attn packed 128x2048: {msa_ * 1e3:.1f} us eager, {gsa_ * 1e3:.1f} us graph")
        del pages_a, qa, ia
        # decode: 32 sequences, one query token each, 640 gathered rows (top-k
        # 512 + window 128) from each sequence's own 32768-row packed cache
        # (612 MB in all, larger than the on-die cache: the rows come from HBM)
        Bd, NRd, Kd = 32, 32768, 640
        kvd = torch.randn(Bd * NRd, 512, generator=ga).to(torch.bfloat16).to(dev)
        pages_d = KVP.pack_dsv4_kv_paged(kvd, 64).view(Bd, NRd // 64, 1, 64, 584)
        del kvd
        qd = torch.randn(Bd, 1, 64, 512, generator=ga).to(torch.bfloat16).to(dev)
        idd = torch.randint(0, NRd, (Bd, 1, Kd), generator=ga).to(torch.int32).to(dev)
        fd = lambda: SA.sparse_attn_packed(qd, pages_d, sink_a, idd, 512 ** -0.5)  # noqa: E731
        fd()
        msd = event_avg_ms(torch, fd, 10, flush)
        gsd = graph_ms(torch, fd)
        bd = Bd * Kd * 584 + 2 * Bd * 64 * 512 * 2 + Bd * Kd * 4
        extra["sparse_attn_packed_decode_b32_k640_h64"] = {
            "ms": round(msd, 5), "graph_ms": round(gsd, 5), "gbs": round(bd / gsd / 1e6, 1),
            "hbm_frac": round(bd / gsd / 1e6 / PEAK_HBM_GBS, 4)}
        log(f"sparse attn packed decode b32: {msd * 1e3:.1f} us eager, {gsd * 1e3:.1f} us graph")
        del pages_d, qd, idd
        extra["hbm_ceiling"] = hbm_ceiling(torch, dev)
        log(f"hbm ceiling: {extra['hbm_ceiling']}")
        # the headline layer with fragment-layout weight copies (register-fed GEMMs)
        tf = frag_table(M, weights)
        extra["prefill_frag_layout"] = prefill_entry(torch, M, K, tf, dev, args, 0)
        log(f"prefill, fragment layout: {extra['prefill_frag_layout']['ms']:.3f} ms")
        del tf
        extra["fp4"] = fp4_extra(torch, M, K, weights, dev, args, flush)
        extra["pow2_scales"] = pow2_extra(torch, M, K, dev, args)
        result["extra"] = extra

    if not args.no_cpu_baseline:
        log("cpu baseline: the oracle over the whole prefill layer")
        pre.step()
        result["cpu_baseline"] = cpu_baseline(torch, weights, pre)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
