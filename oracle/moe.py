"""Oracle: routing, permutation, FP8 GEMM and the MoE layer, restated in numpy.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import fp4 as F4
from . import quant as Q

# --------------------------------------------------------------- routing


def route_scores(logits: np.ndarray, score_func: str) -> np.ndarray:
    """deepseek_infer/model.py:566-571 (fp32)."""
    lg = np.asarray(logits, dtype=np.float32)
    if score_func == "softmax":
        m = lg.max(axis=-1, keepdims=True)
        e = np.exp((lg - m).astype(np.float32)).astype(np.float32)
        return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    if score_func == "sigmoid":
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-lg))).astype(np.float32)
    if score_func == "sqrtsoftplus":
        sp = np.where(lg > 20.0, lg, np.log1p(np.exp(np.minimum(lg, 20.0))))
        return np.sqrt(sp.astype(np.float32)).astype(np.float32)
    raise ValueError(score_func)


def route_topk(logits: np.ndarray, k: int, score_func: str = "softmax",
               bias: Optional[np.ndarray] = None, route_scale: float = 1.0
               ) -> Tuple[np.ndarray, np.ndarray]:
    """deepseek_infer/model.py:565-584 Gate.forward after the projection.

    Selection is topk over ``scores (+ bias)`` in descending order (torch.topk
    order), ties to the lower expert id.  Returns (weights f32 [T,k], ids int64 [T,k]).
    """
    scores = route_scores(logits, score_func)
    sel = scores + np.asarray(bias, dtype=np.float32) if bias is not None else scores
    T, E = sel.shape
    # stable descending sort: sort by (-value, index)
    order = np.lexsort((np.broadcast_to(np.arange(E), sel.shape), -sel.astype(np.float64)), axis=-1)
    ids = order[:, :k].astype(np.int64)
    w = np.take_along_axis(scores, ids, axis=1).astype(np.float32)
    if score_func != "softmax":
        w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    w = (w * np.float32(route_scale)).astype(np.float32)
    return w, ids


def route_hash(logits: np.ndarray, tid2eid: np.ndarray, input_ids: np.ndarray, k: int,
               score_func: str = "sqrtsoftplus", route_scale: float = 1.0
               ) -> Tuple[np.ndarray, np.ndarray]:
    """deepseek_infer/model.py:565-584 with ``self.hash`` (:576-577): ids =
    tid2eid[input_ids]; weights = the scores at those experts (table order),
    renormalised unless softmax, times route_scale (the bias is None there)."""
    scores = route_scores(logits, score_func)
    ids = np.asarray(tid2eid)[np.asarray(input_ids).reshape(-1)].astype(np.int64)
    assert ids.shape[1] == k
    w = np.take_along_axis(scores, ids, axis=1).astype(np.float32)
    if score_func != "softmax":
        w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return (w * np.float32(route_scale)).astype(np.float32), ids


def router_logits(x_bf16: np.ndarray, w_bf16: np.ndarray) -> np.ndarray:
    """model.py:565 linear(x.float(), W.float()) for bf16 x and W: the exact
    dot products (float64 holds every bf16 x bf16 product and their sum over
    H <= 2^20 terms to far below fp32 resolution), rounded to fp32."""
    return (np.asarray(x_bf16, np.float64) @ np.asarray(w_bf16, np.float64).T).astype(np.float32)


def topk_margin(logits: np.ndarray, k: int, score_func: str = "softmax",
                bias: Optional[np.ndarray] = None) -> float:
    """Smallest gap between the k-th and (k+1)-th selection value over tokens
    (used by tests to assert the data has no near-ties)."""
    scores = route_scores(logits, score_func)
    sel = scores + bias if bias is not None else scores
    s = -np.sort(-sel.astype(np.float64), axis=-1)
    if s.shape[1] <= k:
        return float("inf")
    return float(np.min(s[:, k - 1] - s[:, k]))


# ------------------------------------------------------------- permutation


def permute(ids: np.ndarray, E: int) -> Dict[str, np.ndarray]:
    """Stable counting sort of slot = t*k + j by expert id.

    Restates the dispatch order of deepseek_infer/model.py:634-640 and
    engine/v4_moe_fast.py:89-101: experts ascending, ``torch.where(indices == e)``
    row-major inside an expert.
    """
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    counts = np.bincount(flat, minlength=E).astype(np.int32)[:E]
    offsets = np.zeros(E + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    sorted_slot = np.argsort(flat, kind="stable").astype(np.int32)
    slot_pos = np.empty_like(sorted_slot)
    slot_pos[sorted_slot] = np.arange(flat.size, dtype=np.int32)
    return {"counts": counts, "offsets": offsets, "sorted_slot": sorted_slot, "slot_pos": slot_pos}


def permute_bruteforce(ids: np.ndarray, E: int) -> np.ndarray:
    """The reference's own loop (model.py:635-640): for e ascending,
    ``idx, top = where(indices == e)`` -> sorted slot list."""
    ids = np.asarray(ids)
    out = []
    for e in range(E):
        idx, top = np.nonzero(ids == e)
        out.extend((idx * ids.shape[1] + top).tolist())
    return np.asarray(out, dtype=np.int32)


# -------------------------------------------------------------------- GEMM


def fp8_gemm(aq: np.ndarray, sa: np.ndarray, bq: np.ndarray, sb: np.ndarray,
             out_bf16: bool = True) -> np.ndarray:
    """deepseek_infer/kernel.py:257-273 as a dequantize-to-fp32 reference:
    C = (A_e4m3 * sa) @ (B_e4m3 * sb)^T accumulated in float64, rounded to
    fp32 (and to bf16 when ``out_bf16``)."""
    a = Q.dequant_rows(aq, sa, 128).astype(np.float64)
    b = Q.dequant_blocks(bq, sb, 128).astype(np.float64)
    c = (a @ b.T).astype(np.float32)
    return Q.bf16_round(c) if out_bf16 else c


def fp8_gemm_promoted(aq, sa, bq, sb) -> np.ndarray:
    """The reference kernel's structure exactly: per 128-deep K block an fp32
    partial, then ``acc += partial * (sa * sb)`` in fp32 (kernel.py:238-250)."""
    a = Q.e4m3_to_f32(aq).astype(np.float64)
    b = Q.e4m3_to_f32(bq).astype(np.float64)
    M, K = a.shape
    N = b.shape[0]
    acc = np.zeros((M, N), dtype=np.float32)
    sbr = np.repeat(np.asarray(sb, np.float32), 128, axis=0)[:N]
    for kb in range(K // 128):
        sl = slice(kb * 128, (kb + 1) * 128)
        part = (a[:, sl] @ b[:, sl].T).astype(np.float32)  # exact in fp64, one rounding
        scale = (np.asarray(sa, np.float32)[:, kb][:, None] * sbr[:, kb][None, :]).astype(np.float32)
        acc = (acc + part * scale).astype(np.float32)
    return acc


# ---------------------------------------------------------------- experts


def silu(x: np.ndarray) -> np.ndarray:
    """torch F.silu: x / (1 + exp(-x)) in fp32."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def expert_forward(x_bf16: np.ndarray, w: Dict[str, np.ndarray], weights: Optional[np.ndarray],
                   swiglu_limit: float = 0.0, mode: int = 0,
                   trace: Optional[dict] = None) -> np.ndarray:
    """engine/v4_moe_fast.py:43-76 (= deepseek_infer/model.py:596-606) with FP8
    weights: one act_quant for gate and up, bf16 GEMM outputs upcast,
    clamp, silu(gate)*up, *weights, bf16, w2 (act_quant + fp8_gemm) -> bf16.

    ``w`` holds ``w1, w3, w2`` (e4m3 uint8) and ``s1, s3, s2`` (fp32 block
    scales), or with ``fmt == "fp4"`` packed e2m1 weights and e8m0 1x32 scales
    (model.py:113-115: the same act_quant, then fp4_gemm).
    """
    gemm = F4.fp4_gemm if w.get("fmt") == "fp4" else fp8_gemm
    xq, xs = Q.scale_mode_quant(x_bf16, mode, 128)
    gate = gemm(xq, xs, w["w1"], w["s1"])
    up = gemm(xq, xs, w["w3"], w["s3"])
    if swiglu_limit > 0:
        lim = np.float32(swiglu_limit)
        up = np.clip(up, -lim, lim)
        gate = np.minimum(gate, lim)
    h = (silu(gate) * up).astype(np.float32)
    if weights is not None:
        h = (np.asarray(weights, np.float32) * h).astype(np.float32)
    hb = Q.bf16_round(h)
    hq, hs = Q.scale_mode_quant(hb, mode, 128)
    out = gemm(hq, hs, w["w2"], w["s2"])
    if trace is not None:
        trace.update(xq=xq, xs=xs, gate=gate, up=up, h=hb, hq=hq, hs=hs, out=out)
    return out


def moe_forward(x_bf16: np.ndarray, ids: np.ndarray, weights: np.ndarray,
                experts: Sequence[Dict[str, np.ndarray]], shared: Optional[Dict[str, np.ndarray]],
                swiglu_limit: float = 0.0, mode: int = 0,
                expert_outputs: Optional[dict] = None, workers: int = 1) -> np.ndarray:
    """engine/v4_moe_fast.py:79-106 _moe_forward_activated_only (one rank):
    y = 0 (fp32); for each activated expert ascending: y[tok] += expert(x[tok], w);
    y += shared(x); return bf16(y).

    ``workers`` > 1 computes the experts' outputs on that many threads (numpy
    and BLAS release the GIL) and still sums them in ascending expert order:
    the result is the same bytes as with one worker."""
    x = np.asarray(x_bf16, dtype=np.float32)
    ids = np.asarray(ids)
    y = np.zeros_like(x, dtype=np.float32)

    def run(e):
        tok, top = np.nonzero(ids == e)
        return tok, top, expert_forward(x[tok], experts[e], weights[tok, top][:, None],
                                        swiglu_limit, mode)

    def run_shared():
        return expert_forward(x, shared, None, swiglu_limit, mode)

    active = [e for e in np.unique(ids).tolist()]
    if workers > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(workers) as pool:
            jobs = [pool.submit(run, e) for e in active]
            sh_job = pool.submit(run_shared) if shared is not None else None
            results = [j.result() for j in jobs]
            sh = sh_job.result() if sh_job is not None else None
    else:
        results = [run(e) for e in active]
        sh = run_shared() if shared is not None else None
    for e, (tok, top, out) in zip(active, results):
        if expert_outputs is not None:
            expert_outputs[e] = (tok, top, out)
        y[tok] = (y[tok] + out).astype(np.float32)
    if sh is not None:
        if expert_outputs is not None:
            expert_outputs["shared"] = sh
        y = (y + sh).astype(np.float32)
    return Q.bf16_round(y)


def moe_local_partial(x_bf16: np.ndarray, ids: np.ndarray, weights: np.ndarray,
                      experts: Sequence[Optional[Dict[str, np.ndarray]]], expert_begin: int,
                      expert_end: int, swiglu_limit: float = 0.0, mode: int = 0) -> np.ndarray:
    """engine/v4_moe_fast.py:79-102 on one rank of an expert-sharded layer, up
    to its all_reduce: y = 0 (fp32); for each activated expert ascending, skip
    it unless expert_begin <= e < expert_end (:93-97), y[tok] += expert(x[tok],
    w).  Returns the fp32 y (the value the rank hands to all_reduce)."""
    x = np.asarray(x_bf16, dtype=np.float32)
    ids = np.asarray(ids)
    y = np.zeros_like(x, dtype=np.float32)
    for e in np.unique(ids).tolist():
        if e < expert_begin or e >= expert_end or experts[e] is None:
            continue
        tok, top = np.nonzero(ids == e)
        out = expert_forward(x[tok], experts[e], weights[tok, top][:, None], swiglu_limit, mode)
        y[tok] = (y[tok] + out).astype(np.float32)
    return y


def moe_forward_full_loop(x_bf16, ids, weights, experts, shared, swiglu_limit=0.0, mode=0):
    """The official MoE.forward loop (model.py:629-644): all experts, bincount skip."""
    x = np.asarray(x_bf16, dtype=np.float32)
    ids = np.asarray(ids)
    E = len(experts)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    y = np.zeros_like(x, dtype=np.float32)
    for e in range(E):
        if counts[e] == 0:
            continue
        tok, top = np.nonzero(ids == e)
        y[tok] = (y[tok] + expert_forward(x[tok], experts[e], weights[tok, top][:, None],
                                          swiglu_limit, mode)).astype(np.float32)
    if shared is not None:
        y = (y + expert_forward(x, shared, None, swiglu_limit, mode)).astype(np.float32)
    return Q.bf16_round(y)


def make_expert(rng: np.random.Generator, H: int, I: int, std: float = 0.02,
                ue8m0: bool = False) -> Dict[str, np.ndarray]:
    """Synthetic FP8 expert: N(0, std) weights quantized 128x128 (utils/math.py:50-60;
    ``ue8m0``: scales rounded up to powers of two, the e8m0 form model.py:138-142 stores)."""
    out = {}
    for name, shape in (("1", (I, H)), ("3", (I, H)), ("2", (H, I))):
        w = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
        q, s = Q.per_block_cast_to_fp8(w, use_ue8m0=ue8m0)
        out["w" + name] = q
        out["s" + name] = s
    return out


def make_fp4_expert(rng: np.random.Generator, H: int, I: int, std: float = 0.02) -> Dict[str, np.ndarray]:
    """Synthetic MXFP4 expert (the reference's routed-expert format,
    model.py:129-137): N(0, std) weights -> packed e2m1 + e8m0 1x32 scales."""
    out = {"fmt": "fp4"}
    for name, shape in (("1", (I, H)), ("3", (I, H)), ("2", (H, I))):
        q, s = F4.make_fp4_weight(rng, *shape, std=std)
        out["w" + name] = q
        out["s" + name] = s
    return out
