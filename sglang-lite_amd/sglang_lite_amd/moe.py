"""The FP8 MoE expert path on gfx950: routing, permutation, grouped GEMMs, combine.

Every function launches HIP kernels of ``libsglang_lite_amd.so`` on torch's
current stream; torch only allocates the buffers.  Nothing here reads routing
data back to the host, so a layer can be captured into a HIP graph.

Semantics follow the reference's official MoE (``deepseek_infer/model.py:
546-644``) and its fast dispatch (``engine/v4_moe_fast.py:43-106``):

* Gate: ``scores = score_func(logits)``, top-k on ``scores + bias``, weights =
  gathered scores (renormalised unless softmax) times ``route_scale``.
* Experts run only on the slots routed to them; the routing weight multiplies
  ``silu(gate) * up`` before ``w2`` (model.py:603-606).
* ``y = sum over the token's experts in ascending id (fp32) + shared(x)``,
  rounded to bf16.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from .kernel import (FP4, FP8, E8M0, e8m0_to_f32, fp4_bytes, fp4_weight_scale, fp4_weight_to_frag,
                     fp8_weight_to_frag)

SCORE_FUNCS = {"softmax": _lib.SCORE_SOFTMAX, "sigmoid": _lib.SCORE_SIGMOID,
               "sqrtsoftplus": _lib.SCORE_SQRTSOFTPLUS}


def _f32_scale(s: torch.Tensor) -> torch.Tensor:
    """fp32 view of a weight scale (e8m0 converted on the device once)."""
    if s.dtype == torch.float32:
        return s.contiguous()
    if s.dtype == E8M0:
        return e8m0_to_f32(s)
    raise TypeError(f"weight scale must be float32 or float8_e8m0fnu, got {s.dtype}")


def _pow2_scale(s: torch.Tensor) -> bool:
    """Whether a weight scale holds only powers of two: e8m0 by type, fp32
    when every value is a positive normal float with no mantissa bits."""
    if s.dtype == E8M0:
        return True
    bits = s.contiguous().view(torch.int32)
    return bool(((bits & 0x807FFFFF) == 0).logical_and_(bits != 0).all().item())


@dataclass
class ExpertTable:
    """Device array of ``sgl_expert_ptrs`` (E routed experts, then the shared one).

    Holds references to every tensor whose address is in the table so the
    pointers stay valid for the table's lifetime.
    """

    ptrs: torch.Tensor          # int64 [E (+1), 6] on the device
    E: int
    H: int
    I: int
    has_shared: bool
    keep: List[torch.Tensor] = field(default_factory=list)
    fmt: int = _lib.EXPERT_FP8_BLOCK128  # sgl_expert_format of the routed experts (+ flags)

    @staticmethod
    def build(experts: Sequence[Tuple[torch.Tensor, ...]],
              shared: Optional[Tuple[torch.Tensor, ...]] = None,
              frag_layout: bool = False) -> "ExpertTable":
        """``experts``: per expert ``(w1, w3, w2, s1, s3, s2)``, either FP8 (w1/w3
        e4m3 [I, H], w2 e4m3 [H, I], 128x128 scales fp32 or e8m0) or FP4 (w1/w3
        packed e2m1 [I, H/2], w2 [H, I/2] as float4_e2m1fn_x2 / int8 / uint8,
        e8m0 scales per 32 inputs: [I, H/32], [H, I/32]); every routed expert in
        one format.  The shared expert is FP8 (deepseek_infer/model.py:626).

        When every FP8 scale is a power of two (e8m0, as model.py:138-142
        stores them, or fp32 without mantissa bits) the table carries
        ``EXPERT_POW2_SCALES``: with a power-of-two activation ``scale_mode``
        the FP8 GEMMs then apply both scales inside the MFMA.

        ``frag_layout``: also keep a copy of every expert weight in the MFMA
        fragment layout (``fp8_weight_to_frag``; FP4 routed experts with their
        e8m0 scales, ``fp4_weight_to_frag``) and add their records after the
        first set (``EXPERT_FRAG_COPY``): the grouped GEMMs then load those
        weights straight into registers.  Costs a second copy of the expert
        weights.

        A routed expert given as None (an expert another rank holds, as
        deepseek_infer/model.py:616-625 builds them) gets a record of null
        pointers; only :func:`moe_forward_local` with a range that excludes
        it may run such a table."""
        rows = list(experts) + ([shared] if shared is not None else [])
        live = [r for r in rows if r is not None]
        if not live:
            raise ValueError("ExpertTable needs at least one expert")
        routed = [r for r in experts if r is not None]
        fp4 = bool(routed) and routed[0][0].dtype in (FP4, torch.int8, torch.uint8)
        first = routed[0] if routed else live[0]
        w1 = first[0]
        I = int(w1.shape[0])
        H = int(w1.shape[1]) * (2 if fp4 and routed else 1)  # packed e2m1 rows hold two inputs per byte
        dev = w1.device
        keep: List[torch.Tensor] = []
        vals = []
        pow2 = True
        for i, r in enumerate(rows):
            if r is None:
                vals.append([0] * 6)
                continue
            w1, w3, w2, s1, s3, s2 = r
            if fp4 and i < len(experts):
                ws = [fp4_bytes(w) for w in (w1, w3, w2)]
                for w, shape in zip(ws, ((I, H // 2), (I, H // 2), (H, I // 2))):
                    if tuple(w.shape) != shape or not w.is_contiguous():
                        raise ValueError(f"FP4 expert weight must be contiguous {shape}, got "
                                         f"{tuple(w.shape)}")
                fs = [fp4_weight_scale(s) for s in (s1, s3, s2)]
                for sc, shape in zip(fs, ((I, H // 32), (I, H // 32), (H, I // 32))):
                    if tuple(sc.shape) != shape:
                        raise ValueError(f"FP4 expert scale must be {shape}, got {tuple(sc.shape)}")
            else:
                ws = [w1, w3, w2]
                for w, shape in zip(ws, ((I, H), (I, H), (H, I))):
                    if w.dtype != FP8 or tuple(w.shape) != shape or not w.is_contiguous():
                        raise ValueError(f"expert weight must be contiguous e4m3 {shape}, got "
                                         f"{w.dtype} {tuple(w.shape)}")
                pow2 = pow2 and all(_pow2_scale(s) for s in (s1, s3, s2))
                fs = [_f32_scale(s) for s in (s1, s3, s2)]
            _lib.require_device(*ws, *fs, what="ExpertTable")
            keep += [*ws, *fs]
            vals.append([ws[0].data_ptr(), ws[1].data_ptr(), ws[2].data_ptr(),
                         fs[0].data_ptr(), fs[1].data_ptr(), fs[2].data_ptr()])
        if frag_layout:
            if H % 128 or I % 128 or (fp4 and (H % 512 or I % 512)):
                raise ValueError("frag_layout needs H and I multiples of 128 (FP4 experts: of 512)")
            for i, r in enumerate(rows):
                row = list(vals[i])
                if r is None:
                    vals.append(row)
                    continue
                if fp4 and i < len(experts):
                    pairs = [fp4_weight_to_frag(w, sc) for w, sc in zip(r[:3], r[3:])]
                    keep += [t for pr in pairs for t in pr]
                    row = [pr[0].data_ptr() for pr in pairs] + [pr[1].data_ptr() for pr in pairs]
                else:
                    frags = [fp8_weight_to_frag(w) for w in r[:3]]
                    keep += frags
                    row[:3] = [f.data_ptr() for f in frags]
                vals.append(row)
        ptrs = torch.tensor(vals, dtype=torch.int64).to(dev)
        fmt = _lib.EXPERT_FP4_E2M1 if fp4 else _lib.EXPERT_FP8_BLOCK128
        if pow2:
            fmt |= _lib.EXPERT_POW2_SCALES
        if frag_layout:
            fmt |= _lib.EXPERT_FRAG_COPY
        return ExpertTable(ptrs, len(experts), H, I, shared is not None, keep, fmt)


def route_topk(logits: torch.Tensor, k: int, score_func: str = "softmax",
               bias: Optional[torch.Tensor] = None, route_scale: float = 1.0
               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-k routing from fp32 router logits [T, E] (model.py:565-584 after the
    projection).  Returns ``(weights f32 [T, k], ids int32 [T, k])``."""
    _lib.require_device(logits, bias, what="route_topk")
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise TypeError("route_topk: logits must be float32 [T, E]")
    lg = logits.contiguous()
    T, E = lg.shape
    ids = torch.empty(T, k, dtype=torch.int32, device=lg.device)
    w = torch.empty(T, k, dtype=torch.float32, device=lg.device)
    b = None
    if bias is not None:
        b = bias.to(torch.float32).contiguous()
    _lib.call("sgl_moe_route_topk", lg.data_ptr(), T, E, k, SCORE_FUNCS[score_func],
              _lib.ptr(b), float(route_scale), ids.data_ptr(), w.data_ptr(), _lib.stream_of(lg))
    return w, ids


def gate(x: torch.Tensor, weight: torch.Tensor, k: int, score_func: str = "softmax",
         bias: Optional[torch.Tensor] = None, route_scale: float = 1.0,
         tid2eid: Optional[torch.Tensor] = None, input_ids: Optional[torch.Tensor] = None,
         logits: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gate.forward (deepseek_infer/model.py:564-584) in two launches: the router
    projection ``linear(x.float(), W.float())`` on bf16 MFMA (bf16 products are
    exact, fp32 accumulation), then score function, bias, top-k (or the hash
    table row ``tid2eid[input_ids]`` when ``tid2eid`` is given, model.py:576-577),
    renormalisation and ``route_scale``.  ``x`` bf16 [T, H], ``weight`` bf16 [E, H].
    Returns ``(weights f32 [T, k], ids int32 [T, k])``; ``logits`` (fp32 [T, E],
    optional) receives the projection."""
    _lib.require_device(x, weight, bias, tid2eid, input_ids, what="moe_gate")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError(f"moe_gate: x and weight must be bfloat16, got {x.dtype}, {weight.dtype}")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    W = weight.contiguous()
    T, H = x2.shape
    E = W.shape[0]
    if W.shape[1] != H:
        raise ValueError(f"moe_gate: weight is {tuple(W.shape)}, x has H={H}")
    dev = x2.device
    lg = logits if logits is not None else torch.empty(T, E, dtype=torch.float32, device=dev)
    assert lg.dtype == torch.float32 and lg.is_contiguous() and lg.numel() == T * E
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    tab = ids_in = None
    vocab = 0
    if tid2eid is not None:
        if input_ids is None:
            raise ValueError("moe_gate: hash routing needs input_ids")
        tab = tid2eid.to(torch.int32).contiguous()
        if tab.dim() != 2 or tab.shape[1] != k:
            raise ValueError(f"moe_gate: tid2eid must be [vocab, {k}], got {tuple(tab.shape)}")
        vocab = tab.shape[0]
        ids_in = input_ids.reshape(-1).contiguous()
        if ids_in.dtype not in (torch.int32, torch.int64) or ids_in.numel() != T:
            raise ValueError("moe_gate: input_ids must be int32/int64 with one id per token")
    ids = torch.empty(T, k, dtype=torch.int32, device=dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    _lib.call("sgl_moe_gate", x2.data_ptr(), W.data_ptr(), T, H, E, k, SCORE_FUNCS[score_func],
              _lib.ptr(b), float(route_scale), _lib.ptr(tab), vocab, _lib.ptr(ids_in),
              int(ids_in is not None and ids_in.dtype == torch.int64), lg.data_ptr(),
              ids.data_ptr(), w.data_ptr(), _lib.stream_of(x2))
    return w, ids


def _ids32(ids: torch.Tensor) -> torch.Tensor:
    if ids.dtype == torch.int32:
        return ids.contiguous()
    if ids.dtype == torch.int64:
        return ids.to(torch.int32).contiguous()
    raise TypeError(f"expert ids must be int32/int64, got {ids.dtype}")


def permute(ids: torch.Tensor, E: int):
    """Stable counting sort of the slots (t*k+j) by expert id.

    Returns ``(counts [E], offsets [E+1], sorted_slot [T*k], slot_pos [T*k])``, int32."""
    _lib.require_device(ids, what="moe_permute")
    ids = _ids32(ids)
    T, k = ids.shape
    dev = ids.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    sorted_slot = torch.empty(T * k, dtype=torch.int32, device=dev)
    slot_pos = torch.empty(T * k, dtype=torch.int32, device=dev)
    _lib.call("sgl_moe_permute", ids.data_ptr(), T, k, E, counts.data_ptr(), offsets.data_ptr(),
              sorted_slot.data_ptr(), slot_pos.data_ptr(), _lib.stream_of(ids))
    return counts, offsets, sorted_slot, slot_pos


def gate_up(xq, xs, offsets, sorted_slot, route_w, table: ExpertTable, k: int,
            swiglu_limit: float = 0.0, scale_mode: int = _lib.SCALE_TORCH_FP32):
    """Grouped gate/up GEMM + SwiGLU + requant.  Returns ``(hq e4m3 [rows, I], hs f32 [rows, I/128])``."""
    T, H = xq.shape
    rows = T * k + (T if table.has_shared else 0)
    hq = torch.empty(rows, table.I, dtype=FP8, device=xq.device)
    hs = torch.empty(rows, table.I // 128, dtype=torch.float32, device=xq.device)
    _lib.call("sgl_moe_gate_up", xq.data_ptr(), xs.data_ptr(), T, H, table.I, table.E, k,
              offsets.data_ptr(), sorted_slot.data_ptr(), _lib.ptr(route_w), table.ptrs.data_ptr(),
              int(table.has_shared), table.fmt, float(swiglu_limit), int(scale_mode), hq.data_ptr(),
              hs.data_ptr(), _lib.stream_of(xq))
    return hq, hs


def down(hq, hs, offsets, sorted_slot, table: ExpertTable, T: int, k: int,
         scale_mode: int = _lib.SCALE_TORCH_FP32):
    """Grouped down GEMM (``scale_mode``: the mode ``hs`` was made with).
    Returns bf16 [T, k (+1), H] (token-major expert rows)."""
    kk = k + (1 if table.has_shared else 0)
    out = torch.empty(T, kk, table.H, dtype=torch.bfloat16, device=hq.device)
    _lib.call("sgl_moe_down", hq.data_ptr(), hs.data_ptr(), T, table.H, table.I, table.E, k,
              offsets.data_ptr(), sorted_slot.data_ptr(), table.ptrs.data_ptr(),
              int(table.has_shared), table.fmt, int(scale_mode), out.data_ptr(),
              _lib.stream_of(hq))
    return out


def combine(out: torch.Tensor, ids: torch.Tensor, has_shared: bool) -> torch.Tensor:
    """Ordered fp32 combine of [T, k (+1), H] expert rows -> bf16 [T, H]."""
    ids = _ids32(ids)
    T, k = ids.shape
    H = out.shape[-1]
    y = torch.empty(T, H, dtype=torch.bfloat16, device=out.device)
    _lib.call("sgl_moe_combine", out.data_ptr(), ids.data_ptr(), T, k, H, int(has_shared),
              y.data_ptr(), _lib.stream_of(out))
    return y


class MoEWorkspace:
    """Reusable device workspace for :func:`moe_forward`, grown on demand.

    A buffer once handed out is never freed while the workspace lives: a HIP
    graph captured with it keeps its address and writes there on every
    replay, so when a larger call needs more bytes the old buffer moves to
    ``retired`` instead of going back to torch's pool (where another tensor
    could take it).  Growth is geometric (at least 1.5x), which bounds the
    retired bytes by twice the largest buffer; :meth:`reserve` sizes the
    workspace once up front (e.g. for the largest batch a runner captures).
    """

    def __init__(self):
        self.buf: Optional[torch.Tensor] = None
        self.retired: List[torch.Tensor] = []

    def get(self, nbytes: int, device) -> torch.Tensor:
        dev = torch.device(device)
        if self.buf is not None and self.buf.device != dev:
            self.retired.append(self.buf)
            self.buf = None
        if self.buf is None or self.buf.numel() < nbytes:
            size = max(nbytes, 256)
            if self.buf is not None:
                size = max(size, self.buf.numel() * 3 // 2)
                self.retired.append(self.buf)
            self.buf = torch.empty(size, dtype=torch.uint8, device=dev)
        return self.buf

    def reserve(self, T: int, table: "ExpertTable", k: int, device) -> torch.Tensor:
        """Size the workspace for layers of up to ``T`` tokens over ``table``."""
        return self.get(workspace_size(T, table.H, table.I, table.E, k, table.has_shared), device)


def moe_forward(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, table: ExpertTable,
                swiglu_limit: float = 0.0, scale_mode: int = _lib.SCALE_TORCH_FP32,
                workspace: Optional[MoEWorkspace] = None, out: Optional[torch.Tensor] = None
                ) -> torch.Tensor:
    """Routed + shared MoE layer on bf16 x [T, H] given top-k ``ids``/``weights``."""
    _lib.require_device(x, ids, weights, what="moe_forward")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError("moe_forward: x must be bfloat16 [T, H]")
    x = x.contiguous()
    ids = _ids32(ids)
    w = weights.to(torch.float32).contiguous() if weights.dtype != torch.float32 else weights.contiguous()
    T, H = x.shape
    k = ids.shape[1]
    if H != table.H:
        raise ValueError(f"moe_forward: x has H={H}, experts have H={table.H}")
    lib = _lib.load()
    nbytes = int(lib.sgl_moe_workspace_size(T, H, table.I, table.E, k, int(table.has_shared)))
    ws = (workspace or MoEWorkspace()).get(nbytes, x.device)
    y = out if out is not None else torch.empty(T, H, dtype=torch.bfloat16, device=x.device)
    _lib.call("sgl_moe_forward", x.data_ptr(), T, H, table.I, table.E, k, ids.data_ptr(),
              w.data_ptr(), table.ptrs.data_ptr(), int(table.has_shared), table.fmt,
              float(swiglu_limit), int(scale_mode), ws.data_ptr(), ws.numel(), y.data_ptr(),
              _lib.stream_of(x))
    return y


def moe_forward_local(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                      table: ExpertTable, expert_begin: int, expert_end: int,
                      swiglu_limit: float = 0.0, scale_mode: int = _lib.SCALE_TORCH_FP32,
                      workspace: Optional[MoEWorkspace] = None) -> torch.Tensor:
    """One rank's share of an expert-sharded layer (engine/v4_moe_fast.py:79-102
    up to the all-reduce): fp32 [T, H] = the sum, in ascending expert id, of
    each token's outputs from the routed experts in ``[expert_begin,
    expert_end)``.  The shared expert runs in the same launches and its rows
    stay in ``workspace`` for :func:`moe_add_shared` (pass the same object)."""
    _lib.require_device(x, ids, weights, what="moe_forward_local")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError("moe_forward_local: x must be bfloat16 [T, H]")
    x = x.contiguous()
    ids = _ids32(ids)
    w = weights.to(torch.float32).contiguous()
    T, H = x.shape
    k = ids.shape[1]
    if H != table.H:
        raise ValueError(f"moe_forward_local: x has H={H}, experts have H={table.H}")
    ws = (workspace or MoEWorkspace()).get(workspace_size(T, H, table.I, table.E, k,
                                                          table.has_shared), x.device)
    y = torch.empty(T, H, dtype=torch.float32, device=x.device)
    _lib.call("sgl_moe_forward_local", x.data_ptr(), T, H, table.I, table.E, k, ids.data_ptr(),
              w.data_ptr(), table.ptrs.data_ptr(), int(expert_begin), int(expert_end),
              int(table.has_shared), table.fmt, float(swiglu_limit), int(scale_mode),
              ws.data_ptr(), ws.numel(), y.data_ptr(), _lib.stream_of(x))
    return y


def moe_add_shared(y_local: torch.Tensor, table: ExpertTable, k: int,
                   workspace: MoEWorkspace) -> torch.Tensor:
    """``bf16(y_local + shared(x))`` (engine/v4_moe_fast.py:103-106) with the
    shared expert's rows that :func:`moe_forward_local` left in ``workspace``."""
    _lib.require_device(y_local, what="moe_add_shared")
    if not table.has_shared:
        raise ValueError("moe_add_shared: the table has no shared expert")
    if y_local.dtype != torch.float32 or y_local.dim() != 2 or not y_local.is_contiguous():
        raise TypeError("moe_add_shared: y_local must be contiguous float32 [T, H]")
    T, H = y_local.shape
    ws = workspace.buf
    if ws is None:
        raise ValueError("moe_add_shared: the workspace holds no moe_forward_local result")
    y = torch.empty(T, H, dtype=torch.bfloat16, device=y_local.device)
    _lib.call("sgl_moe_add_shared", y_local.data_ptr(), ws.data_ptr(), ws.numel(), T, H, table.I,
              table.E, int(k), y.data_ptr(), _lib.stream_of(y_local))
    return y


def workspace_size(T: int, H: int, I: int, E: int, k: int, has_shared: bool) -> int:
    return int(_lib.load().sgl_moe_workspace_size(T, H, I, E, k, int(has_shared)))


__all__ = ["ExpertTable", "MoEWorkspace", "combine", "down", "gate", "gate_up", "moe_add_shared",
           "moe_forward", "moe_forward_local", "permute", "route_topk", "workspace_size"]
