# SPDX-License-Identifier: Apache-2.0
"""MoE prefill with grouped INT8 GEMMs on gfx950 (benchmark configuration 4).

The reference repository has no MoE operator; this module follows the benchmark's
formulation ("route with softmax + top-8, then a per-expert INT8 GEMM with a
SiLU*mul epilogue, then scatter-add with the routing weights") on the same
conventions as the rest of rdna2_ops: per-token INT8 activations (absmax /
127, round half to even), per-expert per-output-channel INT8 weights, order-F
fp32 epilogues (int8_gemm.py:53-63), caller-owned prepared weights, a fresh
output per call, launches on the current torch stream, and hand-written HIP
kernels behind the C ABI of include/qgemm.h (qg_moe_*):

  dispatch   routing (softmax, top-k by logit), per-expert counting sort with
             segments padded to ``pad`` rows, and the grouped GEMM tile table,
             all on the GPU (no host synchronisation); for hidden <= 2048 the
             routing launch also quantizes x per token
  gate/up    grouped GEMM gathering each routed row's token, SiLU * mul
             epilogue -> h bf16 [rows, F]
  quantize   h per routed row (absmax / 127, half even)
  down       grouped GEMM, epilogue * routing weight -> y bf16 [T * k, H]
  combine    out = bf16(sum over k of y) in top-k order (deterministic)
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib


# Largest hidden size whose x rows the routing launch quantizes itself
# (include/qgemm.h, qg_moe_dispatch_qx); wider rows take qg_quant_rows_i8.
MOE_ROUTE_QUANT_MAX_H = 2048


@dataclass
class MoeInt8Weights:
    """Prepared expert weights (caller-owned, like PackedInt4).

    w13: int8 [E, 2F, H]; rows 32 b .. 32 b + 15 are the gate rows and
         32 b + 16 .. 32 b + 31 the up rows of features 16 b .. 16 b + 15
    s13: fp32 [E, 2F] per-row scales in the same order
    w2:  int8 [E, H, F], s2: fp32 [E, H]
    """
    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor

    @property
    def n_experts(self) -> int:
        return self.w13.shape[0]

    @property
    def hidden(self) -> int:
        return self.w13.shape[2]

    @property
    def inter(self) -> int:
        return self.w2.shape[2]


def _quant_rows(x: torch.Tensor, q: torch.Tensor, step: torch.Tensor) -> None:
    m, k = x.shape
    _lib.check(_lib.library().qg_quant_rows_i8(
        _lib.ptr(x), _lib.DTYPE_CODE[x.dtype], x.stride(0), x.stride(1), m, k, _lib.ptr(q), q.stride(0),
        _lib.ptr(step), _lib.ROUND_HALF_EVEN, _lib.stream_of(x)), "qg_quant_rows_i8")


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """[E, F, ...] gate and up -> [E, 2F, ...] in the 16-row interleave of
    MoeInt8Weights.w13 (F % 16 == 0)."""
    e, f = gate.shape[:2]
    rest = gate.shape[2:]
    g = gate.reshape(e, f // 16, 16, *rest)
    u = up.reshape(e, f // 16, 16, *rest)
    return torch.stack([g, u], dim=2).reshape(e, 2 * f, *rest).contiguous()


def prepare_moe_weights(w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor) -> MoeInt8Weights:
    """Quantize per expert and output channel (absmax / 127, round half to
    even) on the GPU and lay out gate/up for the SiLU*mul epilogue.
    w_gate, w_up: [E, F, H]; w_down: [E, H, F]; floating, on the GPU."""
    if w_gate.shape != w_up.shape or w_gate.ndim != 3 or w_down.ndim != 3:
        raise ValueError("w_gate / w_up [E, F, H] and w_down [E, H, F] required")
    e, f, h = w_gate.shape
    if w_down.shape != (e, h, f):
        raise ValueError("w_down must be [E, H, F]")
    if f % 64 or h % 128 or f % 128:
        raise ValueError("F and H must be multiples of 128")
    for w in (w_gate, w_up, w_down):
        if w.device.type != "cuda" or not w.is_floating_point():
            raise TypeError("floating GPU weights required")
    _lib.require_gfx950(w_gate)

    def quant(w):
        w2d = w.reshape(-1, w.shape[-1]).contiguous()
        q = torch.empty(w2d.shape, dtype=torch.int8, device=w.device)
        s = torch.empty(w2d.shape[0], dtype=torch.float32, device=w.device)
        _quant_rows(w2d, q, s)
        return q.reshape(w.shape), s.reshape(w.shape[:-1])

    qg, sg = quant(w_gate)
    qu, su = quant(w_up)
    q2, s2 = quant(w_down)
    return MoeInt8Weights(interleave_gate_up(qg, qu), interleave_gate_up(sg, su), q2, s2)


def _check_weights(p: MoeInt8Weights):
    e, f2, h = p.w13.shape
    if (p.w13.dtype != torch.int8 or p.w2.dtype != torch.int8 or p.s13.shape != (e, f2)
            or p.w2.shape != (e, h, f2 // 2) or p.s2.shape != (e, h)
            or p.s13.dtype != torch.float32 or p.s2.dtype != torch.float32):
        raise ValueError("invalid MoeInt8Weights")
    for t in (p.w13, p.s13, p.w2, p.s2):
        if not t.is_contiguous():
            raise ValueError("prepared weights must be contiguous")


def moe_int8_forward(x: torch.Tensor, router_logits: torch.Tensor, weights: MoeInt8Weights, *, top_k: int = 8,
                     pad: int = 64, return_intermediates: bool = False):
    """MoE FFN prefill: x bf16 [T, H], router_logits [T, E] -> bf16 [T, H].

    With ``return_intermediates`` also returns a dict of the device tensors of
    every stage (routing, dispatch tables, x quantization, h, h
    quantization, y)."""
    _check_weights(weights)
    if x.ndim != 2 or x.dtype != torch.bfloat16 or x.shape[1] != weights.hidden:
        raise ValueError("x must be bf16 [T, H]")
    t, h = x.shape
    e, f = weights.n_experts, weights.inter
    if router_logits.shape != (t, e):
        raise ValueError("router_logits must be [T, E]")
    if x.device != weights.w13.device or router_logits.device != x.device:
        raise ValueError("all tensors on one device")
    if not 1 <= top_k <= e or e > 64:
        raise ValueError("1 <= top_k <= E <= 64 required")
    _lib.require_gfx950(x)
    if t == 0:  # empty input: empty output, nothing launched
        out = torch.empty(0, h, dtype=torch.bfloat16, device=x.device)
        return out if not return_intermediates else (out, {})
    lib = _lib.library()
    dev = x.device
    rows_c, tiles_c = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(lib.qg_moe_sizes(t, e, top_k, pad, ctypes.byref(rows_c), ctypes.byref(tiles_c)), "qg_moe_sizes")
    rows, tiles_n = rows_c.value, tiles_c.value
    logits = router_logits.float().contiguous()
    x = x.contiguous()
    i32 = dict(dtype=torch.int32, device=dev)
    experts = torch.empty(t, top_k, **i32)
    rweights = torch.empty(t, top_k, dtype=torch.float32, device=dev)
    counts = torch.empty(_lib.MOE_COUNTS_PER_EXPERT * e, **i32)
    row_token = torch.empty(rows, **i32)
    row_weight = torch.empty(rows, dtype=torch.float32, device=dev)
    row_slot = torch.empty(rows, **i32)
    tiles = torch.empty(tiles_n, 4, **i32)
    stream = _lib.stream_of(x)
    P = _lib.ptr
    xq = torch.empty(t, h, dtype=torch.int8, device=dev)
    xs = torch.empty(t, dtype=torch.float32, device=dev)
    if h % 8 == 0 and h <= MOE_ROUTE_QUANT_MAX_H and x.data_ptr() % 16 == 0:
        # the routing launch quantizes x as well (bit-identical to qg_quant_rows_i8)
        _lib.check(lib.qg_moe_dispatch_qx(P(logits), e, t, e, top_k, pad, P(experts), P(rweights), P(counts),
                                          P(row_token), P(row_weight), P(row_slot), rows, P(tiles), tiles_n,
                                          P(x), h, h, P(xq), h, P(xs), stream), "qg_moe_dispatch_qx")
    else:
        _lib.check(lib.qg_moe_dispatch(P(logits), e, t, e, top_k, pad, P(experts), P(rweights), P(counts),
                                       P(row_token), P(row_weight), P(row_slot), rows, P(tiles), tiles_n, stream),
                   "qg_moe_dispatch")
        _quant_rows(x, xq, xs)
    hbuf = torch.empty(rows, f, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.qg_moe_grouped_gemm(P(xq), h, t, P(row_token), rows, h, P(weights.w13), h, 2 * f * h, 2 * f, e,
                                       P(tiles), tiles_n, P(xs), P(weights.s13), None, None, _lib.MOE_EPI_SILU_MUL,
                                       P(hbuf), f, rows, stream), "qg_moe_grouped_gemm gate/up")
    hq = torch.empty(rows, f, dtype=torch.int8, device=dev)
    hs = torch.empty(rows, dtype=torch.float32, device=dev)
    _quant_rows(hbuf, hq, hs)
    y = torch.empty(t * top_k, h, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.qg_moe_grouped_gemm(P(hq), f, rows, None, rows, f, P(weights.w2), f, h * f, h, e, P(tiles),
                                       tiles_n, P(hs), P(weights.s2), P(row_weight), P(row_slot),
                                       _lib.MOE_EPI_ROUTE, P(y), h, t * top_k, stream), "qg_moe_grouped_gemm down")
    out = torch.empty(t, h, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.qg_moe_combine(P(y), t, top_k, h, P(out), h, stream), "qg_moe_combine")
    if not return_intermediates:
        return out
    return out, {"experts": experts, "weights": rweights, "counts": counts, "row_token": row_token,
                 "row_weight": row_weight, "row_slot": row_slot, "tiles": tiles, "xq": xq, "xs": xs, "h": hbuf,
                 "hq": hq, "hs": hs, "y": y, "rows_max": rows}


def grouped_gemm_i32(a: torch.Tensor, row_token, tiles: torch.Tensor, w: torch.Tensor, rows_max: int) -> torch.Tensor:
    """The raw grouped INT8 product (QG_MOE_EPI_I32) for tests: int32
    [rows_max, N], routed row r = a[row_token[r]] x w[expert(r)]^T (rows of
    padding left as they were: zero)."""
    e, n, k = w.shape
    out = torch.zeros(rows_max, n, dtype=torch.int32, device=a.device)
    P = _lib.ptr
    _lib.check(_lib.library().qg_moe_grouped_gemm(
        P(a), a.stride(0), a.shape[0], P(row_token), rows_max, k, P(w), k, n * k, n, e, P(tiles), tiles.shape[0],
        None, None, None, None, _lib.MOE_EPI_I32, P(out), n, rows_max, _lib.stream_of(a)), "qg_moe_grouped_gemm i32")
    return out
