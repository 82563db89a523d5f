"""Oracle for the MoE prefill grouped INT8 path (test infrastructure only).

The reference repository has no MoE kernel; benchmark configuration 4 defines
the computation, and its CPU baseline is "route with softmax + top-8, then a
per-expert _int_mm loop with a SiLU*mul epilogue, then scatter-add with the
routing weights". This module restates that computation in numpy on the CPU,
with the roundings placed where the GPU path places them:

  route     experts = the top_k router logits per token (descending; equal
            logits: lower expert first); weights = softmax(logits)[experts]
            in fp32 (not renormalised over the top k);
  quantize  x per token: absmax / 127, round half to even (oracle/int8.py);
  gate/up   g, u = order-F dequant of the exact int32 products with the
            per-expert per-channel weight scales (int8_gemm.py:53-63 order);
            h = bf16(silu(g) * u) in fp32, silu(g) = g / (1 + exp(-g));
  down      h quantized per routed row (same rule); y = f32(acc) * (sh * sw)
            in fp32, then y * routing weight in fp32, stored as bf16;
  combine   out[t] = bf16(sum over k of f32(y[t, k])) in top-k order.

Integer parts are exact (float64 BLAS of int8 values: |acc| < 2^53).
"""
from __future__ import annotations

import numpy as np

from . import int8 as o8

F32 = np.float32


def route_topk(logits: np.ndarray, top_k: int):
    """(experts int32 [T, k], weights fp32 [T, k]) — softmax over all experts
    in fp32, selection by logit (ties: lower index)."""
    lg = np.asarray(logits, dtype=np.float32)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :top_k].astype(np.int32)
    mx = lg.max(axis=1, keepdims=True)
    e = np.exp((lg - mx).astype(np.float32)).astype(np.float32)
    p = (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    w = np.take_along_axis(p, order, axis=1).astype(np.float32)
    return order, w


def dispatch(experts: np.ndarray, n_experts: int, pad: int = 64):
    """Counting sort of the routed (token, k) slots by expert, each expert's
    segment padded to a multiple of ``pad`` rows. Returns (counts [E],
    offsets [E], rows_total, row_token [rows] (-1 = padding), row_slot [rows]
    (t * k + j, -1 = padding)) with tokens in ascending order inside a segment
    (the GPU places them in arbitrary order within the segment)."""
    t_n, k = experts.shape
    flat = experts.reshape(-1)
    counts = np.bincount(flat, minlength=n_experts).astype(np.int64)
    padded = (counts + pad - 1) // pad * pad
    offsets = np.concatenate([[0], np.cumsum(padded)[:-1]]).astype(np.int64)
    rows = int(padded.sum())
    row_token = np.full(rows, -1, np.int64)
    row_slot = np.full(rows, -1, np.int64)
    cursor = offsets.copy()
    for s in np.argsort(flat, kind="stable"):
        e = flat[s]
        row_token[cursor[e]] = s // k
        row_slot[cursor[e]] = s
        cursor[e] += 1
    return counts, offsets, rows, row_token, row_slot


def silu(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (g / (F32(1) + np.exp(-g).astype(np.float32))).astype(np.float32)


def gate_up(xq_rows, xs_rows, wq_gate, sg, wq_up, su):
    """h = bf16(silu(g) * u) for routed rows of one expert: xq_rows int8 [R, H],
    xs_rows fp32 [R]; wq_* int8 [F, H]; s* fp32 [F]. Returns fp32 values of the
    bf16 h [R, F]."""
    g = o8.epilogue_f(o8.int8_matmul(xq_rows, wq_gate.T), xs_rows, sg, out="f32")
    u = o8.epilogue_f(o8.int8_matmul(xq_rows, wq_up.T), xs_rows, su, out="f32")
    return o8.round_to((silu(g) * u).astype(np.float32), "bf16")


def down(hq_rows, hs_rows, wq_down, sd, w_rows):
    """y = bf16((f32(acc) * (hs * sd)) * w) for routed rows of one expert."""
    y = o8.epilogue_f(o8.int8_matmul(hq_rows, wq_down.T), hs_rows, sd, out="f32")
    return o8.round_to((y * np.asarray(w_rows, np.float32)[:, None]).astype(np.float32), "bf16")


def combine(y_slots: np.ndarray) -> np.ndarray:
    """y_slots fp32 [T, k, H] (bf16 values) -> fp32 values of bf16(sum over k
    in order)."""
    acc = np.zeros(y_slots[:, 0].shape, np.float32)
    for j in range(y_slots.shape[1]):
        acc = (acc + y_slots[:, j]).astype(np.float32)
    return o8.round_to(acc, "bf16")


def quantize_experts(w: np.ndarray):
    """Per-expert per-output-channel int8: w fp32 [E, N, K] -> (int8 [E, N, K],
    fp32 scales [E, N]) with absmax / 127, round half to even."""
    qs, ss = [], []
    for e in range(w.shape[0]):
        q, s = o8.quant_rows(w[e])
        qs.append(q)
        ss.append(s)
    return np.stack(qs), np.stack(ss)


def moe_forward(x, logits, wq_gate, sg, wq_up, su, wq_down, sd, top_k, tokens=None):
    """Whole forward for the tokens ``tokens`` (default all): x fp32 values
    [T, H]; returns (out fp32 values of bf16 [len(tokens), H], dict of the
    intermediates per (token, k) slot: experts, weights, h, y)."""
    x = np.asarray(x, np.float32)
    experts, weights = route_topk(logits, top_k)
    if tokens is None:
        tokens = np.arange(x.shape[0])
    tokens = np.asarray(tokens)
    xq, xs = o8.quant_rows(x[tokens])
    h_all = np.zeros((len(tokens), top_k, wq_gate.shape[1]), np.float32)
    y_all = np.zeros((len(tokens), top_k, wq_down.shape[1]), np.float32)
    for e in range(wq_gate.shape[0]):
        sel = np.argwhere(experts[tokens] == e)  # (token index, j)
        if len(sel) == 0:
            continue
        ti, j = sel[:, 0], sel[:, 1]
        h = gate_up(xq[ti], xs[ti], wq_gate[e], sg[e], wq_up[e], su[e])
        hq, hs = o8.quant_rows(h)
        y = down(hq, hs, wq_down[e], sd[e], weights[tokens][ti, j])
        h_all[ti, j] = h
        y_all[ti, j] = y
    return combine(y_all), {"experts": experts[tokens], "weights": weights[tokens], "h": h_all, "y": y_all}


def moe_forward_bruteforce(x, logits, wq_gate, sg, wq_up, su, wq_down, sd, top_k):
    """Token-by-token restatement with float64 loops over experts (small cases
    only), independent of the grouped organisation above."""
    x = np.asarray(x, np.float32)
    t_n = x.shape[0]
    out = np.zeros((t_n, wq_down.shape[1]), np.float32)
    for t in range(t_n):
        lg = np.asarray(logits[t], np.float32)
        ranked = sorted(range(len(lg)), key=lambda e: (-float(lg[e]), e))[:top_k]
        ex = np.exp((lg - lg.max()).astype(np.float32)).astype(np.float32)
        p = (ex / ex.sum(dtype=np.float32)).astype(np.float32)
        xq, xs = o8.quant_rows(x[t:t + 1])
        acc = np.zeros(wq_down.shape[1], np.float32)
        for e in ranked:
            g = xq[0].astype(np.float64) @ wq_gate[e].T.astype(np.float64)
            u = xq[0].astype(np.float64) @ wq_up[e].T.astype(np.float64)
            g = (g.astype(np.float32) * (xs[0] * sg[e]).astype(np.float32)).astype(np.float32)
            u = (u.astype(np.float32) * (xs[0] * su[e]).astype(np.float32)).astype(np.float32)
            h = o8.round_to((silu(g) * u).astype(np.float32), "bf16")[None]
            hq, hs = o8.quant_rows(h)
            y = hq[0].astype(np.float64) @ wq_down[e].T.astype(np.float64)
            y = (y.astype(np.float32) * (hs[0] * sd[e]).astype(np.float32)).astype(np.float32)
            y = o8.round_to((y * p[e]).astype(np.float32), "bf16")
            acc = (acc + y).astype(np.float32)
        out[t] = o8.round_to(acc, "bf16")
    return out
