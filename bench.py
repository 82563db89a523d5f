#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-weight GEMM hot path (one GPU).

Workload (the W8A8 INT8 GEMM metric's chain): the
fused DiT-block INT8 GEMM chain at M = 4096 tokens, hidden 3072:
  QKV   = W8A8(x)              N = 9216,  K = 3072
  H     = GELU_tanh(W8A8(x))   N = 12288, K = 3072
  Y     = W8A8(H)              N = 3072,  K = 12288
where W8A8(.) = per-token int8 quantization of the fp16 input (absmax/127,
half-even) followed by the int8 MFMA GEMM with the fused fp32 epilogue
(per-token x per-channel scale, bias, optional GELU, fp16 out).
One step = one pass of this chain; inputs and int8 weights are resident in HBM
before timing; weights are synthetic N(0, 0.02) quantized per output channel.

Prints one JSON line (driver contract). ``value`` = whole-chain TOPS
(2*M*N*K summed over the three GEMMs, divided by the step time).
``roofline`` covers the dominant kernel (the int8 GEMM), timed with HIP events
around each GEMM launch on its stream inside the timed steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "rdna2-gfx1030-ai-handbook_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W8A8 INT8 GEMM TOPS (% MFMA peak); W4A16 decode HBM GB/s (% peak)"
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-rows", type=int, default=4096, help="tokens in the CPU-baseline sample")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 512 MiB device copy (calibrates FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


class Chain:
    """Preallocated buffers and direct C-ABI launches of the cfg1 chain."""

    def __init__(self, torch, lib, _lib, quantize, cfg, dev):
        self.t, self.lib, self.L = torch, lib, _lib
        self.m = cfg.x.shape[0]
        self.x = cfg.x.to(dev)
        self.layers = []
        for w, b, act in ((cfg.w_qkv, cfg.b_qkv, 0), (cfg.w_up, cfg.b_up, _lib.EPI_GELU_TANH),
                          (cfg.w_down, cfg.b_down, 0)):
            wq, ws = quantize(w.to(dev))
            n, k = wq.shape
            self.layers.append(dict(
                wq=wq, ws=ws.reshape(-1).contiguous(), b=b.to(dev), n=n, k=k, epi=act,
                xq=torch.empty((self.m, k), dtype=torch.int8, device=dev),
                xs=torch.empty((self.m,), dtype=torch.float32, device=dev),
                out=torch.empty((self.m, n), dtype=torch.float16, device=dev)))
        self.stream = torch.cuda.current_stream(dev)
        self.s = self.stream.cuda_stream
        self.inputs = [self.x, self.x, self.layers[1]["out"]]

    def quant(self, i):
        L, P = self.layers[i], self.L.ptr
        x = self.inputs[i]
        st = self.lib.qg_quant_rows_i8(P(x), self.L.F16, L["k"], 1, self.m, L["k"], P(L["xq"]), L["k"],
                                       P(L["xs"]), self.L.ROUND_HALF_EVEN, self.s)
        self.L.check(st, "quant")

    def gemm(self, i):
        L, P = self.layers[i], self.L.ptr
        st = self.lib.qg_int8_gemm(P(L["xq"]), L["k"], 1, P(L["wq"]), 1, L["k"], self.m, L["n"], L["k"],
                                   P(L["xs"]), P(L["ws"]), L["n"], P(L["b"]), self.L.F16, P(L["out"]),
                                   self.L.F16, L["epi"], None, 0, self.s)
        self.L.check(st, "gemm")

    def ops(self):
        return sum(2 * self.m * L["n"] * L["k"] for L in self.layers)

    def step(self, events=None):
        for i in range(3):
            self.quant(i)
            if events is not None:
                e0 = self.t.cuda.Event(enable_timing=True)
                e1 = self.t.cuda.Event(enable_timing=True)
                e0.record(self.stream)
            self.gemm(i)
            if events is not None:
                e1.record(self.stream)
                events.append((i, e0, e1))


def run_cfg0(torch, lib, _lib, quantize, synthetic, dev, iters=50):
    """Secondary: cfg0 W8A8 linear (quant + GEMM) and the GEMM alone."""
    c = synthetic.cfg0()
    x, bias = c.x.to(dev), c.bias.to(dev)
    wq, ws = quantize(c.w.to(dev))
    ws = ws.reshape(-1).contiguous()
    m, k = x.shape
    n = wq.shape[0]
    xq = torch.empty((m, k), dtype=torch.int8, device=dev)
    xs = torch.empty((m,), dtype=torch.float32, device=dev)
    out = torch.empty((m, n), dtype=torch.float16, device=dev)
    s = torch.cuda.current_stream(dev)
    P = _lib.ptr

    def quant():
        _lib.check(lib.qg_quant_rows_i8(P(x), _lib.F16, k, 1, m, k, P(xq), k, P(xs), 0, s.cuda_stream), "q")

    def gemm():
        _lib.check(lib.qg_int8_gemm(P(xq), k, 1, P(wq), 1, k, m, n, k, P(xs), P(ws), n, P(bias), _lib.F16,
                                    P(out), _lib.F16, 0, None, 0, s.cuda_stream), "g")

    for _ in range(5):
        quant(); gemm()
    torch.cuda.synchronize()
    res = {}
    for label, fn in (("gemm", gemm), ("quant", quant)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(iters):
            fn()
        e1.record(s)
        e1.synchronize()
        res[label] = e0.elapsed_time(e1) / iters
    ops = 2.0 * m * n * k
    gemm_tops = ops / (res["gemm"] * 1e-3) / 1e12
    lin_tops = ops / ((res["gemm"] + res["quant"]) * 1e-3) / 1e12
    quant_bytes = m * k * 2 + m * k + m * 4
    return {"cfg0_gemm_us": round(res["gemm"] * 1e3, 2), "cfg0_gemm_tops": round(gemm_tops, 1),
            "cfg0_gemm_frac_int8_peak": round(gemm_tops / PEAK_INT8_TOPS, 4),
            "cfg0_quant_us": round(res["quant"] * 1e3, 2),
            "cfg0_quant_gbs": round(quant_bytes / (res["quant"] * 1e-3) / 1e9, 1),
            "cfg0_w8a8_linear_tops": round(lin_tops, 1)}


def traffic_bytes():
    """HBM bytes per launch of the GEMM kernel in this chain, measured with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by a plain-copy calibration)
    and recorded in profiles/int8_gemm_cfg1_chain_traffic.json; None if absent."""
    path = ROOT / "profiles" / "int8_gemm_cfg1_chain_traffic.json"
    try:
        return json.loads(path.read_text())["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1; sharding is described in DESIGN.md)", file=sys.stderr, flush=True)
        sys.exit(2)
    import torch
    from rdna2_ops import _lib, synthetic
    from rdna2_ops.quantize import quantize_int8_rowwise

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        # A plain copy of known size: 512 MiB read + 512 MiB written per launch
        # (larger than the 256 MB Infinity Cache), for scaling HBM counters.
        src = torch.ones(512 * 2 ** 20 // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_each_way": src.numel() * 4, "launches": 5}), flush=True)
        return
    lib = _lib.library()
    chain = Chain(torch, lib, _lib, quantize_int8_rowwise, synthetic.cfg1(), dev)
    for _ in range(args.warmup):
        chain.step()
    torch.cuda.synchronize()

    events = []
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(chain.stream)
    for _ in range(args.steps):
        chain.step(events)
    stop.record(chain.stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    ops = chain.ops()
    value = ops / (ms * 1e-3) / 1e12

    gemm_ms = sum(e0.elapsed_time(e1) for _, e0, e1 in events)
    gemm_ops = ops * args.steps
    per_layer = {}
    for i, e0, e1 in events:
        per_layer.setdefault(i, []).append(e0.elapsed_time(e1))
    achieved = gemm_ops / (gemm_ms * 1e-3) / 1e12
    layer_info = {}
    for i, name in enumerate(("qkv", "up_gelu", "down")):
        L = chain.layers[i]
        t = sum(per_layer[i]) / len(per_layer[i])
        layer_info[name] = {"us": round(t * 1e3, 2),
                            "tops": round(2 * chain.m * L["n"] * L["k"] / (t * 1e-3) / 1e12, 1)}

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TOPS", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized per channel)",
        "config": {"workload": "cfg1 DiT-block W8A8 INT8 GEMM chain: M=4096, hidden=3072; "
                               "QKV N=9216; MLP up N=12288 + GELU-tanh; MLP down K=12288->N=3072; "
                               "per-token int8 quant prologue on each GEMM; fp16 in/out",
                   "tokens": chain.m, "hidden": 3072, "ops_per_step": ops},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_INT8_TOPS,
                     "unit": "TOPS", "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": traffic_bytes(),
                     "kernel": "k_i8_gemm<256,192> (int8 MFMA GEMM + fused epilogue)",
                     "per_launch": layer_info},
    }
    if not args.no_secondary:
        line["secondary"] = run_cfg0(torch, lib, _lib, quantize_int8_rowwise, synthetic, dev)
    if not args.no_cpu_baseline:
        from oracle.cpu_baseline import time_cfg1_chain
        cpu_ops, cpu_s, threads, sample = time_cfg1_chain(rows=args.cpu_rows, seconds=args.cpu_seconds)
        line["cpu_baseline"] = {"value": round(cpu_ops / 1e12, 4), "unit": "TOPS", "cores": threads,
                                "kind": "port", "sample": sample, "seconds_per_sample": round(cpu_s, 3)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
