#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-weight GEMM hot path (one GPU).

Workload (benchmark configuration 1, the W8A8 INT8 GEMM metric's chain): the
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
around each GEMM launch on the chain's stream in instrumented chain rounds,
alternated with the plain rounds that give ``value`` (the event records add
about 4 % to a step).
``roofline_w4a16_decode`` is the metric's second half: the W4A16 decode kernel
(benchmark configuration 2, M = 1) in GB/s against the 8 TB/s HBM peak, timed
with events around graph replays of 120 launches over 12 rotated weight copies;
its ``read_floor`` is qg_read_floor over the same byte count, rotated the same
way (the plain-read floor of this box).
``roofline_cfg0`` is the INT8 GEMM alone at benchmark configuration 0, where
the metric's >= 60 % bar is quoted. ``secondary`` holds cfg0's quantizer,
W4A16 M = 16 / 2048, the FP8 configuration 3, MoE (configuration 4), W4A8
and the MOSS production INT8 shapes (M 1061, fp32 out).

Timing protocol (the reference's, rdna2-ops/bench_int8_gemm.py:259-268):
--rounds alternating rounds (forward order on even rounds, reverse on odd) of
the chain (exactly --steps steps per round between synchronisations; a plain
and an instrumented round each), the cfg0 GEMM and quantizer and the two
decode shapes; every figure is the median
over rounds, the per-round samples are reported. ``clock`` is the GPU's GFX
clock read with amdsmi over a 2.5 s window of the same chain after the rounds.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "rdna2-gfx1030-ai-handbook_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W8A8 INT8 GEMM TOPS (% MFMA peak); W4A16 decode HBM GB/s (% peak)"
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s
PEAK_BF16_TFLOPS = 2500.0 # MI355X dense bf16 MFMA, 2.5 PFLOP/s


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-rows", type=int, default=4096, help="tokens in the CPU-baseline sample")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--rounds", type=int, default=3,
                    help="alternating timing rounds; every figure is the median over rounds")
    ap.add_argument("--only", choices=("w4a16", "fp8", "moe", "w4a8", "cfg0", "decode", "moss", "clock",
                                       "stages"),
                    default=None,
                    help="run one secondary measurement alone and print it (for profiling)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 512 MiB device copy (calibrates FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


class Chain:
    """Preallocated buffers and direct C-ABI launches of the cfg1 chain."""

    def __init__(self, torch, lib, _lib, quantize, cfg, dev, stream=None):
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
        self.stream = stream if stream is not None else torch.cuda.current_stream(dev)
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

    def step(self, events=None, pairs=None):
        """One chain step. With ``events``, each GEMM launch is bracketed by the
        next pre-created event pair from the iterator ``pairs`` (no event is
        created inside a timed region) and (layer, start, end) is appended."""
        for i in range(3):
            self.quant(i)
            if events is not None:
                e0, e1 = next(pairs)
                e0.record(self.stream)
            self.gemm(i)
            if events is not None:
                e1.record(self.stream)
                events.append((i, e0, e1))


class Cfg0:
    """Benchmark configuration 0 (M 4096, N = K = 3072, fp16 in / out, seed 0):
    the per-token quantizer and the INT8 GEMM with the order-F epilogue and
    bias, each launched through the C ABI on preallocated buffers."""

    def __init__(self, torch, lib, _lib, quantize, synthetic, dev, iters=50):
        self.t, self.lib, self.L, self.iters = torch, lib, _lib, iters
        c = synthetic.cfg0()
        self.x, self.bias = c.x.to(dev), c.bias.to(dev)
        self.wq, ws = quantize(c.w.to(dev))
        self.ws = ws.reshape(-1).contiguous()
        self.m, self.k = self.x.shape
        self.n = self.wq.shape[0]
        self.xq = torch.empty((self.m, self.k), dtype=torch.int8, device=dev)
        self.xs = torch.empty((self.m,), dtype=torch.float32, device=dev)
        self.out = torch.empty((self.m, self.n), dtype=torch.float16, device=dev)
        self.stream = torch.cuda.current_stream(dev)
        for _ in range(5):
            self.quant()
            self.gemm()
        torch.cuda.synchronize()

    def quant(self):
        P, L = self.L.ptr, self.L
        L.check(self.lib.qg_quant_rows_i8(P(self.x), L.F16, self.k, 1, self.m, self.k, P(self.xq), self.k,
                                          P(self.xs), L.ROUND_HALF_EVEN, self.stream.cuda_stream), "quant")

    def gemm(self):
        P, L, m, n, k = self.L.ptr, self.L, self.m, self.n, self.k
        L.check(self.lib.qg_int8_gemm(P(self.xq), k, 1, P(self.wq), 1, k, m, n, k, P(self.xs), P(self.ws), n,
                                      P(self.bias), L.F16, P(self.out), L.F16, 0, None, 0,
                                      self.stream.cuda_stream), "gemm")

    def _time(self, fn):
        e0, e1 = self.t.cuda.Event(enable_timing=True), self.t.cuda.Event(enable_timing=True)
        gc.disable()
        try:
            e0.record(self.stream)
            for _ in range(self.iters):
                fn()
            e1.record(self.stream)
            e1.synchronize()
        finally:
            gc.enable()
        return e0.elapsed_time(e1) / self.iters

    def time_gemm(self):
        return self._time(self.gemm)

    def time_quant(self):
        return self._time(self.quant)

    def ops(self):
        return 2.0 * self.m * self.n * self.k

    def quant_bytes(self):
        return self.m * self.k * 2 + self.m * self.k + self.m * 4

    def profile_run(self):
        """One quant + GEMM pair after warm-up (for rocprofv3 runs)."""
        ms = self.time_gemm()
        return {"gemm_us": round(ms * 1e3, 2), "tops": round(self.ops() / (ms * 1e-3) / 1e12, 1)}


def _graph_time(torch, fn, launches, replays=4):
    """Capture ``launches`` calls of fn(i) in a HIP graph on a side stream and
    return the average time per call (ms) over ``replays`` replays, timed with
    events on that stream (no host launch cost inside the timed region)."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for i in range(4):
            fn(i, s.cuda_stream)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(launches):
                fn(i, s.cuda_stream)
        g.replay()
        s.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(replays):
            g.replay()
        e1.record(s)
        e1.synchronize()
    return e0.elapsed_time(e1) / (launches * replays)


def _w4_weights(torch, dev, copies):
    """Benchmark configuration 2 weights (K 4096, N 14336, g128, uint4 storage with
    bf16 scales and packed uint4 zero points) and ``copies - 1`` clones."""
    from rdna2_ops import int4_weight_gemm_v07 as w4
    N, K, G = 14336, 4096, 128
    gen = torch.Generator().manual_seed(2)
    p0 = w4.pack_uint4((torch.randn(N, K, generator=gen) * 0.02).to(dev), group_size=G)
    ps = [p0] + [w4.PackedInt4(p0.data.clone(), p0.scales.clone(), p0.zeros.clone(), p0.sums, N, K, G, False,
                               signed=False, zeros_packed=True) for _ in range(copies - 1)]
    return gen, ps


class DecodeW4:
    """The W4A16 decode shapes of benchmark configuration 2 (M = 1 and 16, bf16
    activations and output). Each sample is one replay of a HIP graph of 120
    launches rotating over ``copies`` weight copies (366 MB, more than the
    256 MB MALL), so every launch streams its weights from HBM; the time per
    launch is the replay's event time / 120."""

    N, K, G = 14336, 4096, 128

    def __init__(self, torch, lib, _lib, dev, copies=12, launches=120):
        self.t, self.lib, self.L, self.copies, self.launches = torch, lib, _lib, copies, launches
        gen, self.ps = _w4_weights(torch, dev, copies)
        p0 = self.ps[0]
        self.wbytes = p0.data.numel() * 4 + p0.scales.numel() * 2 + p0.zeros.numel() * 4
        self.graphs = {}
        for m in (1, 16):
            a = torch.randn(m, self.K, generator=gen).to(torch.bfloat16).to(dev)
            y = torch.empty(m, self.N, dtype=torch.bfloat16, device=dev)
            self.graphs[m] = self._capture(m, a, y)
        # the read floor: qg_read_floor over `copies` buffers of the M = 1
        # launch's algorithmic bytes, rotated the same way
        self.floor_bytes = (self.wbytes + self.K * 2 + self.N * 2 + 15) // 16 * 16
        self.floor_bufs = [torch.ones(self.floor_bytes, dtype=torch.uint8, device=dev) for _ in range(copies)]
        self.sink = torch.zeros(1, dtype=torch.int32, device=dev)
        self.graphs["floor"] = self._capture_floor()

    def _call(self, m, a, y, p, stream):
        P, L = self.L.ptr, self.L
        L.check(self.lib.qg_w4a16_gemm(P(a), L.BF16, self.K, m, self.K, P(p.data), self.N, self.G, p.flags,
                                       P(p.scales), L.BF16, P(p.zeros), None, 0, P(y), L.BF16, None, 0, stream),
                "w4a16")

    def _capture(self, m, a, y):
        torch = self.t
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for i in range(4):
                self._call(m, a, y, self.ps[i % self.copies], s.cuda_stream)
            s.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for i in range(self.launches):
                    self._call(m, a, y, self.ps[i % self.copies], s.cuda_stream)
            g.replay()
            s.synchronize()
        return g, s, a, y

    def _capture_floor(self):
        torch, P, L = self.t, self.L.ptr, self.L

        def call(i, stream):
            L.check(self.lib.qg_read_floor(P(self.floor_bufs[i % self.copies]), self.floor_bytes, P(self.sink),
                                           stream), "read_floor")
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for i in range(4):
                call(i, s.cuda_stream)
            s.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for i in range(self.launches):
                    call(i, s.cuda_stream)
            g.replay()
            s.synchronize()
        return g, s, None, None

    def time_floor(self):
        return self.time("floor")

    def time(self, m):
        g, s, _, _ = self.graphs[m]
        torch = self.t
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            e0.record(s)
            g.replay()
            e1.record(s)
        e1.synchronize()
        return e0.elapsed_time(e1) / self.launches

    def result(self, m, ms, samples):
        nbytes = self.wbytes + m * self.K * 2 + m * self.N * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        return {"us": round(ms * 1e3, 2), "GBs": round(gbs, 1), "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                "TFLOPs": round(2 * m * self.N * self.K / (ms * 1e-3) / 1e12, 1), "bytes": nbytes,
                "us_by_round": [round(v * 1e3, 2) for v in samples]}

    def floor_result(self, ms, samples):
        gbs = self.floor_bytes / (ms * 1e-3) / 1e9
        return {"us": round(ms * 1e3, 2), "GBs": round(gbs, 1), "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                "bytes": self.floor_bytes, "kernel": "k_read_floor (qg_read_floor: 4 x 512-thread workgroups per CU, 4 x 1 KB wave requests in flight)",
                "us_by_round": [round(v * 1e3, 2) for v in samples]}

    @staticmethod
    def kernel_name(m):
        return ("k_w4_gemv1 (one row: 32 columns x 8 waves, global->LDS copies, 16x16x32 bf16 MFMA)" if m == 1
                else "k_w4_decode<RP=16,CT=4,G=128,uint4>")


def run_w4a16(torch, lib, _lib, dev, rows=(1, 16, 2048), copies=12):
    """Benchmark configuration 2 at the given row counts, each the median of three
    samples: decode rows (<= 16) through DecodeW4's rotated graphs, prefill
    (2048) over one weight with graph replays of 10 launches; for 2048 also the
    reference's default ``dequant`` method (this library's unpack to bf16, then
    the library GEMM) with HIP events over eager calls."""
    from rdna2_ops import int4_weight_gemm_v07 as w4
    out = {}
    dec = [m for m in rows if m <= 16]
    if dec:
        d = DecodeW4(torch, lib, _lib, dev, copies=copies)
        for m in dec:
            samples = [d.time(m) for _ in range(3)]
            out[m] = d.result(m, statistics.median(samples), samples)
        fs = [d.time_floor() for _ in range(3)]
        out["read_floor"] = d.floor_result(statistics.median(fs), fs)
    if 2048 in rows:
        N, K, G, m = 14336, 4096, 128, 2048
        gen, ps = _w4_weights(torch, dev, 1)
        p0 = ps[0]
        wbytes = p0.data.numel() * 4 + p0.scales.numel() * 2 + p0.zeros.numel() * 4
        a = torch.randn(m, K, generator=gen).to(torch.bfloat16).to(dev)
        y = torch.empty(m, N, dtype=torch.bfloat16, device=dev)
        P = _lib.ptr

        wsb = int(lib.qg_w4a16_gemm_workspace_bytes(m, N, K, G, p0.flags))
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)

        def call(i, stream):
            _lib.check(lib.qg_w4a16_gemm(P(a), _lib.BF16, K, m, K, P(p0.data), N, G, p0.flags, P(p0.scales),
                                         _lib.BF16, P(p0.zeros), None, 0, P(y), _lib.BF16, P(ws), wsb, stream),
                       "w4a16")
        ms = statistics.median([_graph_time(torch, call, 10, replays=2) for _ in range(3)])
        bytes_ = wbytes + m * K * 2 + m * N * 2
        out[m] = {"us": round(ms * 1e3, 2), "GBs": round(bytes_ / (ms * 1e-3) / 1e9, 1),
                  "frac_hbm_peak": round(bytes_ / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                  "TFLOPs": round(2 * m * N * K / (ms * 1e-3) / 1e12, 1),
                  "frac_bf16_peak": round(2 * m * N * K / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                  "bytes": bytes_}

        def dequant():
            return w4.int4_linear_a16(a, p0, method="dequant")
        for _ in range(3):
            dequant()
        torch.cuda.synchronize()
        samples = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                dequant()
            e1.record()
            torch.cuda.synchronize()
            samples.append(e0.elapsed_time(e1) / 10)
        dms = statistics.median(samples)
        out["2048_dequant_method"] = {"us": round(dms * 1e3, 2),
                                      "TFLOPs": round(2 * m * N * K / (dms * 1e-3) / 1e12, 1)}
    return out


def run_fp8(torch, lib, _lib, dev):
    """Benchmark configuration 3: e4m3 weights with per-channel absmax/448 scales,
    bf16 activations M 4096, K 3072, N 3072 and 12288, bf16 out. Timed per
    call of qg_fp8w_gemm: on these grids the 2-byte ping-pong GEMM with the fp8
    W stages converted exactly to bf16 in registers."""
    from rdna2_ops import fp8_weight_gemm_v06 as f8
    gen = torch.Generator().manual_seed(3)
    res = {}
    for n in (3072, 12288):
        m, k = 4096, 3072
        codes, sc = f8.quantize_weight_e4m3((torch.randn(n, k, generator=gen) * 0.02).to(dev))
        a = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
        y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        P = _lib.ptr
        # workspace: packed operands only when they are not canonical
        wsb = lib.qg_fp8w_gemm_workspace_bytes(P(a), k, 1, P(codes), k, 1, m, n, k)
        ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=dev)

        def call(i, stream, a=a, y=y, codes=codes, sc=sc, n=n, ws=ws, wsb=wsb):
            _lib.check(lib.qg_fp8w_gemm(P(a), _lib.BF16, k, 1, m, k, P(codes), _lib.E4M3, k, 1, n, P(sc), None, 0,
                                        P(y), _lib.BF16, P(ws) if wsb else None, wsb, stream), "fp8w")
        ms = statistics.median([_graph_time(torch, call, 10, replays=2) for _ in range(3)])
        tf = 2 * m * n * k / (ms * 1e-3) / 1e12
        res[n] = {"us": round(ms * 1e3, 1), "TFLOPs": round(tf, 1), "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
        # the reference's decode method: this library's fp8 -> bf16 decode,
        # then the library (hipBLASLt) GEMM, HIP events over eager calls;
        # without the per-channel scale (the reference has none; with it the
        # method adds fp32 passes over the output that the fused epilogue avoids)
        def decode(a=a, codes=codes):
            return f8.fp8_weight_gemm(a, codes, method="decode")
        for _ in range(3):
            decode()
        torch.cuda.synchronize()
        dsamples = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                decode()
            e1.record()
            torch.cuda.synchronize()
            dsamples.append(e0.elapsed_time(e1) / 10)
        dms = statistics.median(dsamples)
        res[f"{n}_decode_method_unscaled"] = {"us": round(dms * 1e3, 1), "TFLOPs": round(2 * m * n * k / (dms * 1e-3) / 1e12, 1)}
    return res


def run_moe(torch, dev, iters=20):
    """Secondary: benchmark configuration 4, MoE prefill (4096 tokens, top-8 of 64
    experts, hidden 2048, F 768) through rdna2_ops.moe_int8: routing, dispatch,
    x quantization, grouped gate/up GEMM + SiLU*mul, h quantization, grouped
    down GEMM * routing weight, combine. Ops count the routed rows only
    (309.2 G, no padding); bytes are the algorithmic ~487 MB (weights once,
    int8 activations, bf16 h written and read, bf16 out)."""
    from rdna2_ops import moe_int8, synthetic
    c = synthetic.cfg4()
    prep = moe_int8.prepare_moe_weights(c.w_gate.to(dev), c.w_up.to(dev), c.w_down.to(dev))
    x, lg = c.x.to(dev), c.logits.to(dev)
    for _ in range(3):
        moe_int8.moe_int8_forward(x, lg, prep, top_k=c.top_k)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream(dev)
    samples = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(iters):
            moe_int8.moe_int8_forward(x, lg, prep, top_k=c.top_k)
        e1.record(s)
        e1.synchronize()
        samples.append(e0.elapsed_time(e1) / iters)
    ms = statistics.median(samples)
    t, h = c.x.shape
    e, f = c.w_gate.shape[0], c.w_gate.shape[1]
    ops = 2.0 * t * c.top_k * (h * 2 * f + f * h)
    nbytes = e * 3 * f * h + t * h * 2 + t * c.top_k * h + 2 * (t * c.top_k * f * 2) + t * h * 2
    tops = ops / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 1), "TOPS": round(tops, 1), "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4),
            "GBs_algorithmic": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "ops": ops, "bytes": nbytes}


def run_w4a8(torch, dev, iters=20):
    """Secondary (no benchmark configuration): W4A8 on the int8 MFMA,
    int4_linear_a8 float output, on the cfg0 shape with g128 affine nk
    weights and on the reference's own check shape (M 1061, g32, kn).
    TOPS = 2 M N K per call; HIP events over `iters` back-to-back calls."""
    from rdna2_ops import int4_weight_gemm_v07 as w4
    res = {}
    for label, (m, n, k, g, layout) in (("cfg0_shape_g128", (4096, 3072, 3072, 128, "nk")),
                                        ("moss_1061_g32_kn", (1061, 3072, 3072, 32, "kn"))):
        gen = torch.Generator(device=dev).manual_seed(7)
        w = torch.randn(n, k, device=dev, generator=gen) * 0.01
        p = w4.pack_int4(w, group_size=g, symmetric=False, layout=layout)
        a = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=dev, generator=gen)
        sa = torch.rand(m, device=dev, generator=gen) * 0.01
        for _ in range(3):
            w4.int4_linear_a8(a, p, sa)
        torch.cuda.synchronize()
        s = torch.cuda.current_stream(dev)
        samples = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(iters):
                w4.int4_linear_a8(a, p, sa)
            e1.record(s)
            e1.synchronize()
            samples.append(e0.elapsed_time(e1) / iters)
        us = statistics.median(samples) * 1e3
        tops = 2.0 * m * n * k / (us * 1e-6) / 1e12
        _, md = w4.int4_linear_a8(a, p, sa, return_kernel=True)
        res[label] = {"us": round(us, 1), "TOPS": round(tops, 1), "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4),
                      "shape": [m, n, k], "group": g, "kernel": md["variant"], "tile": md["tile"]}
    return res


# The reference's fused INT8 GEMM on the four MOSS production shapes (M 1061,
# fp32 out, rounding="separate", no bias, weight.T view) on its gfx1030 box, ms
# (rdna2-ops/results/int8_gemm_moss_shapes_v05.json rows 0-3,
# RDNA2_OPTIMIZATION_GUIDE_KO.md:1135-1138): context only, other hardware.
MOSS_SHAPES = ((3072, 3072, 0.698), (9216, 3072, 1.869), (16384, 3072, 3.302), (3072, 8192, 1.932))


def run_moss(torch, lib, _lib, dev, iters=50):
    """Secondary: the MOSS INT8 production calls (M = 1061 tokens; (N, K) of
    the four projections), the shapes the reference's own INT8 numbers are
    quoted on. Per shape:
      kernel  — qg_int8_gemm on preallocated buffers (int8 rows, the weight.T
                view, fp32 out, order F without bias = the reference's
                rounding="separate" contract), HIP-graph replays of 50 launches;
      int8_gemm_dequant — the Python operator as MOSS calls it (fresh output,
                validation, ctypes), back-to-back calls timed with events;
      comfy_eager — the product step of comfy_int8.int8_linear's intercepted
                fp32 path: int8_gemm_dequant with epilogue_order="eager" (the
                same launch: orders F and E coincide for fp32 output);
      w8a8_linear — this library's quantizer + GEMM on fp32 x (qg_w8a8_linear);
      w8a8_linear_convrot256_residual — the same with the MOSS linear's
                opt-in fusions (qg_w8a8_linear_ex): the ConvRot g256 rotation
                in the quantizer launch and an fp32 residual x per-channel
                scale in the GEMM epilogue.
    TOPS = 2 M N K per call."""
    from rdna2_ops.int8_gemm import int8_gemm_dequant, w8a8_linear
    from rdna2_ops.quantize import quantize_int8_rowwise
    m = 1061
    gen = torch.Generator().manual_seed(11)
    res = {}
    s = torch.cuda.current_stream(dev)

    def events(fn):
        samples = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(iters):
                fn()
            e1.record(s)
            e1.synchronize()
            samples.append(e0.elapsed_time(e1) / iters)
        return statistics.median(samples)

    for n, k, ref_ms in MOSS_SHAPES:
        x = torch.randn(m, k, generator=gen).to(dev)
        wq, ws = quantize_int8_rowwise((torch.randn(n, k, generator=gen) * 0.02).to(dev))
        ws = ws.reshape(-1).contiguous()
        xq, xs = quantize_int8_rowwise(x)
        xs = xs.reshape(-1).contiguous()
        out = torch.empty((m, n), dtype=torch.float32, device=dev)
        P = _lib.ptr

        def kernel(i, stream):
            _lib.check(lib.qg_int8_gemm(P(xq), k, 1, P(wq), 1, k, m, n, k, P(xs), P(ws), n, None, 0, P(out),
                                        _lib.F32, 0, None, 0, stream), "moss gemm")

        k_ms = statistics.median(_graph_time(torch, kernel, iters) for _ in range(3))
        rhs = wq.T
        api = lambda: int8_gemm_dequant(xq, rhs, xs, ws, None, rounding="separate")
        eager = lambda: int8_gemm_dequant(xq, rhs, xs, ws, None, out_dtype=torch.float32, epilogue_order="eager")
        lin = lambda: w8a8_linear(x, wq, ws, out_dtype=torch.float32)
        # the MOSS linear's opt-in fusions (qg_w8a8_linear_ex): ConvRot g256
        # prologue, fp32 residual with a per-channel scale (4-wave kernel)
        res_in = torch.randn(m, n, generator=gen).to(dev)
        res_sc = (torch.rand(n, generator=gen) + 0.5).to(dev)
        lin_ex = lambda: w8a8_linear(x, wq, ws, out_dtype=torch.float32, convrot_groupsize=256,
                                     residual=res_in, residual_scale=res_sc)
        for f in (api, eager, lin, lin_ex):
            f()
        torch.cuda.synchronize()
        api_ms, eager_ms, lin_ms, ex_ms = events(api), events(eager), events(lin), events(lin_ex)
        ops = 2.0 * m * n * k
        tops = ops / (k_ms * 1e-3) / 1e12
        res[f"{m}x{n}x{k}"] = {
            "kernel_us": round(k_ms * 1e3, 2), "kernel_tops": round(tops, 1),
            "kernel_frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4),
            "int8_gemm_dequant_us": round(api_ms * 1e3, 2), "comfy_eager_product_us": round(eager_ms * 1e3, 2),
            "w8a8_linear_us": round(lin_ms * 1e3, 2),
            "w8a8_linear_tops": round(ops / (lin_ms * 1e-3) / 1e12, 1),
            "w8a8_linear_convrot256_residual_us": round(ex_ms * 1e3, 2),
            "reference_gfx1030_ms": ref_ms}
    return res


def run_clock(torch, lib, _lib, dev, ms_target=20.0):
    """The shader clock an int8 MFMA load sustains on this board (qg_mfma_clock):
    every CU runs 8 waves issuing v_mfma_i32_32x32x32_i8 back to back for about
    ``ms_target`` ms, in three modes (constant operands; random operands; random
    operands plus the INT8 GEMM's LDS fragment reads). Per mode: the median over
    waves of shader-clock cycles / 100 MHz ticks (MHz), the SIMD's MFMA issue
    interval, and the int8 throughput that rate gives at that clock."""
    res = {}
    out = torch.zeros(256 * 8 * 2, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev)
    for mode, label in ((0, "constant_operands"), (1, "random_operands"), (2, "random_operands_gemm_lds_reads")):
        iters = 20000
        for _ in range(2):  # warm-up launch, then one sized to ms_target
            _lib.check(lib.qg_mfma_clock(mode, iters, _lib.ptr(out), s.cuda_stream), "qg_mfma_clock")
            torch.cuda.synchronize()
            o = out.cpu().numpy().view("uint32").reshape(-1, 2).astype("float64")
            us = float(statistics.median(o[:, 1])) / 100.0
            iters = max(1000, min(1 << 22, int(iters * ms_target * 1e3 / max(us, 1.0))))
        mhz = statistics.median((o[:, 0] / o[:, 1] * 100.0).tolist())
        # two waves per SIMD share the pipe: per-SIMD interval = the longer
        # wave's cycles / all MFMAs the SIMD issued
        cyc = float(o[:, 0].max())
        per_mfma_simd = cyc / (iters * 6 * 2)
        tops = 256 * 4 * 65536.0 / per_mfma_simd * mhz * 1e6 / 1e12
        res[label] = {"mhz": round(mhz, 1), "cycles_per_mfma_per_simd": round(per_mfma_simd, 2),
                      "iters": iters, "wave_us_median": round(float(statistics.median(o[:, 1])) / 100.0, 1),
                      "int8_tops_at_that_rate": round(tops, 1),
                      "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4)}
    return res


def run_stages(torch, lib, _lib, dev, launches=20):
    """Where the cycles of the INT8 GEMM go (qg_int8_gemm_stages: the ping-pong
    kernel with shader-clock stamps), at configuration 0 and the three chain
    shapes. Per shape, medians over waves (and stages) of the last of
    ``launches`` back-to-back launches, in shader-clock cycles: the wave's
    life, the prologue (entry to the first stage), the main loop, the epilogue
    (to its stores' completion), the stage, and the stage's phases per wave
    group; the clock (cycles / 100 MHz ticks) and the MFMA-busy fraction of a
    SIMD over the wave's life (48 MFMAs per stage and SIMD, 32 cycles each)."""
    import numpy as np
    res = {}
    gen = torch.Generator().manual_seed(5)
    shapes = {"cfg0": (4096, 3072, 3072), "qkv": (4096, 9216, 3072), "down": (4096, 3072, 12288)}
    s = torch.cuda.current_stream(dev)
    P = _lib.ptr
    for name, (m, n, k) in shapes.items():
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=gen).to(dev)
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=gen).to(dev)
        sa = (torch.rand(m, generator=gen) * 0.01 + 1e-3).to(dev)
        sw = (torch.rand(n, generator=gen) * 0.01 + 1e-3).to(dev)
        bias = (torch.randn(n, generator=gen) * 0.01).half().to(dev)
        out = torch.empty((m, n), dtype=torch.float16, device=dev)
        grid = min(256, -(-m // 256) * -(-n // 192))
        words = grid * 8 * 272
        st = torch.zeros(words, dtype=torch.int32, device=dev)
        for _ in range(launches):
            _lib.check(lib.qg_int8_gemm_stages(P(a), P(w), m, n, k, P(sa), P(sw), P(bias), P(out), P(st), words,
                                               s.cuda_stream), "qg_int8_gemm_stages")
        torch.cuda.synchronize()
        raw = st.cpu().numpy().view(np.uint32).reshape(grid, 8, 272).astype(np.int64)
        S = int(raw[0, 0, 263])
        ext = raw[:, :, 256:]
        life = (ext[:, :, 3] - ext[:, :, 0]) % 2 ** 32
        ticks = (ext[:, :, 5] - ext[:, :, 4]) % 2 ** 32
        pts = raw[:, :, :256].reshape(grid, 8, 4, 64)
        X, Y = pts[:, :4], pts[:, 4:]
        Sx = min(S, 64)

        def med(v):
            return int(np.median(np.asarray(v) % 2 ** 32))
        r = {"shape": [m, n, k], "stages": S, "tiles_per_workgroup": -(-(-(-m // 256) * -(-n // 192)) // grid),
             "mhz": round(float(np.median(life / ticks * 100.0)), 1),
             "wave_cycles": med(life),
             # entry to the first stage (one tile per workgroup and at most 64
             # stages: otherwise stage 0's stamp belongs to a later tile / stage)
             "prologue": (med(X[:, :, 1, 0] - ext[:, :4, 0])
                          if S <= 64 and -(-m // 256) * -(-n // 192) <= grid else None),
             "epilogue": med(ext[:, :, 2] - ext[:, :, 1]),
             "stage": med(X[:, :, 1, 2:Sx] - X[:, :, 1, 1:Sx - 1]),
             "mfma_ideal_stage": 48 * 32,
             "X_mfma_issue": med(X[:, :, 2, 1:Sx - 1] - X[:, :, 1, 1:Sx - 1]),
             "X_wait_B1": med(X[:, :, 3, 1:Sx - 1] - X[:, :, 2, 1:Sx - 1]),
             "X_lds_reads_and_copies": med(X[:, :, 0, 2:Sx] - X[:, :, 3, 1:Sx - 1]),
             "X_wait_B0": med(X[:, :, 1, 1:Sx - 1] - X[:, :, 0, 1:Sx - 1]),
             "Y_lds_reads_and_copies": med(Y[:, :, 1, 1:Sx - 1] - Y[:, :, 0, 1:Sx - 1]),
             "Y_wait_copies_B1": med(Y[:, :, 2, 1:Sx - 1] - Y[:, :, 1, 1:Sx - 1]),
             "Y_mfma_issue": med(Y[:, :, 3, 1:Sx - 1] - Y[:, :, 2, 1:Sx - 1]),
             "Y_to_B0": med(Y[:, :, 0, 2:Sx] - Y[:, :, 3, 1:Sx - 1])}
        tiles = -(-m // 256) * -(-n // 192)
        r["mfma_busy_of_wave_life"] = round(48 * 32 * S * tiles / grid / r["wave_cycles"], 4)
        res[name] = r
    return res


def traffic_record(name):
    """HBM bytes per launch of a kernel, from rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE runs (each scaled by the same counter's reading for a plain copy
    of known size) recorded in profiles/<name>, with where they came from;
    (None, None) if absent. The counters cannot be read inside this process,
    so the figure is the one of the last profiling run of that kernel."""
    path = ROOT / "profiles" / name
    try:
        rec = json.loads(path.read_text())
        return rec["hbm_bytes_per_launch"], {"file": "profiles/" + name, "kernel": rec.get("kernel"),
                                             "measured": rec.get("measured")}
    except (OSError, KeyError, ValueError):
        return None, None


class ClockSampler:
    """Reads the GPU's GFX (shader) clock with amdsmi from a host thread while
    the same chain runs back to back for ``seconds``. amdsmi's clock values
    refresh about once per second, far slower than one timed round, so the
    clock is read over this separate sustained window rather than during the
    rounds; samples of the first second (the previous, idle reading) are
    dropped. Per-XCD clocks come from the GPU metrics table when it has them.
    Reports nothing if amdsmi cannot read the clock on this box."""

    def __init__(self, period_s=0.05):
        self.period = period_s
        self.samples = []
        self.error = None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self._smi = amdsmi
            self._handle = amdsmi.amdsmi_get_processor_handles()[0]
            amdsmi.amdsmi_get_clock_info(self._handle, amdsmi.AmdSmiClkType.GFX)
        except Exception as e:  # no amdsmi, no permission, no device
            self._smi = None
            self.error = f"{type(e).__name__}: {e}"

    def _read(self):
        smi = self._smi
        try:
            m = smi.amdsmi_get_gpu_metrics_info(self._handle)
            xcd = [float(v) for v in (m.get("current_gfxclks") or []) if isinstance(v, (int, float)) and v > 0]
            if xcd:
                return sum(xcd) / len(xcd)
        except Exception:
            pass
        info = smi.amdsmi_get_clock_info(self._handle, smi.AmdSmiClkType.GFX)
        return float(info.get("clk", info.get("cur_clk", 0)))

    def sustained(self, torch, step, seconds=2.5, settle=1.0):
        """Run ``step()`` back to back for ``seconds`` and sample the clock."""
        if self._smi is None:
            return self
        import threading
        stop = threading.Event()
        t0 = time.perf_counter()

        def run():
            while not stop.is_set():
                try:
                    v = self._read()
                except Exception as e:
                    self.error = f"{type(e).__name__}: {e}"
                    return
                if time.perf_counter() - t0 >= settle:
                    self.samples.append(v)
                stop.wait(self.period)
        th = threading.Thread(target=run, daemon=True)
        th.start()
        while time.perf_counter() - t0 < seconds:
            for _ in range(20):
                step()
            torch.cuda.synchronize()
        stop.set()
        th.join()
        return self

    def summary(self):
        if not self.samples:
            return {"source": "amdsmi GFX clock", "available": False, "error": self.error}
        s = sorted(self.samples)
        return {"source": "amdsmi GFX clock (mean of the XCD clocks), sampled every 50 ms while the chain "
                          "ran back to back for 2.5 s after the timed rounds (first second dropped: amdsmi "
                          "refreshes about once per second)",
                "available": True, "median_mhz": round(s[len(s) // 2], 1), "min_mhz": round(s[0], 1),
                "max_mhz": round(s[-1], 1), "samples": len(s)}


def alternating_rounds(items, rounds):
    """The reference's timing protocol (rdna2-ops/bench_int8_gemm.py:259-268):
    every round times every item once, in list order on even rounds and in
    reverse order on odd ones; each item's result is the median over rounds.
    ``items`` maps a name to a callable returning one sample (ms)."""
    samples = {name: [] for name in items}
    names = list(items)
    for r in range(rounds):
        for name in (names if r % 2 == 0 else names[::-1]):
            samples[name].append(items[name]())
    return {name: (statistics.median(v), v) for name, v in samples.items()}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path; run with --gpus 1",
              file=sys.stderr, flush=True)
        sys.exit(2)
    if args.rounds < 1:
        print("--rounds must be at least 1", file=sys.stderr, flush=True)
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
    if args.only:
        runs = {"w4a16": lambda: run_w4a16(torch, lib, _lib, dev), "fp8": lambda: run_fp8(torch, lib, _lib, dev),
                "moe": lambda: run_moe(torch, dev), "w4a8": lambda: run_w4a8(torch, dev),
                "cfg0": lambda: Cfg0(torch, lib, _lib, quantize_int8_rowwise, synthetic, dev).profile_run(),
                "decode": lambda: run_w4a16(torch, lib, _lib, dev, rows=(1,)),
                "moss": lambda: run_moss(torch, lib, _lib, dev),
                "clock": lambda: run_clock(torch, lib, _lib, dev),
                "stages": lambda: run_stages(torch, lib, _lib, dev)}
        res = runs[args.only]()
        print(json.dumps({"only": args.only, "result": res}), flush=True)
        return
    # the chain runs on a stream of its own (default priority)
    chain_stream = torch.cuda.Stream(device=dev)
    chain = Chain(torch, lib, _lib, quantize_int8_rowwise, synthetic.cfg1(), dev, stream=chain_stream)
    for _ in range(args.warmup):
        chain.step()
    torch.cuda.synchronize()

    events = []

    def chain_round(instrumented):
        """Exactly --steps chain steps between two synchronisations; ms per step.
        Instrumented rounds bracket every GEMM launch with a pair of timing
        events (the roofline's per-launch durations); the plain rounds give
        ``value``: the six event records per step cost about 16 us of a
        ~430 us step (measured on MI355X, same process). The events are created
        before the timed region and the garbage collector is paused inside it:
        creating events there made the host, not the GPU, the bottleneck of one
        round in several (host enqueue 0.77 ms per step against 0.04)."""
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        pairs = iter([(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(3 * args.steps)]) if instrumented else None
        torch.cuda.synchronize()
        gc.disable()
        try:
            start.record(chain.stream)
            for _ in range(args.steps):
                if instrumented:
                    chain.step(events, pairs)
                else:
                    chain.step()
            stop.record(chain.stream)
            torch.cuda.synchronize()
        finally:
            gc.enable()
        return start.elapsed_time(stop) / args.steps

    items = {"chain": lambda: chain_round(False), "chain_gemm_events": lambda: chain_round(True)}
    cfg0 = decode = None
    if not args.no_secondary:
        cfg0 = Cfg0(torch, lib, _lib, quantize_int8_rowwise, synthetic, dev)
        decode = DecodeW4(torch, lib, _lib, dev)
        items.update(cfg0_gemm=cfg0.time_gemm, cfg0_quant=cfg0.time_quant,
                     w4a16_m1=lambda: decode.time(1), w4a16_m16=lambda: decode.time(16),
                     read_floor=decode.time_floor)
    timed = alternating_rounds(items, args.rounds)
    clock = ClockSampler().sustained(torch, chain.step)
    ms, chain_samples = timed["chain"]
    ops = chain.ops()
    value = ops / (ms * 1e-3) / 1e12

    # the dominant kernel: each GEMM launch of the chain bracketed by events on
    # its stream, every step of every round
    per_layer = {}
    for i, e0, e1 in events:
        per_layer.setdefault(i, []).append(e0.elapsed_time(e1))
    gemm_ms_per_step = sum(statistics.median(v) for v in per_layer.values())
    achieved = ops / (gemm_ms_per_step * 1e-3) / 1e12
    layer_info = {}
    for i, name in enumerate(("qkv", "up_gelu", "down")):
        L = chain.layers[i]
        t = statistics.median(per_layer[i])
        layer_info[name] = {"us": round(t * 1e3, 2),
                            "tops": round(2 * chain.m * L["n"] * L["k"] / (t * 1e-3) / 1e12, 1)}
    traffic, traffic_src = traffic_record("int8_gemm_cfg1_chain_traffic.json")

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TOPS", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized per channel)",
        "config": {"workload": "cfg1 DiT-block W8A8 INT8 GEMM chain: M=4096, hidden=3072; "
                               "QKV N=9216; MLP up N=12288 + GELU-tanh; MLP down K=12288->N=3072; "
                               "per-token int8 quant prologue on each GEMM; fp16 in/out",
                   "tokens": chain.m, "hidden": 3072, "ops_per_step": ops},
        "protocol": {"rounds": args.rounds, "order": "alternating (forward on even rounds, reverse on odd)",
                     "statistic": "median over rounds", "steps_per_round": args.steps,
                     "chain_ms_per_step_by_round": [round(v, 5) for v in chain_samples],
                     "value_from": "plain chain rounds (no events between launches)",
                     "roofline_from": "instrumented chain rounds (an event pair around every GEMM launch on "
                                      "the chain's stream), alternated with the plain rounds",
                     "instrumented_chain_ms_per_step_by_round": [round(v, 5) for v in timed["chain_gemm_events"][1]]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_INT8_TOPS,
                     "unit": "TOPS", "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "k_i8_gemm_pp<256x192 tile, 8 waves> (int8 MFMA GEMM, ping-pong main loop, fused epilogue, persistent grid)",
                     "per_launch": layer_info},
        "clock": clock.summary(),
    }
    if not args.no_secondary:
        g_ms, g_s = timed["cfg0_gemm"]
        q_ms, q_s = timed["cfg0_quant"]
        cfg0_ops = cfg0.ops()
        g_tops = cfg0_ops / (g_ms * 1e-3) / 1e12
        c0_traffic, c0_src = traffic_record("int8_gemm_cfg0_traffic.json")
        # the >= 60 % bar of the metric is quoted on configuration 0
        line["roofline_cfg0"] = {
            "bound": "mfma", "achieved": round(g_tops, 1), "peak": PEAK_INT8_TOPS, "unit": "TOPS",
            "frac": round(g_tops / PEAK_INT8_TOPS, 4), "traffic": c0_traffic, "traffic_source": c0_src,
            "kernel": "k_i8_gemm_pp<256x192 tile, 8 waves> (M=4096, N=K=3072, fp16 out, order F + bias)",
            "us_per_launch": round(g_ms * 1e3, 2), "us_by_round": [round(v * 1e3, 2) for v in g_s]}
        sec = {"cfg0_gemm_us": round(g_ms * 1e3, 2), "cfg0_gemm_tops": round(g_tops, 1),
               "cfg0_gemm_frac_int8_peak": round(g_tops / PEAK_INT8_TOPS, 4),
               "cfg0_quant_us": round(q_ms * 1e3, 2),
               "cfg0_quant_gbs": round(cfg0.quant_bytes() / (q_ms * 1e-3) / 1e9, 1),
               "cfg0_w8a8_linear_tops": round(cfg0_ops / ((g_ms + q_ms) * 1e-3) / 1e12, 1)}
        w4 = {m: decode.result(m, *timed[f"w4a16_m{m}"]) for m in (1, 16)}
        dec = w4[1]
        d_traffic, d_src = traffic_record("w4a16_decode_cfg2_traffic.json")
        # second half of the headline metric: W4A16 decode (M = 1) HBM GB/s
        line["roofline_w4a16_decode"] = {
            "bound": "hbm", "achieved": dec["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": dec["frac_hbm_peak"], "traffic": d_traffic, "traffic_source": d_src,
            "kernel": decode.kernel_name(1) + " (M=1, K 4096, N 14336, g128 uint4, "
                      f"{decode.copies} rotated weight copies)",
            "us_per_launch": dec["us"], "us_by_round": dec["us_by_round"], "algorithmic_bytes": dec["bytes"]}
        floor = decode.floor_result(*timed["read_floor"])
        line["roofline_w4a16_decode"]["read_floor"] = floor
        line["roofline_w4a16_decode"]["frac_of_read_floor"] = round(floor["us"] / dec["us"], 4)
        sec["w4a16_m1"] = w4[1]
        sec["w4a16_m16"] = w4[16]
        pre = run_w4a16(torch, lib, _lib, dev, rows=(2048,))
        sec["w4a16_prefill_m2048"] = pre[2048]
        sec["w4a16_prefill_m2048_dequant_method"] = pre["2048_dequant_method"]
        sec["fp8_cfg3"] = run_fp8(torch, lib, _lib, dev)
        sec["moe_cfg4"] = run_moe(torch, dev)
        sec["w4a8"] = run_w4a8(torch, dev)
        sec["moss_int8"] = run_moss(torch, lib, _lib, dev)
        line["secondary"] = sec
    if not args.no_cpu_baseline:
        from oracle.cpu_baseline import cpu_model, time_cfg1_chain
        cpu_ops, cpu_s, threads, sample = time_cfg1_chain(rows=args.cpu_rows, seconds=args.cpu_seconds)
        # the reference's own benchmark setting: 2 threads (bench_int8_gemm.py:54), a smaller sample
        ops2, s2, _, sample2 = time_cfg1_chain(rows=min(512, args.cpu_rows), threads=2,
                                               seconds=min(4.0, args.cpu_seconds))
        line["cpu_baseline"] = {"value": round(cpu_ops / 1e12, 4), "unit": "TOPS", "cores": threads,
                                "kind": "port", "sample": sample, "seconds_per_sample": round(cpu_s, 3),
                                "cpu_model": cpu_model(),
                                "threads_2": {"value": round(ops2 / 1e12, 4), "unit": "TOPS", "sample": sample2}}
        if not args.no_secondary:
            from oracle.cpu_baseline import time_w4a16_decode
            gbs, sec_s, threads, sample = time_w4a16_decode(seconds=min(5.0, args.cpu_seconds))
            line["cpu_baseline_w4a16_decode"] = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads,
                                                 "kind": "port", "sample": sample}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
