"""Reference torch CPU formulation of the hot path, timed as bench.py's
``cpu_baseline`` leg (test/measurement infrastructure only — never the product).

W8A8 (cfg0 / cfg1), as restated in the benchmark's CPU-baseline formulation:
  per-token quantize  amax -> /127 -> x/step -> round (half-even) -> clamp -> int8
  torch._int_mm       exact int32 on the CPU
  epilogue order F    f32(acc) * f32(sa*sw), + bias in fp32 (separate ops), GELU-tanh
                      for the MLP up projection, one rounding to fp16
(rdna2-ops/rdna2_ops/int8_gemm.py:53-63, fp8_weight_gemm_v06.py:76-92/:193).
"""
from __future__ import annotations

import os
import time

import torch


def _quant(x):
    x = x.float()
    step = torch.clamp(x.abs().amax(1, keepdim=True) / 127.0, min=1e-20)
    return torch.round(x / step).clamp(-127, 127).to(torch.int8), step


def w8a8_linear_cpu(x, wq_t, ws, bias, activation=None):
    """x fp16 [M,K]; wq_t int8 [K,N] (contiguous); ws fp32 [N]; bias fp16 [N]."""
    xq, xs = _quant(x)
    acc = torch._int_mm(xq, wq_t)
    v = acc.float() * (xs * ws.reshape(1, -1))
    v = v + bias.float().reshape(1, -1)
    if activation == "gelu_tanh":
        v = torch.nn.functional.gelu(v, approximate="tanh")
    return v.to(torch.float16)


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", read from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_cfg1_chain(rows=4096, hidden=3072, threads=None, seconds=10.0, seed=1):
    """Time the cfg1 chain (QKV, up+GELU, down) on ``rows`` tokens on the CPU,
    repeating whole passes for about ``seconds`` (at least two).

    Returns (ops_per_second, median_seconds_per_pass, threads, sample description).
    The weights are random int8 of the real shapes (their values do not change
    the CPU work); the activations are the first ``rows`` tokens' worth of a
    seeded N(0,1) input.
    """
    threads = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, hidden, generator=g).to(torch.float16)
    layers = []
    for n, k, act in ((3 * hidden, hidden, None), (4 * hidden, hidden, "gelu_tanh"), (hidden, 4 * hidden, None)):
        wq_t = torch.randint(-127, 128, (k, n), generator=g, dtype=torch.int8)
        ws = torch.rand(n, generator=g) * 1e-3
        b = (torch.randn(n, generator=g) * 0.01).to(torch.float16)
        layers.append((wq_t, ws, b, act))

    def one_pass():
        q = w8a8_linear_cpu(x, *layers[0])
        h = w8a8_linear_cpu(x, *layers[1])
        y = w8a8_linear_cpu(h, *layers[2])
        return q, y

    one_pass()  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 2 or time.perf_counter() - start < seconds:
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
    times.sort()
    sec = times[len(times) // 2]
    ops = 2 * rows * hidden * (3 * hidden + 4 * hidden + 4 * hidden)
    return ops / sec, sec, threads, (f"cfg1 chain on {rows} of 4096 tokens, torch CPU int8 (_int_mm), "
                                     f"median of {len(times)} passes in {time.perf_counter() - start:.1f} s")


def time_w4a16_decode(n=14336, k=4096, group=128, seconds=5.0, seed=2, threads=None):
    """CPU formulation of the W4A16 decode (benchmark configuration 2, M = 1):
    dequantise the uint4 weight (q - z) * s to fp32, F.linear in fp32, cast to
    bf16 — as restated in the benchmark's CPU-baseline formulation. Repeated for about
    ``seconds``; returns (GB/s of the packed weight streamed, median seconds,
    threads, sample description)."""
    threads = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (n, k // group), generator=g, dtype=torch.uint8)
    s = (torch.rand(n, k // group, generator=g) * 1e-3).to(torch.bfloat16)
    a = torch.randn(1, k, generator=g).to(torch.bfloat16)

    def once():
        w = (q.view(n, k // group, group).float() - z.float()[..., None]) * s.float()[..., None]
        return torch.nn.functional.linear(a.float(), w.view(n, k)).to(torch.bfloat16)

    once()
    times = []
    start = time.perf_counter()
    while len(times) < 2 or time.perf_counter() - start < seconds:
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    times.sort()
    sec = times[len(times) // 2]
    wbytes = n * k // 2 + n * (k // group) * 2 + n * ((k // group + 7) // 8) * 4
    return wbytes / sec / 1e9, sec, threads, (f"W4A16 M=1 K={k} N={n} g{group}, torch CPU dequant + fp32 "
                                               f"F.linear, median of {len(times)} passes")
