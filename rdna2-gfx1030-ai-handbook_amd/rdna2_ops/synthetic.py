"""Seeded synthetic inputs of the benchmark configurations.

Every tensor is drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in
the fixed order written below, so a CPU checker and the GPU see identical bytes.
The benchmark fixes cfg0's seed (0); seeds 1-4 of cfg1-cfg4 are this build's choice.
There are no datasets or checkpoints: all data is synthetic.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Cfg0:
    x: torch.Tensor       # fp16 [M, K], N(0,1) with 0.1 % outliers x20
    w: torch.Tensor       # fp16 [N, K], N(0, 0.02)
    bias: torch.Tensor    # fp16 [N], N(0, 0.01)


def cfg0(m=4096, n=3072, k=3072, seed=0) -> Cfg0:
    """W8A8 INT8 linear (benchmark configuration 0)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    outlier = torch.rand(m, k, generator=g) < 0.001
    x[outlier] *= 20.0
    w = torch.randn(n, k, generator=g) * 0.02
    bias = torch.randn(n, generator=g) * 0.01
    return Cfg0(x.to(torch.float16), w.to(torch.float16), bias.to(torch.float16))


@dataclass
class Cfg1:
    x: torch.Tensor       # fp16 [M, H]
    w_qkv: torch.Tensor   # fp16 [3H, H]
    b_qkv: torch.Tensor
    w_up: torch.Tensor    # fp16 [4H, H]
    b_up: torch.Tensor
    w_down: torch.Tensor  # fp16 [H, 4H]
    b_down: torch.Tensor


def cfg1(m=4096, hidden=3072, seed=1) -> Cfg1:
    """Fused DiT-block INT8 GEMM chain (benchmark configuration 1): QKV N=3H, MLP up
    N=4H with GELU-tanh, MLP down K=4H -> N=H; same scheme as config 0."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, hidden, generator=g)
    ws = []
    for n, k in ((3 * hidden, hidden), (4 * hidden, hidden), (hidden, 4 * hidden)):
        w = torch.randn(n, k, generator=g) * 0.02
        b = torch.randn(n, generator=g) * 0.01
        ws += [w.to(torch.float16), b.to(torch.float16)]
    return Cfg1(x.to(torch.float16), *ws)


@dataclass
class Cfg4:
    x: torch.Tensor        # bf16 [T, H]
    logits: torch.Tensor   # fp32 [T, E]
    w_gate: torch.Tensor   # fp32 [E, F, H]
    w_up: torch.Tensor     # fp32 [E, F, H]
    w_down: torch.Tensor   # fp32 [E, H, F]
    top_k: int


def cfg4(tokens=4096, hidden=2048, experts=64, inter=768, top_k=8, seed=4) -> Cfg4:
    """MoE prefill grouped INT8 GEMM (benchmark configuration 4): router logits and
    activations N(0, 1), expert weights N(0, 0.02), drawn in this order."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(tokens, experts, generator=g)
    x = torch.randn(tokens, hidden, generator=g).to(torch.bfloat16)
    w_gate = torch.randn(experts, inter, hidden, generator=g) * 0.02
    w_up = torch.randn(experts, inter, hidden, generator=g) * 0.02
    w_down = torch.randn(experts, hidden, inter, generator=g) * 0.02
    return Cfg4(x, logits, w_gate, w_up, w_down, top_k)
