# SPDX-License-Identifier: Apache-2.0
"""Kitchen-side plumbing shared by the MOSS export and the research adapters.

The reference runs the same fp32 Kitchen pipeline around a replaceable INT8
product in three places: the MOSS production export
(rdna2-ops/rdna2_ops/comfy_int8.py:71-145, duplicated as
production/MOSS_RDNA2_INT8/backend.py), the scoped MOSS research candidate
(rdna2-ops/rdna2_ops/int8_gemm.py:217-271) and, without the Kitchen helpers,
the patientx candidate (int8_gemm.py:274-330). Here the pipeline exists once,
with the product as a parameter, together with the scoped attribute swap the
two research context managers use.

Attribution: the pipeline's step order is the one of comfy_kitchen 0.2.40's
eager ``int8_linear`` (comfy_kitchen/backends/eager/quantization.py,
Copyright (c) 2025 Comfy Org, Apache-2.0) as adapted by the reference. The
order is the interface callers depend on (the same bits must come out); the
Kitchen helpers for each step are called, never re-implemented.
"""
from __future__ import annotations

from contextlib import contextmanager

import torch


def fp32_linear(kitchen, x, weight, weight_scale, *, bias, convrot, convrot_groupsize, input_act,
                input_act_weight, input_act_eps, residual, residual_scale, product):
    """Kitchen's eager INT8 linear with the INT8 product supplied by the caller.

    Steps, in the reference's order (comfy_int8.py:98-145): Kitchen's input
    activation; the inner-dimension check; the weight moved to x's device and
    made contiguous; the weight scale flattened to fp32 and checked (one or N
    elements); Kitchen's ConvRot rotation when asked for; Kitchen's per-row
    quantizer on the rows of x; the product; the leading shape restored;
    Kitchen's residual.

    ``kitchen`` is Kitchen's eager quantization module.
    ``product(x_8, x_scale, weight, scale, bias)`` receives the int8 rows
    [M, K], their fp32 steps [M, 1], the contiguous int8 weight [N, K], the
    fp32 scale vector and the caller's bias, and returns [M, N] with the bias
    applied.
    """
    x = kitchen._apply_input_act(x, input_act, input_act_weight, input_act_eps)
    k = x.shape[-1]
    if k != weight.shape[-1]:
        raise ValueError(f"Input and weight inner dimensions must match, got {k} and {weight.shape[-1]}")
    weight = weight.to(device=x.device).contiguous()
    n = weight.shape[0]
    scale = weight_scale.to(device=x.device, dtype=torch.float32).reshape(-1)
    if scale.numel() not in (1, n):
        raise ValueError(f"INT8 weight scale must be scalar or per-output-channel, got "
                         f"{tuple(weight_scale.shape)} for weight shape {tuple(weight.shape)}")
    if convrot:
        if k % convrot_groupsize:
            raise ValueError(f"ConvRot group size {convrot_groupsize} does not divide input features {k}")
        rotation = kitchen._build_hadamard(convrot_groupsize, device=x.device, dtype=x.dtype)
        x = kitchen._rotate_activation(x, rotation, convrot_groupsize)
    lead = x.shape[:-1]
    x_8, x_scale = kitchen.quantize_int8_rowwise(x.reshape(-1, k))
    y = product(x_8, x_scale, weight, scale, bias)
    return kitchen._apply_residual(y.reshape(*lead, n), residual, residual_scale)


@contextmanager
def swapped(owner, replacements, changed_message):
    """Bind ``owner.<name> = replacement`` for each entry for the duration of
    the block, then put the saved callables back. If any attribute no longer
    holds this block's replacement on exit, someone else patched it meanwhile:
    raise RuntimeError(changed_message) and leave the foreign binding alone
    (the reference's rule, int8_gemm.py:266-271, 324-330)."""
    saved = {name: getattr(owner, name) for name in replacements}
    for name, replacement in replacements.items():
        setattr(owner, name, replacement)
    try:
        yield
    finally:
        if any(getattr(owner, name) is not replacement for name, replacement in replacements.items()):
            raise RuntimeError(changed_message)
        for name, original in saved.items():
            setattr(owner, name, original)


class CallStats:
    """Per-context counters of the research adapters: GEMM hits, precision
    fallbacks and hits per (M, N, K) key — the dictionary the reference's
    candidates yield (int8_gemm.py:233, 262-264)."""

    def __init__(self):
        self.data = {"hits": 0, "fallbacks": 0, "shapes": {}}

    def hit(self, m, n, k):
        self.data["hits"] += 1
        key = str((m, n, k))
        self.data["shapes"][key] = self.data["shapes"].get(key, 0) + 1

    def fallback(self):
        self.data["fallbacks"] += 1
