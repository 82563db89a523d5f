# SPDX-License-Identifier: Apache-2.0
"""MOSS production export of Kitchen's eager ``int8_linear`` on the gfx950 INT8 GEMM.

Interface of rdna2-ops/rdna2_ops/comfy_int8.py (= production/MOSS_RDNA2_INT8/
backend.py): ``int8_linear`` with Kitchen's signature, ``install_backend``,
``disable_backend``, ``kitchen_int8_without_transpose_copy``, ``get_stats``
and ``reset_stats``, the MOSS_RDNA2_INT8_STATS switch, and the same refusals
(RuntimeError) when the install state or Kitchen's export is not what is
expected. Like the reference, the module imports comfy_kitchen at import time
and changes one attribute only: the eager backend module's exported
``int8_linear``.

Attribution: the linear reproduces comfy_kitchen 0.2.40's eager
``int8_linear`` (comfy_kitchen/backends/eager/quantization.py, inspected
sha256 4412eb5bbd12cb2c9a09c5c9e076e744e16bf39632fe624e4df739b84681ef12;
Copyright (c) 2025 Comfy Org, Apache-2.0) as adapted by the reference's
comfy_int8.py: the quantization, scale order, dtype conversion, bias and
residual steps must produce the same bits. The code is this package's own.

Intercepted calls (fp32 activations and fp32 output, the MOSS production
precision) consume the weight as the ``weight.T`` view. When the installed
accumulator is this library's ``int8_matmul``, the INT32 product and
Kitchen's eager epilogue (f32(acc) * (x_scale * w_scale) rounded to the
output dtype, then + bias in the output dtype; comfy_int8.py:128-143) are one
gfx950 launch with that order, bit-identical to the two-step form. Any other
installed accumulator is called as the reference calls it, followed by the
epilogue in torch. Other precisions go to Kitchen's saved export unchanged.
"""
from __future__ import annotations

import os
from contextlib import contextmanager
from threading import Lock

import torch
from comfy_kitchen.backends import eager as eager_backend
from comfy_kitchen.backends.eager import quantization as eager
from comfy_kitchen.registry import registry

from . import _kitchen, int8_gemm

# Kitchen bounds its fp32 intermediate to 256 MiB per chunk of rows.
_CHUNK_BYTES = 256 * 1024 * 1024


class _LayoutStats:
    """GEMM counters behind MOSS_RDNA2_INT8_STATS=1: a call count and calls per
    (weight shape, weight stride, rhs stride, device). No tensor is kept and
    nothing is logged per call (comfy_int8.py:30-68)."""

    def __init__(self, enabled):
        self.enabled = enabled
        self.lock = Lock()
        self.calls = 0
        self.layouts = {}

    def record(self, weight, rhs):
        key = (tuple(weight.shape), tuple(weight.stride()), tuple(rhs.stride()), str(weight.device))
        with self.lock:
            self.calls += 1
            self.layouts[key] = self.layouts.get(key, 0) + 1

    def snapshot(self):
        with self.lock:
            rows = [{"shape": k[0], "weight_stride": k[1], "rhs_stride": k[2], "device": k[3],
                     "dtype": "torch.int8", "calls": c} for k, c in self.layouts.items()]
            return {"enabled": self.enabled, "calls": self.calls, "weight_layouts": rows}

    def clear(self):
        with self.lock:
            self.calls = 0
            self.layouts.clear()


class _ExportState:
    """What install_backend changed: the accumulator bound to this export and
    Kitchen's saved export (None while not installed)."""

    def __init__(self):
        self.lock = Lock()
        self.gemm = None
        self.saved = None


_stats = _LayoutStats(os.environ.get("MOSS_RDNA2_INT8_STATS", "0") == "1")
_state = _ExportState()
_scope_lock = Lock()


def get_stats():
    """Successful GEMM counts and weight layouts (MOSS_RDNA2_INT8_STATS=1)."""
    return _stats.snapshot()


def reset_stats():
    _stats.clear()


def _scaled_in_chunks(acc, x_scale, scale, out_dtype):
    """Kitchen's epilogue on an INT32 product: per chunk of rows,
    f32(acc) * (x_scale * w_scale), rounded to out_dtype (comfy_int8.py:128-140)."""
    m, n = acc.shape
    rows = max(1, min(m, _CHUNK_BYTES // (n * 4)))
    w_row = scale.reshape(1, -1)
    pieces = []
    for lo in range(0, m, rows):
        part = acc[lo:lo + rows].float()
        step = x_scale[lo:lo + rows].to(device=part.device, dtype=torch.float32) * w_row
        pieces.append((part * step).to(out_dtype))
    return torch.cat(pieces, dim=0)


def _product(gemm, out_dtype):
    """The INT8 product step of the intercepted linear for accumulator ``gemm``."""

    def run(x_8, x_scale, weight, scale, bias):
        rhs = weight.T
        if gemm is int8_gemm.int8_matmul and x_8.is_cuda:
            b32 = None if bias is None else bias.to(device=x_8.device, dtype=torch.float32).reshape(-1).contiguous()
            y = int8_gemm.int8_gemm_dequant(
                x_8, rhs, x_scale.to(torch.float32).reshape(-1).contiguous(), scale.contiguous(), b32,
                out_dtype=out_dtype, epilogue_order="eager")
        else:
            y = _scaled_in_chunks(gemm(x_8, rhs), x_scale, scale, out_dtype)
            if bias is not None:
                y = y + bias.to(device=y.device, dtype=y.dtype).reshape(1, -1)
        if _stats.enabled:
            _stats.record(weight, rhs)
        return y

    return run


def int8_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    convrot: bool = False,
    convrot_groupsize: int = 256,
    input_act: str | None = None,
    input_act_weight: torch.Tensor | None = None,
    input_act_eps: float = 0.0,
    residual: torch.Tensor | None = None,
    residual_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """Kitchen's eager INT8 linear with a weight.T GEMM (comfy_int8.py:71-145)."""
    gemm = _state.gemm
    if gemm is None:
        raise RuntimeError("Install the MOSS INT8 eager export before calling it")
    options = dict(bias=bias, convrot=convrot, convrot_groupsize=convrot_groupsize, input_act=input_act,
                   input_act_weight=input_act_weight, input_act_eps=input_act_eps, residual=residual,
                   residual_scale=residual_scale)
    if x.dtype != torch.float32 or out_dtype != torch.float32:
        return eager.int8_linear(x, weight, weight_scale, out_dtype=out_dtype, **options)
    return _kitchen.fp32_linear(eager, x, weight, weight_scale, product=_product(gemm, out_dtype), **options)


def _resolves_to(fn):
    return registry.get_implementation("int8_linear", backend="eager") is fn


def install_backend(strided_int8_matmul):
    """Bind ``strided_int8_matmul`` (already installed as Kitchen's
    ``_int8_matmul_accumulate``) and replace the eager backend's exported
    int8_linear with this module's (comfy_int8.py:148-186). Repeating the call
    with the same GEMM is a no-op; a different GEMM, an export changed by
    someone else, a missing accumulator hook or a registry that does not
    resolve the export raise RuntimeError, leaving Kitchen as it was. Call it
    before Comfy's worker starts or between completed workloads."""
    if not callable(strided_int8_matmul):
        raise TypeError("strided_int8_matmul must be callable")
    with _state.lock:
        if _state.saved is not None:
            if _state.gemm is not strided_int8_matmul:
                raise RuntimeError("MOSS INT8 export is already bound to a different GEMM")
            if eager_backend.int8_linear is not int8_linear:
                raise RuntimeError("Kitchen eager int8_linear changed while this patch was installed")
            return
        if eager._int8_matmul_accumulate is not strided_int8_matmul:
            raise RuntimeError("Install the MI355X INT8 GEMM as Kitchen's accumulator first")
        kitchen_export = eager.int8_linear
        if eager_backend.int8_linear is not kitchen_export:
            raise RuntimeError("Expected Kitchen's unmodified eager int8_linear export")
        if not _resolves_to(kitchen_export):
            raise RuntimeError("Kitchen eager dispatch does not resolve the expected export")
        _state.gemm = strided_int8_matmul
        eager_backend.int8_linear = int8_linear
        try:
            if not _resolves_to(int8_linear):
                raise RuntimeError("Kitchen eager dispatch did not pick up its replacement export")
        except Exception:
            eager_backend.int8_linear = kitchen_export
            _state.gemm = None
            raise
        _state.saved = kitchen_export


def disable_backend():
    """Put Kitchen's saved export back (comfy_int8.py:189-203); the GEMM stays
    installed as Kitchen's accumulator. A no-op when not installed; refuses
    (RuntimeError) to overwrite an export someone else replaced. For a rollback
    that survives restarts use MOSS_RDNA2_INT8_LAYOUT=legacy."""
    with _state.lock:
        if _state.saved is None:
            return
        if eager_backend.int8_linear is not int8_linear:
            raise RuntimeError("Kitchen eager int8_linear changed; refusing to overwrite it")
        eager_backend.int8_linear = _state.saved
        _state.saved = None


@contextmanager
def kitchen_int8_without_transpose_copy(strided_int8_matmul):
    """install_backend for the duration of a block in an exclusively owned
    workload, then disable_backend (comfy_int8.py:206-227). Nested or
    concurrent blocks raise RuntimeError."""
    if not _scope_lock.acquire(blocking=False):
        raise RuntimeError("Nested or concurrent Kitchen INT8 contexts are unsupported")
    try:
        install_backend(strided_int8_matmul)
        try:
            yield
        finally:
            disable_backend()
    finally:
        _scope_lock.release()
