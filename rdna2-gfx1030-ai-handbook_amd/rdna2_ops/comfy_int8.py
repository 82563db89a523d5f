# SPDX-License-Identifier: Apache-2.0
"""Kitchen eager INT8 linear without a weight-transpose copy (MI355X).

Drop-in for rdna2-ops/rdna2_ops/comfy_int8.py (= production/MOSS_RDNA2_INT8/
backend.py): the same exported ``int8_linear`` signature and semantics, the
same ``install_backend`` / ``disable_backend`` / ``get_stats`` /
``reset_stats`` / ``kitchen_int8_without_transpose_copy`` life-cycle and
safety checks, and the MOSS_RDNA2_INT8_STATS counters. Like the reference it
imports comfy_kitchen (0.2.40) at module import and changes only the eager
backend module's exported callable — no registry identity, priority,
bytecode, package file or weight storage.

What changes on MI355X: for the intercepted case (fp32 activations and fp32
output, the measured MOSS production path) the weight is consumed as the
``weight.T`` view (no transpose copy) and, when the installed GEMM is this
library's ``int8_matmul``, the INT32 product and Kitchen's chunked eager
epilogue (comfy_int8.py:128-143) run as one fused gfx950 kernel with the
same operation order (``epilogue_order="eager"``): round(f32(acc) * (sa*sw))
to out_dtype, then + bias in out_dtype. With out_dtype = fp32 both steps are
the plain fp32 operations of the reference, so the result is identical bit
for bit. Any other installed GEMM is called exactly like the reference does.
Kitchen's quantizer, ConvRot, input activation and residual helpers are used
unchanged.
"""
from __future__ import annotations

import os
from contextlib import contextmanager
from threading import Lock

import torch
from comfy_kitchen.backends import eager as eager_backend
from comfy_kitchen.backends.eager import quantization as eager
from comfy_kitchen.registry import registry

from . import int8_gemm

_matmul = None
_original_export = None
_installed = False
_installation_lock = Lock()
_stats_enabled = os.environ.get("MOSS_RDNA2_INT8_STATS", "0") == "1"
_stats_lock = Lock()
_calls = 0
_layouts = {}


def _record_layout(weight, rhs):
    global _calls
    key = (tuple(weight.shape), tuple(weight.stride()), tuple(rhs.stride()), str(weight.device))
    with _stats_lock:
        _calls += 1
        _layouts[key] = _layouts.get(key, 0) + 1


def get_stats():
    """Successful GEMM counts / layouts when MOSS_RDNA2_INT8_STATS=1 (no tensors kept,
    no per-call logging) — comfy_int8.py:47-62."""
    with _stats_lock:
        return {
            "enabled": _stats_enabled,
            "calls": _calls,
            "weight_layouts": [
                {"shape": shape, "weight_stride": stride, "rhs_stride": rhs_stride,
                 "device": device, "dtype": "torch.int8", "calls": count}
                for (shape, stride, rhs_stride, device), count in _layouts.items()
            ],
        }


def reset_stats():
    global _calls
    with _stats_lock:
        _calls = 0
        _layouts.clear()


def _eager_epilogue(result, x_scale, weight_scale, out_dtype):
    """Kitchen's chunked fp32 scaling, then the cast (comfy_int8.py:128-140)."""
    m, n = result.shape
    chunk_size = max(1, min(m, 256 * 1024 * 1024 // (n * 4)))
    weight_scale = weight_scale.reshape(1, -1)
    parts = []
    for i in range(0, m, chunk_size):
        end = min(i + chunk_size, m)
        chunk = result[i:end].float()
        scales = x_scale[i:end].to(device=chunk.device, dtype=torch.float32) * weight_scale
        parts.append((chunk * scales).to(out_dtype))
    return torch.cat(parts, dim=0)


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
    """Pinned eager INT8 linear semantics with a stride-aware weight.T GEMM
    (comfy_int8.py:71-145)."""
    if _matmul is None:
        raise RuntimeError("Install the MOSS INT8 eager export before calling it")
    # Only the measured production precision (fp32 in / out) is intercepted.
    if x.dtype != torch.float32 or out_dtype != torch.float32:
        return eager.int8_linear(
            x, weight, weight_scale, bias=bias, out_dtype=out_dtype,
            convrot=convrot, convrot_groupsize=convrot_groupsize,
            input_act=input_act, input_act_weight=input_act_weight,
            input_act_eps=input_act_eps, residual=residual,
            residual_scale=residual_scale,
        )
    x = eager._apply_input_act(x, input_act, input_act_weight, input_act_eps)
    if x.shape[-1] != weight.shape[-1]:
        raise ValueError(
            f"Input and weight inner dimensions must match, got {x.shape[-1]} and {weight.shape[-1]}"
        )
    weight = weight.to(device=x.device).contiguous()
    weight_scale = weight_scale.to(device=x.device, dtype=torch.float32).reshape(-1)
    if weight_scale.numel() not in (1, weight.shape[0]):
        raise ValueError(
            f"INT8 weight scale must be scalar or per-output-channel, got {tuple(weight_scale.shape)} "
            f"for weight shape {tuple(weight.shape)}"
        )
    if convrot:
        if x.shape[-1] % convrot_groupsize != 0:
            raise ValueError(
                f"ConvRot group size {convrot_groupsize} does not divide input features {x.shape[-1]}"
            )
        h = eager._build_hadamard(convrot_groupsize, device=x.device, dtype=x.dtype)
        x = eager._rotate_activation(x, h, convrot_groupsize)

    orig_shape = x.shape
    x_2d = x.reshape(-1, x.shape[-1])
    x_8, x_scale = eager.quantize_int8_rowwise(x_2d)
    rhs = weight.T
    if _matmul is int8_gemm.int8_matmul and x_8.is_cuda:
        # one fused launch: INT32 product + Kitchen's eager epilogue order
        b32 = None if bias is None else bias.to(device=x.device, dtype=torch.float32).reshape(-1).contiguous()
        result = int8_gemm.int8_gemm_dequant(
            x_8, rhs, x_scale.to(torch.float32).reshape(-1).contiguous(), weight_scale.contiguous(), b32,
            out_dtype=out_dtype, epilogue_order="eager")
    else:
        result = _eager_epilogue(_matmul(x_8, rhs), x_scale, weight_scale, out_dtype)
        if bias is not None:
            result = result + bias.to(device=result.device, dtype=result.dtype).reshape(1, -1)
    if _stats_enabled:
        _record_layout(weight, rhs)
    result = result.reshape(*orig_shape[:-1], weight.shape[0])
    return eager._apply_residual(result, residual, residual_scale)


def install_backend(strided_int8_matmul):
    """Replace only the eager backend module's exported int8_linear callable
    (comfy_int8.py:148-186). The caller installs ``strided_int8_matmul`` as
    Kitchen's ``_int8_matmul_accumulate`` first. Call before starting Comfy's
    worker or between completed workloads."""
    global _matmul, _original_export, _installed
    if not callable(strided_int8_matmul):
        raise TypeError("strided_int8_matmul must be callable")
    with _installation_lock:
        if _installed:
            if _matmul is not strided_int8_matmul:
                raise RuntimeError("MOSS INT8 export is already bound to a different GEMM")
            if eager_backend.int8_linear is not int8_linear:
                raise RuntimeError("Kitchen eager int8_linear changed while this patch was installed")
            return
        if eager._int8_matmul_accumulate is not strided_int8_matmul:
            raise RuntimeError("Install the MI355X INT8 GEMM as Kitchen's accumulator first")
        original = eager.int8_linear
        if eager_backend.int8_linear is not original:
            raise RuntimeError("Expected Kitchen's unmodified eager int8_linear export")
        if registry.get_implementation("int8_linear", backend="eager") is not original:
            raise RuntimeError("Kitchen eager dispatch does not resolve the expected export")
        _original_export = original
        _matmul = strided_int8_matmul
        try:
            eager_backend.int8_linear = int8_linear
            if registry.get_implementation("int8_linear", backend="eager") is not int8_linear:
                raise RuntimeError("Kitchen eager dispatch did not pick up its replacement export")
        except Exception:
            eager_backend.int8_linear = original
            _original_export = None
            _matmul = None
            raise
        _installed = True


def disable_backend():
    """Restore the original eager export (comfy_int8.py:189-203). Refuses to
    overwrite another patch's export. For a persistent rollback restart with
    MOSS_RDNA2_INT8_LAYOUT=legacy."""
    global _installed
    with _installation_lock:
        if not _installed:
            return
        if eager_backend.int8_linear is not int8_linear:
            raise RuntimeError("Kitchen eager int8_linear changed; refusing to overwrite it")
        eager_backend.int8_linear = _original_export
        _installed = False


_context_lock = Lock()


@contextmanager
def kitchen_int8_without_transpose_copy(strided_int8_matmul):
    """Scoped export replacement for an exclusively owned workload
    (comfy_int8.py:206-227); nested or concurrent contexts are refused."""
    if not _context_lock.acquire(blocking=False):
        raise RuntimeError("Nested or concurrent Kitchen INT8 contexts are unsupported")
    try:
        install_backend(strided_int8_matmul)
        try:
            yield
        finally:
            disable_backend()
    finally:
        _context_lock.release()
