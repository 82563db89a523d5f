"""Per-row (per-token) dynamic INT8 quantization on gfx950.

``quantize_int8_rowwise`` has the call shape of Kitchen's
``eager.quantize_int8_rowwise`` (third-party comfy_kitchen 0.2.40, called at
rdna2-ops/rdna2_ops/comfy_int8.py:122 and int8_gemm.py:255): it returns
``(codes int8 [M, K], scale fp32 [M, 1])``. The arithmetic is the benchmark's
per-token rule, step = max(absmax / 127, 1e-20) and q = round_half_even(x / step)
with IEEE division, clamped to [-127, 127]; ``rounding="half_away"`` selects the
reference's in-tree Triton quantizer instead
(rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:76-92, floor(z + .5) / ceil(z - .5)).
"""
from __future__ import annotations

import torch

from . import _lib

_X_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2)


def quantize_int8_rowwise(x, *, rounding="half_even"):
    """Return (int8 codes [M, K], fp32 steps [M, 1]) for a 2-D [M, K] tensor."""
    if x.ndim != 2:
        raise ValueError("Expected a 2-D [M, K] tensor")
    if x.dtype not in _X_DTYPES:
        raise TypeError("x must be fp32/fp16/bf16/fp8")
    if rounding not in ("half_even", "half_away"):
        raise ValueError("rounding must be half_even or half_away")
    _lib.require_gfx950(x)
    if min(x.stride()) < 0:
        raise ValueError("Negative strides are unsupported")
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    step = torch.empty((m, 1), dtype=torch.float32, device=x.device)
    if m:
        xv = x.view(torch.uint8) if x.dtype in (torch.float8_e4m3fn, torch.float8_e5m2) else x
        status = _lib.library().qg_quant_rows_i8(
            _lib.ptr(xv), _lib.DTYPE_CODE[x.dtype], x.stride(0), x.stride(1), m, k, _lib.ptr(q), k,
            _lib.ptr(step), _lib.ROUND_HALF_EVEN if rounding == "half_even" else _lib.ROUND_HALF_AWAY,
            _lib.stream_of(x))
        _lib.check(status, "qg_quant_rows_i8")
    return q, step


def rotate_quantize_int8_rowwise(x, group_size=256, *, rounding="half_even"):
    """ConvRot then the per-row quantizer in one launch (qg_rot_quant_rows_i8).

    Every group of ``group_size`` (a power of two in [2, 1024] dividing K,
    K <= 16384) consecutive values of each row of the 2-D [M, K] fp32/fp16/bf16
    tensor ``x`` is multiplied by H / sqrt(group_size), H the Sylvester
    Hadamard matrix (Kitchen's _build_hadamard + _rotate_activation at
    rdna2-ops/rdna2_ops/comfy_int8.py:117-118), then the rows are quantized as
    by quantize_int8_rowwise. The rotation runs as fast Walsh-Hadamard
    butterflies in fp32: the same sums as Kitchen's dense product in another
    order, equal to a few fp32 ulps. Returns (int8 codes [M, K], fp32 steps [M, 1]).
    """
    if x.ndim != 2:
        raise ValueError("Expected a 2-D [M, K] tensor")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError("x must be fp32/fp16/bf16")
    if rounding not in ("half_even", "half_away"):
        raise ValueError("rounding must be half_even or half_away")
    m, k = x.shape
    g = int(group_size)
    if g < 2 or g > 1024 or g & (g - 1) or k % g or k > 16384:
        raise ValueError(f"group_size {group_size} must be a power of two in [2, 1024] dividing K={k} "
                         f"(K <= 16384)")
    _lib.require_gfx950(x)
    if k and x.stride(1) != 1:
        x = x.contiguous()
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    step = torch.empty((m, 1), dtype=torch.float32, device=x.device)
    if m:
        status = _lib.library().qg_rot_quant_rows_i8(
            _lib.ptr(x), _lib.DTYPE_CODE[x.dtype], x.stride(0), m, k, g, _lib.ptr(q), k, _lib.ptr(step),
            _lib.ROUND_HALF_EVEN if rounding == "half_even" else _lib.ROUND_HALF_AWAY, _lib.stream_of(x))
        _lib.check(status, "qg_rot_quant_rows_i8")
    return q, step
