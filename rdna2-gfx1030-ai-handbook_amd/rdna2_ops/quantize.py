"""Per-row (per-token) dynamic INT8 quantization on gfx950.

``quantize_int8_rowwise`` has the call shape of Kitchen's
``eager.quantize_int8_rowwise`` (third-party comfy_kitchen 0.2.40, called at
rdna2-ops/rdna2_ops/comfy_int8.py:122 and int8_gemm.py:255): it returns
``(codes int8 [M, K], scale fp32 [M, 1])``. The arithmetic is the BASELINE
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
