# SPDX-License-Identifier: Apache-2.0
"""gfx950 INT8 GEMM with an optional FP32 dequantization epilogue (MI355X).

Drop-in for rdna2-ops/rdna2_ops/int8_gemm.py: the same entry points, argument
meaning, validation order and exceptions, served by hand-written gfx950 HIP
kernels in librdna2_qgemm.so (int8 MFMA, LDS-DMA pipeline) instead of Triton.

The two scale products retain their order: float(acc) * (row_scale * col_scale).
rounding="separate" keeps multiply and add separate (MOSS eager semantics,
int8_gemm.py:53-63 with enable_fp_fusion=False); rounding="fused" uses one FMA
for multiply+bias (int8_gemm.py:191, the patientx behaviour).

Triton launch knobs (tile, num_warps, num_stages, group_m, wrapped,
partial_dot) are accepted and validated exactly as the reference does
(int8_gemm.py:144-147, :155-156) so callers keep working; on MI355X they are
hints only — the library picks its own MFMA tile — and results never depend
on them: integer accumulation is exact and the epilogue is per element.
``wrapped`` asks for the reference's variant that loads the unused rows and
columns of edge tiles from valid indices and masks only the stores
(int8_gemm.py:70-123); every kernel of this library already loads edge rows
from clamped, valid indices, so both settings run the same kernel.
``partial_dot`` (the wrapped variant's acc += dot form, :103-106) adds exact
int32 partial products, the same sums. The returned kernel metadata records
both requests.

New keyword arguments (defaults keep the reference's behaviour):
``out_dtype`` (fp32 default; fp16/bf16 round the fp32 epilogue once, RNE),
``activation`` (None or "gelu_tanh", applied in fp32 before rounding) and
``epilogue_order`` ("reference" = order above, "eager" = Kitchen's eager
order, comfy_int8.py:128-143: round(acc*scale) then + round(bias) in out dtype).
"""
from contextlib import contextmanager
import sys

import torch

from . import _kitchen, _lib

_MAX_K = 131071
_ROT_MAX_K = 16384  # QG_ROT_MAX_K: the ConvRot prologue holds one fp32 row in LDS


def _validate(a, b, tile, num_warps, num_stages, group_m):
    """Contract of rdna2-ops/rdna2_ops/int8_gemm.py:131-149 (arch: gfx950)."""
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("Expected [M,K] @ [K,N]")
    if a.dtype != torch.int8 or b.dtype != torch.int8:
        raise TypeError("Both GEMM operands must be INT8")
    if a.device.type != "cuda" or b.device != a.device:
        raise ValueError("Inputs must share a HIP device")
    _lib.require_gfx950(a)
    if any(s < 0 for s in a.stride() + b.stride()):
        raise ValueError("Negative strides are unsupported")
    if a.shape[1] > _MAX_K:
        raise ValueError("K could overflow signed INT32 for arbitrary signed INT8 inputs")
    if len(tile) != 3 or any(v < 16 or v > 256 or v & (v - 1) for v in tile):
        raise ValueError("Tile dimensions must be powers of two in [16,256]")
    if num_warps not in (4, 8) or num_stages not in (1, 2, 3) or group_m not in (1, 2, 4, 8):
        raise ValueError("Unsupported launch configuration")
    if torch.compiler.is_compiling() or torch.cuda.is_current_stream_capturing():
        raise RuntimeError("Only explicit eager calls are supported")


_OUT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_ACTIVATIONS = {None: 0, "gelu_tanh": _lib.EPI_GELU_TANH}


def _epilogue_flags(rounding, activation, epilogue_order):
    if activation not in _ACTIVATIONS:
        raise ValueError("activation must be None or 'gelu_tanh'")
    if epilogue_order not in ("reference", "eager"):
        raise ValueError("epilogue_order must be 'reference' or 'eager'")
    flags = _ACTIVATIONS[activation]
    if epilogue_order == "eager":
        if activation is not None or rounding == "fused":
            raise ValueError("The eager epilogue order has no activation and no FMA rounding")
        flags |= _lib.EPI_ORDER_EAGER
    elif rounding == "fused":
        flags |= _lib.EPI_ORDER_FUSED_FMA
    return flags


def _launch(a, b, a_scale, b_scale, bias, *, tile, num_warps, num_stages, group_m, rounding,
            return_kernel, wrapped=False, partial_dot=False, out_dtype=torch.float32,
            activation=None, epilogue_order="reference"):
    """Host dispatch of rdna2-ops/rdna2_ops/int8_gemm.py:152-192 onto the C ABI."""
    _validate(a, b, tile, num_warps, num_stages, group_m)
    if partial_dot and not wrapped:
        raise ValueError("partial_dot requires the explicitly wrapped-load variant")
    dequant = a_scale is not None
    m, k = a.shape
    n = b.shape[1]
    if rounding not in ("separate", "fused"):
        raise ValueError("rounding must be separate or fused")
    if dequant:
        for value, size, label in ((a_scale, m, "a_scale"), (b_scale, n, "b_scale")):
            if not isinstance(value, torch.Tensor):
                raise TypeError(label + " must be a device tensor")
            if value.device != a.device or value.dtype != torch.float32 or not value.is_contiguous():
                raise ValueError(label + " must be contiguous FP32 on the input device")
            if value.numel() != size and not (label == "b_scale" and value.numel() == 1):
                raise ValueError(label + " has the wrong number of elements")
            if torch.is_grad_enabled() and value.requires_grad:
                raise ValueError("Autograd is unsupported")
        if bias is not None:
            if (bias.device != a.device or bias.numel() != n or not bias.is_contiguous()
                    or bias.dtype not in (torch.float32, torch.float16, torch.bfloat16)):
                raise ValueError("Bias must be a contiguous floating point vector of length N")
            if torch.is_grad_enabled() and bias.requires_grad:
                raise ValueError("Autograd is unsupported")
        if out_dtype not in _OUT_DTYPES:
            raise ValueError("out_dtype must be float32, float16 or bfloat16")
        flags = _epilogue_flags(rounding, activation, epilogue_order)
    else:
        if out_dtype not in (torch.float32, torch.int32) or activation is not None:
            raise ValueError("The integer GEMM has no dtype conversion or activation")
        flags = 0
    odt = out_dtype if dequant else torch.int32
    out = torch.empty((m, n), device=a.device, dtype=odt)
    if m == 0 or n == 0:
        return (out, None) if return_kernel else out
    lib = _lib.library()
    ws_bytes = lib.qg_int8_gemm_workspace_bytes(
        _lib.ptr(a), a.stride(0), a.stride(1), _lib.ptr(b), b.stride(0), b.stride(1), m, n, k)
    ws = _lib.workspace(ws_bytes, a.device)
    wsp, wsn = _lib.ws_ptr(ws)
    status = lib.qg_int8_gemm(
        _lib.ptr(a), a.stride(0), a.stride(1), _lib.ptr(b), b.stride(0), b.stride(1), m, n, k,
        _lib.ptr(a_scale) if dequant else None, _lib.ptr(b_scale) if dequant else None,
        b_scale.numel() if dequant else 0,
        _lib.ptr(bias) if dequant else None,
        _lib.DTYPE_CODE[bias.dtype] if (dequant and bias is not None) else 0,
        _lib.ptr(out), _lib.DTYPE_CODE[odt], flags, wsp, wsn, _lib.stream_of(a))
    _lib.check(status, "qg_int8_gemm")
    if not return_kernel:
        return out
    # the C ABI's choice: >= 192 tiles of 256 x 192 take the persistent 8-wave
    # ping-pong kernel, smaller grids the 4-wave 128 x 128 one (K stage 128)
    big = (-(-m // 256)) * (-(-n // 192)) >= 192
    tile_used = (256, 192, 128) if big else (128, 128, 128)
    meta = _lib.kernel_metadata("int8_mfma_32x32x32_pingpong" if big else "int8_mfma_32x32x32", tile_used,
                                "k_i8_gemm_ppINS0_5I8GeoILi256ELi192E" if big else "k_i8_gemmINS0_5I8GeoILi128ELi128E")
    meta.update(packed_operands=ws_bytes > 0, requested_tile=list(tile), epilogue_flags=flags,
                requested_wrapped=bool(wrapped), requested_partial_dot=bool(partial_dot))
    return out, meta


def int8_matmul(a, b, *, tile=(32, 64, 64), num_warps=4, num_stages=1,
                group_m=4, return_kernel=False, wrapped=False, partial_dot=False):
    """Exact INT8 -> INT32 matmul; accepts both [K,N] layouts without copying.

    Mirrors rdna2-ops/rdna2_ops/int8_gemm.py:195-200. ``b`` may be ``weight.T``
    (strides (1, K), read in place) or any other positive-stride [K, N] view
    (packed once into workspace by the library).
    """
    return _launch(a, b, None, None, None, tile=tile, num_warps=num_warps,
                   num_stages=num_stages, group_m=group_m, rounding="separate",
                   return_kernel=return_kernel, wrapped=wrapped, partial_dot=partial_dot)


def int8_gemm_dequant(a, b, a_scale, b_scale, bias=None, *, tile=(32, 64, 64),
                      num_warps=4, num_stages=1, group_m=4,
                      rounding="separate", return_kernel=False, wrapped=False, partial_dot=False,
                      out_dtype=torch.float32, activation=None, epilogue_order="reference"):
    """INT32 GEMM and row/scalar or row/column FP32 dequantization in one kernel.

    Mirrors rdna2-ops/rdna2_ops/int8_gemm.py:203-214. Inputs are already
    quantized. A fresh contiguous output is allocated. Finite scales/bias are a
    precondition; no GPU-wide finite scan is inserted.
    """
    return _launch(a, b, a_scale, b_scale, bias, tile=tile, num_warps=num_warps,
                   num_stages=num_stages, group_m=group_m, rounding=rounding,
                   return_kernel=return_kernel, wrapped=wrapped, partial_dot=partial_dot,
                   out_dtype=out_dtype, activation=activation, epilogue_order=epilogue_order)


def w8a8_linear(x, weight, weight_scale, bias=None, *, out_dtype=None, activation=None,
                rounding="half_even", epilogue_order="reference", convrot_groupsize=None, residual=None,
                residual_scale=None):
    """Fused W8A8 linear: per-token INT8 quantization of ``x`` (absmax/127),
    INT8 MFMA GEMM against ``weight`` [N, K] and the dequant/bias/activation
    epilogue, in one library call (qg_w8a8_linear).

    x: [..., K] fp32/fp16/bf16 with unit K stride. weight: int8 [N, K].
    weight_scale: fp32 [N] (or [N, 1]) or a one-element tensor.
    rounding: "half_even" (per-token rule of the benchmark) or "half_away" (the
    reference's in-tree _quant_rows, fp8_weight_gemm_v06.py:87-90).
    out_dtype defaults to x.dtype.

    Opt-in MOSS steps (qg_w8a8_linear_ex; the MOSS linear applies them around
    its GEMM at comfy_int8.py:112-122 and :145):
    convrot_groupsize: a power of two g in [2, 1024] dividing K (MOSS: 256):
    every group of g values of a row is rotated by H_g / sqrt(g) before the
    quantizer, with fast Walsh-Hadamard butterflies (the weight must have been
    rotated the same way when it was quantized). Kitchen's dense fp32 rotation
    forms the same sums in another order: the rotated values agree to a few
    fp32 ulps, so a code can differ by one where a quotient sits within a few
    ulps of a rounding tie.
    residual: [..., N] fp32/fp16/bf16 (x's leading shape) added in fp32 after
    the scale, bias and activation steps, times residual_scale (fp32, 1 or N
    values) when given, before the one rounding to out_dtype: fp32 outputs
    are Kitchen's fp32 sequence scale -> + bias -> + residual bit for bit.
    Not with epilogue_order="eager".
    """
    if x.dtype not in _OUT_DTYPES or weight.dtype != torch.int8 or weight.ndim != 2:
        raise TypeError("x must be fp32/fp16/bf16 and weight int8 [N, K]")
    if x.shape[-1] != weight.shape[1]:
        raise ValueError("Input and weight inner dimensions differ")
    if x.device.type != "cuda" or weight.device != x.device:
        raise ValueError("Inputs must share a HIP device")
    _lib.require_gfx950(x)
    if rounding not in ("half_even", "half_away"):
        raise ValueError("rounding must be half_even or half_away")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in _OUT_DTYPES:
        raise ValueError("out_dtype must be float32, float16 or bfloat16")
    k = x.shape[-1]
    if k > _MAX_K:
        raise ValueError("K could overflow signed INT32 for arbitrary signed INT8 inputs")
    n = weight.shape[0]
    ws_scale = weight_scale.reshape(-1)
    if (ws_scale.dtype != torch.float32 or ws_scale.device != x.device or not ws_scale.is_contiguous()
            or ws_scale.numel() not in (1, n)):
        raise ValueError("weight_scale must be contiguous FP32 with 1 or N elements")
    if bias is not None and (bias.device != x.device or bias.numel() != n or not bias.is_contiguous()
                             or bias.dtype not in _OUT_DTYPES):
        raise ValueError("Bias must be a contiguous floating point vector of length N")
    if convrot_groupsize is not None:
        g = int(convrot_groupsize)
        if g < 2 or g > 1024 or g & (g - 1) or k % g or k > _ROT_MAX_K:
            raise ValueError(f"ConvRot group size {convrot_groupsize} must be a power of two in [2, 1024] "
                             f"dividing input features {k} (K <= {_ROT_MAX_K})")
    if residual is not None:
        if epilogue_order == "eager":
            raise ValueError("The residual term is not available with epilogue_order='eager'")
        if (residual.dtype not in _OUT_DTYPES or residual.device != x.device
                or tuple(residual.shape) != (*x.shape[:-1], n)):
            raise ValueError("residual must be a floating point tensor of shape [..., N] on x's device")
    elif residual_scale is not None:
        raise ValueError("residual_scale needs a residual")
    rs = None
    if residual_scale is not None:
        rs = residual_scale.reshape(-1)
        if (rs.dtype != torch.float32 or rs.device != x.device or not rs.is_contiguous()
                or rs.numel() not in (1, n)):
            raise ValueError("residual_scale must be contiguous FP32 with 1 or N elements")
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    x2 = x.reshape(-1, k)
    if k and x2.stride(1) != 1:
        x2 = x2.contiguous()
    m = x2.shape[0]
    r2 = None
    if residual is not None:
        r2 = residual.reshape(m, n)
        if n and r2.stride(1) != 1:
            r2 = r2.contiguous()
    flags = _epilogue_flags("separate", activation, epilogue_order)
    out = torch.empty((m, n), device=x.device, dtype=out_dtype)
    if m and n:
        lib = _lib.library()
        need = lib.qg_w8a8_linear_workspace_bytes(_lib.ptr(weight), weight.stride(0), m, n, k)
        ws = _lib.workspace(need, x.device)
        wsp, wsn = _lib.ws_ptr(ws)
        rnd = _lib.ROUND_HALF_EVEN if rounding == "half_even" else _lib.ROUND_HALF_AWAY
        bias_code = _lib.DTYPE_CODE[bias.dtype] if bias is not None else 0
        if convrot_groupsize is None and residual is None:
            status = lib.qg_w8a8_linear(
                _lib.ptr(x2), _lib.DTYPE_CODE[x2.dtype], x2.stride(0), m, k, _lib.ptr(weight),
                weight.stride(0), n, _lib.ptr(ws_scale), ws_scale.numel(), _lib.ptr(bias), bias_code,
                _lib.ptr(out), _lib.DTYPE_CODE[out_dtype], rnd, flags, wsp, wsn, _lib.stream_of(x))
            _lib.check(status, "qg_w8a8_linear")
        else:
            status = lib.qg_w8a8_linear_ex(
                _lib.ptr(x2), _lib.DTYPE_CODE[x2.dtype], x2.stride(0), m, k, _lib.ptr(weight),
                weight.stride(0), n, _lib.ptr(ws_scale), ws_scale.numel(), _lib.ptr(bias), bias_code,
                int(convrot_groupsize or 0), _lib.ptr(r2), _lib.DTYPE_CODE[r2.dtype] if r2 is not None else 0,
                r2.stride(0) if r2 is not None else 0, _lib.ptr(rs), rs.numel() if rs is not None else 0,
                _lib.ptr(out), _lib.DTYPE_CODE[out_dtype], rnd, flags, wsp, wsn, _lib.stream_of(x))
            _lib.check(status, "qg_w8a8_linear_ex")
    return out.reshape(*x.shape[:-1], n)


def _research_knobs(tile, num_warps, num_stages, group_m, wrapped, partial_dot):
    return dict(tile=tile, num_warps=num_warps, num_stages=num_stages, group_m=group_m, wrapped=wrapped,
                partial_dot=partial_dot)


@contextmanager
def moss_int8_gemm_candidate(*, tile=(32, 64, 64), num_warps=4,
                             num_stages=1, group_m=4, wrapped=False, partial_dot=False):
    """Scoped MOSS research export: Kitchen's eager backend exports a linear whose
    INT8 product and fp32 epilogue are one ``int8_gemm_dequant`` launch in the
    reference order (rounding="separate": f32(acc) * (sa * sw), then + bias).

    Interface of rdna2-ops/rdna2_ops/int8_gemm.py:217-271. fp32 activations
    with fp32 output are served; every other call goes to the saved Kitchen
    export and counts as a fallback. Kitchen's input activation, ConvRot,
    quantizer and residual run unchanged around the product. Yields the
    per-context counters {"hits", "fallbacks", "shapes"}. On exit the saved
    export is restored, unless someone else replaced the candidate meanwhile
    (RuntimeError). For an exclusively owned process: no registry entry, code
    object, file or weight is changed.
    """
    from comfy_kitchen.backends import eager as backend
    from comfy_kitchen.backends.eager import quantization as kitchen
    saved = backend.int8_linear
    stats = _kitchen.CallStats()
    knobs = _research_knobs(tile, num_warps, num_stages, group_m, wrapped, partial_dot)

    def product(x_8, x_scale, weight, scale, bias):
        b32 = None if bias is None else bias.to(device=x_8.device, dtype=torch.float32).reshape(-1)
        y = int8_gemm_dequant(x_8, weight.T, x_scale, scale, b32, rounding="separate", **knobs)
        stats.hit(x_8.shape[0], weight.shape[0], x_8.shape[1])
        return y

    def candidate(x, weight, weight_scale, bias=None, out_dtype=torch.bfloat16, convrot=False,
                  convrot_groupsize=256, input_act=None, input_act_weight=None, input_act_eps=0.0,
                  residual=None, residual_scale=None):
        options = dict(bias=bias, convrot=convrot, convrot_groupsize=convrot_groupsize, input_act=input_act,
                       input_act_weight=input_act_weight, input_act_eps=input_act_eps, residual=residual,
                       residual_scale=residual_scale)
        if x.dtype != torch.float32 or out_dtype != torch.float32:
            stats.fallback()
            return saved(x, weight, weight_scale, out_dtype=out_dtype, **options)
        return _kitchen.fp32_linear(kitchen, x, weight, weight_scale, product=product, **options)

    with _kitchen.swapped(backend, {"int8_linear": candidate},
                          "MOSS eager export changed during the research context"):
        yield stats.data


# Source file of the patientx Qwen INT8 bridge (an external ComfyUI node)
# whose two GEMM wrappers the patientx candidate replaces.
_PATIENTX_BRIDGE = "RDNA2-Qwen21-INT8/rocm_int8_kitchen_patch.py"
_PATIENTX_WRAPPERS = ("triton_int8_linear", "triton_int8_linear_per_row")


def _loaded_patientx_bridge():
    hits = [mod for mod in tuple(sys.modules.values())
            if mod is not None and str(getattr(mod, "__file__", "")).endswith(_PATIENTX_BRIDGE)]
    if len(hits) != 1:
        raise RuntimeError("Expected one already-loaded Qwen patientx bridge")
    return hits[0]


def _patientx_weight_scale(weight_scale, weight, device, per_row):
    """The fp32 column-scale vector patientx hands its GEMM (int8_gemm.py:304-309):
    the per-row wrapper's [N] view, a tensor scale moved to the device, or a
    Python number as a one-element tensor."""
    if per_row:
        return weight_scale.reshape(weight.shape[0]).contiguous()
    if isinstance(weight_scale, torch.Tensor):
        return weight_scale.to(device, non_blocking=True).reshape(-1)
    return torch.tensor([weight_scale], device=device, dtype=torch.float32)


@contextmanager
def qwen_int8_gemm_candidate(patch_module=None, *, tile=(32, 64, 64),
                             num_warps=4, num_stages=1, group_m=4, wrapped=False, partial_dot=False):
    """Scoped replacement of the patientx bridge's two GEMM wrappers
    (``triton_int8_linear`` and ``triton_int8_linear_per_row``) by
    ``int8_gemm_dequant`` with the FMA epilogue (rounding="fused":
    fma(f32(acc), sa * sw, bias), the patientx Triton behaviour).

    Interface of rdna2-ops/rdna2_ops/int8_gemm.py:274-330. The bridge module
    is found among the loaded modules by its source path unless given; its own
    row quantizer (``triton_quantize_rowwise`` in the wrapper's globals) stays
    in use. fp32 input with compute_dtype fp32 is served, every other call goes
    to the saved wrapper (a fallback). Yields {"hits", "fallbacks", "shapes"};
    on exit both wrappers are restored, unless either was replaced meanwhile
    (RuntimeError).
    """
    bridge = _loaded_patientx_bridge() if patch_module is None else patch_module
    stats = _kitchen.CallStats()
    knobs = _research_knobs(tile, num_warps, num_stages, group_m, wrapped, partial_dot)

    def replacement_for(name):
        saved = getattr(bridge, name)
        per_row = name.endswith("_per_row")
        quantize = saved.__globals__["triton_quantize_rowwise"]

        def candidate(x, weight, weight_scale, bias=None, compute_dtype=torch.float16):
            if x.dtype != torch.float32 or compute_dtype != torch.float32:
                stats.fallback()
                return saved(x, weight, weight_scale, bias=bias, compute_dtype=compute_dtype)
            lead, k = x.shape[:-1], x.shape[-1]
            rows = x.reshape(-1, k)
            a, sa = quantize(rows.float() if per_row else rows)
            ws = _patientx_weight_scale(weight_scale, weight, x.device, per_row)
            y = int8_gemm_dequant(a, weight.T, sa, ws, bias, rounding="fused", **knobs)
            stats.hit(a.shape[0], weight.shape[0], a.shape[1])
            return y.reshape(*lead, weight.shape[0])

        return candidate

    with _kitchen.swapped(bridge, {name: replacement_for(name) for name in _PATIENTX_WRAPPERS},
                          "Qwen patientx callable changed during the research context"):
        yield stats.data
