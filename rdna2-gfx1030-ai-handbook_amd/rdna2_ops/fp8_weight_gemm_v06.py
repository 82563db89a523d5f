# SPDX-License-Identifier: Apache-2.0
"""FP8 (OCP e4m3fn / e5m2) weight-only GEMM on gfx950 (MI355X).

Drop-in for rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py: ``decode_fp8_weight``,
``prepare_int8_weight`` and ``fp8_weight_gemm`` keep their signatures,
methods, argument checks and caller-owned preparation contract. FP8 is a
storage format; the device work runs in hand-written gfx950 HIP kernels of
librdna2_qgemm.so (C ABI: include/qgemm.h):

  upcast        F.linear(a, w.to(a.dtype)) — the reference's native-cast baseline
  decode        the HIP decoder, then the library GEMM F.linear
  prepared_fp16 F.linear with a caller-owned decoded weight
  fused_dot2    the fused kernel: fp8 -> bf16 / fp16 conversion in registers in
                front of the MFMA, exact products, fp32 accumulation (the
                reference's fused Triton kernel, :49-73)
  int8          per-row INT8 quantisation (half away from zero) of A and of
                the decoded W, then the INT8 GEMM with the fp32 epilogue
  prepared_int8 the same with a caller-owned (INT8 weight, fp32 scale)

Extensions (defaults keep the reference's behaviour): bf16 activations (the
output and bias then are bf16) and ``w_scale``, an fp32 per-output-channel
scale applied to the fp32 accumulator before the bias (benchmark configuration
3: w_scale = absmax / 448, see ``quantize_weight_e4m3``).
"""
from __future__ import annotations

import torch

from . import _lib

_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)
_ACT = (torch.float16, torch.bfloat16)


def _weight(w):
    """Contract of fp8_weight_gemm_v06.py:100-106 (arch: gfx950)."""
    if w.ndim != 2 or w.dtype not in _FP8:
        raise TypeError("Weight must be a plain unscaled FP8 [N,K] tensor")
    if w.device.type != "cuda":
        raise ValueError("This explicit implementation targets HIP gfx950")
    _lib.require_gfx950(w)
    if min(w.shape) <= 0 or min(w.stride()) <= 0 or sum((n - 1) * s for n, s in zip(w.shape, w.stride())) >= 2 ** 31:
        raise ValueError("Nonempty positive strides and signed-32-bit address span required")


def decode_fp8_weight(w, *, out_dtype=torch.float16, metadata=None):
    """Decode each storage value; all finite FP8 values are exact in fp16,
    fp32 and bf16 (fp8_weight_gemm_v06.py:109-124)."""
    _weight(w)
    if out_dtype not in (torch.float16, torch.float32, torch.bfloat16):
        raise TypeError("Decode output must be FP16, FP32 or BF16")
    n, k = w.shape
    out = torch.empty((n, k), dtype=out_dtype, device=w.device)
    _lib.check(_lib.library().qg_fp8_decode(
        _lib.ptr(w), _lib.DTYPE_CODE[w.dtype], w.stride(0), w.stride(1), n, k, _lib.ptr(out),
        _lib.DTYPE_CODE[out_dtype], _lib.stream_of(w)), "qg_fp8_decode")
    if metadata is not None:
        metadata.update(method="software_decode", output_dtype=str(out_dtype), variant="k_fp8_decode")
    return out


def prepare_int8_weight(w):
    """Caller-owned (INT8 [N,K], fp32 per-output scale) of the decoded weight,
    rows quantised with the half-away-from-zero rule (:127-137, :76-92)."""
    _weight(w)
    n, k = w.shape
    if k > 32768:
        raise ValueError("This bounded row quantizer supports K<=32768")
    packed = torch.empty((n, k), dtype=torch.int8, device=w.device)
    scales = torch.empty(n, dtype=torch.float32, device=w.device)
    _lib.check(_lib.library().qg_quant_rows_i8(
        _lib.ptr(w), _lib.DTYPE_CODE[w.dtype], w.stride(0), w.stride(1), n, k, _lib.ptr(packed), k,
        _lib.ptr(scales), _lib.ROUND_HALF_AWAY, _lib.stream_of(w)), "qg_quant_rows_i8")
    return packed, scales


def quantize_weight_e4m3(w):
    """Benchmark configuration 3 weight preparation (offline): per output channel
    s = absmax / 448 (1 for an all-zero row), codes = e4m3fn(clamp(w / s, +-448))
    with round-to-nearest-even. Returns (codes [N, K] float8_e4m3fn, s [N] fp32)."""
    if w.ndim != 2 or not w.is_floating_point():
        raise ValueError("floating [N,K] weight required")
    x = w.float()
    s = x.abs().amax(1) / 448.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    codes = (x / s[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return codes, s.contiguous()


def _fused(a, w, bias, w_scale):
    m, k = a.shape
    n = w.shape[0]
    out = torch.empty((m, n), dtype=a.dtype, device=a.device)
    lib = _lib.library()
    ws_bytes = lib.qg_fp8w_gemm_workspace_bytes(_lib.ptr(a), a.stride(0), a.stride(1), _lib.ptr(w),
                                                w.stride(0), w.stride(1), m, n, k)
    wsp, wsn = _lib.ws_ptr(_lib.workspace(ws_bytes, a.device))
    _lib.check(lib.qg_fp8w_gemm(
        _lib.ptr(a), _lib.DTYPE_CODE[a.dtype], a.stride(0), a.stride(1), m, k, _lib.ptr(w),
        _lib.DTYPE_CODE[w.dtype], w.stride(0), w.stride(1), n, _lib.ptr(w_scale), _lib.ptr(bias),
        _lib.DTYPE_CODE[bias.dtype] if bias is not None else 0, _lib.ptr(out), _lib.DTYPE_CODE[a.dtype],
        wsp, wsn, _lib.stream_of(a)), "qg_fp8w_gemm")
    return out


def _int8_path(a, qw, sw, bias):
    """quant rows (half away) -> INT8 GEMM -> fp32 epilogue, rounded once to
    a.dtype: the reference's int8_gemm_dequant(...).to(a.dtype) (:181-193)."""
    from .int8_gemm import int8_gemm_dequant
    m, k = a.shape
    if k > 32768:
        raise ValueError("This bounded row quantizer supports K<=32768")
    qa = torch.empty((m, k), dtype=torch.int8, device=a.device)
    sa = torch.empty(m, dtype=torch.float32, device=a.device)
    _lib.check(_lib.library().qg_quant_rows_i8(
        _lib.ptr(a), _lib.DTYPE_CODE[a.dtype], a.stride(0), a.stride(1), m, k, _lib.ptr(qa), k, _lib.ptr(sa),
        _lib.ROUND_HALF_AWAY, _lib.stream_of(a)), "qg_quant_rows_i8")
    return int8_gemm_dequant(qa, qw.T, sa, sw, bias, tile=(64, 128, 64), num_warps=4, num_stages=2,
                             group_m=8, out_dtype=a.dtype)


def fp8_weight_gemm(a, w, *, bias=None, method="upcast", prepared=None, tile=(64, 64, 32), num_warps=4,
                    metadata=None, w_scale=None):
    """fp16 (or bf16) A[M,K] times FP8 weight[N,K] -> [M,N] in A's dtype
    (fp8_weight_gemm_v06.py:140-206). ``w_scale``: optional fp32 [N]
    per-channel scale (not in the reference)."""
    _weight(w)
    if a.ndim != 2 or a.shape[1] != w.shape[1] or a.dtype not in _ACT or a.device != w.device:
        raise ValueError("FP16 [M,K] activation and matching FP8 [N,K] weight required")
    if (torch.compiler.is_compiling() or torch.cuda.is_current_stream_capturing()
            or torch.is_autocast_enabled("cuda") or torch.jit.is_tracing() or torch.jit.is_scripting()
            or torch._C._are_functorch_transforms_active()
            or getattr(torch.autograd.forward_ad, "_current_level", -1) >= 0
            or torch.is_grad_enabled() and (a.requires_grad or w.requires_grad)):
        raise ValueError("Only explicit eager inference is supported")
    if min(a.shape) <= 0 or min(a.stride()) <= 0 or sum((n - 1) * s for n, s in zip(a.shape, a.stride())) >= 2 ** 31:
        raise ValueError("Nonempty positive-stride activation required")
    m, k = a.shape
    n = w.shape[0]
    if m * n >= 2 ** 31:
        raise ValueError("Output exceeds supported indexing span")
    if bias is not None and (bias.shape != (n,) or bias.device != a.device or bias.dtype != a.dtype
                             or not bias.is_contiguous() or torch.is_grad_enabled() and bias.requires_grad):
        raise ValueError("Bias must be a contiguous FP16 vector of length N")
    if w_scale is not None and (w_scale.shape != (n,) or w_scale.dtype != torch.float32
                                or w_scale.device != a.device or not w_scale.is_contiguous()):
        raise ValueError("w_scale must be a contiguous fp32 vector of length N")
    if method in ("upcast", "decode", "prepared_fp16"):
        if method == "upcast":
            wd = w.to(a.dtype)
        elif method == "decode":
            wd = decode_fp8_weight(w, out_dtype=a.dtype)
        else:
            if prepared is None or prepared.shape != w.shape or prepared.device != w.device or prepared.dtype != a.dtype:
                raise ValueError("Provide the current FP16 prepared weight")
            wd = prepared
        if w_scale is None:
            return torch.nn.functional.linear(a, wd, bias)
        y = torch.nn.functional.linear(a, wd).float() * w_scale[None, :]
        return (y + bias.float()[None, :] if bias is not None else y).to(a.dtype)
    if method in ("int8", "prepared_int8"):
        if w_scale is not None:
            raise ValueError("w_scale is applied by the fused / decode methods only")
        if method == "prepared_int8" and (not isinstance(prepared, tuple) or len(prepared) != 2):
            raise ValueError("Provide the current (INT8 weight, FP32 row scale)")
        qw, sw = prepare_int8_weight(w) if method == "int8" else prepared
        if (qw.shape != w.shape or qw.device != w.device or qw.dtype != torch.int8
                or sw.shape != (n,) or sw.device != w.device or sw.dtype != torch.float32):
            raise ValueError("Invalid prepared INT8 weight/scales")
        result = _int8_path(a, qw, sw, bias)
        if metadata is not None:
            metadata.update(method=method, variant="k_i8_gemm")
        return result
    if method != "fused_dot2":
        raise ValueError("Unknown method: " + method)
    if len(tile) != 3 or any(x not in (16, 32, 64, 128) for x in tile) or num_warps not in (4, 8):
        raise ValueError("Unsupported tile or warp count")
    result = _fused(a, w, bias, w_scale)
    if metadata is not None:
        # the C ABI's choice: >= 192 tiles of 256 x 192 run the 2-byte
        # ping-pong GEMM with fp8 W stages converted exactly to A's type in
        # registers; smaller grids the fused decode kernel (256 x 128 tiles
        # from four of them per CU)
        m, n = a.shape[0], w.shape[0]
        f16 = int(a.dtype == torch.float16)
        kp = -(-a.shape[1] // 128) * 128
        if (-(-m // 256)) * (-(-n // 192)) >= 192 and 2 * m * kp < 2 ** 31:
            variant = "fp8w_f16_pingpong" if f16 else "fp8w_bf16_pingpong"
            tile_used = (256, 192, 64)
            hint = "k_f8w_gemm_ppINS0_5F8GeoILi256ELi192ELi4ELi2ELi3EEELi{}ELb{}ELb{}E".format(
                _lib.DTYPE_CODE[a.dtype], f16, int(w.dtype == torch.float8_e5m2))
        else:
            wide = m >= 256 and (-(-m // 256)) * (-(-n // 128)) >= 4 * 256
            variant, tile_used = "fp8_fused_mfma", ((256, 128, 128) if wide else (128, 128, 128))
            hint = "k_wd_gemmILi{}ELi128ELb0ELb{}ELi2ELi4ELi{}ELi128E".format(
                3 if w.dtype == torch.float8_e5m2 else 2, f16, tile_used[0])
        metadata.update(_lib.kernel_metadata(variant, tile_used, hint), method=method,
                        tile=list(tile), launched_tile=list(tile_used), num_warps=num_warps)
    return result
