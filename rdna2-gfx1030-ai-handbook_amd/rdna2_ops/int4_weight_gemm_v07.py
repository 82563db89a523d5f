# SPDX-License-Identifier: Apache-2.0
"""Grouped INT4 weight storage and the W4A16 GEMM on gfx950 (MI355X).

Drop-in for rdna2-ops/rdna2_ops/int4_weight_gemm_v07.py: ``PackedInt4``,
``pack_int4_cpu`` / ``unpack_int4_cpu``, ``pack_int4``, ``unpack_int4`` and
``int4_linear_a16`` keep their signatures, argument checks and storage
format (signed 4-bit q and fp32 scale / int32 zero point per output-row K
group, W = (q - zero) * scale; linear INT4, never a codebook format). The
device work runs in hand-written gfx950 HIP kernels of librdna2_qgemm.so
(C ABI: include/qgemm.h); a missing library is an error.

``int4_linear_a16`` methods:
  dequant   unpack_int4 (HIP) to fp16/bf16, then the library GEMM F.linear
            (the reference's "decode + rocBLAS" method);
  prepared  F.linear with a caller-owned dequantised weight;
  dot2      the fused kernel: nibbles are expanded in registers and fed to the
            bf16/fp16 MFMA; each group scale multiplies the exact group partial
            sum in fp32 (the reference's dot2 rounds each weight to fp16 first).
  fused     alias of dot2.

``int4_linear_a8`` (W4A8, int8 activations with a per-row scale): every
method of the reference (dot4, dot4_prepared, dot4_split, dot4_words, dot8)
runs one gfx950 kernel on the int8 MFMA with the reference's exact integer
group sums and fp32 group-scale order (bit-identical results);
``prepare_dot8_activation`` and ``int8_activation_to_fp16`` keep their
interfaces.

Extensions (defaults keep the reference's behaviour): bf16 activations (the
output and bias then are bf16), and the uint4 storage of benchmark configuration 2
``pack_uint4`` — unsigned nibbles, bf16 scales, uint4 zero points packed 8 per
int32 (PackedInt4 with ``signed=False, zeros_packed=True``).

The caller owns packed weights and re-packs them after weight/LoRA changes.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib

_GROUPS = (32, 64, 128)


@dataclass
class PackedInt4:
    """Caller-owned W4 weight (int4_weight_gemm_v07.py:20-46; derived from the
    reference's container, see the notice above pack_int4_cpu).

    ``signed`` / ``zeros_packed`` describe the storage coordinates: the
    reference format is signed=True, zeros_packed=False (int32 zero points);
    the uint4 format (unsigned nibbles, packed zero points) is signed=False, zeros_packed=True."""
    data: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    sums: torch.Tensor
    n: int
    k: int
    group_size: int
    symmetric: bool
    layout: str = "nk"
    order: str = "low"
    signed: bool = True
    zeros_packed: bool = False

    def to(self, device):
        return PackedInt4(*(t.to(device) for t in (self.data, self.scales, self.zeros, self.sums)),
                          self.n, self.k, self.group_size, self.symmetric, self.layout, self.order,
                          self.signed, self.zeros_packed)

    @property
    def bytes(self):
        return sum(t.numel() * t.element_size() for t in (self.data, self.scales, self.zeros, self.sums))

    @property
    def logical_stride(self):
        return self.data.stride() if self.layout == "nk" else self.data.T.stride()

    @property
    def flags(self):
        f = 0
        if self.signed:
            f |= _lib.W4_SIGNED_NIBBLES
        if self.order == "high":
            f |= _lib.W4_ORDER_HIGH
        if self.layout == "kn":
            f |= _lib.W4_LAYOUT_KN
        if self.zeros_packed:
            f |= _lib.W4_ZEROS_PACKED
        return f


# ------------------------------------------------------------------ CPU packing
# PackedInt4 above and pack_int4_cpu / unpack_int4_cpu below are derived from
# rdna2-ops/rdna2_ops/int4_weight_gemm_v07.py:20-92 (the storage container and
# the CPU pack rule are the interchange format packed weights must share with
# the reference; the expressions follow the reference's, with an int32-wrap
# fix and a shared shift helper). That code's notice:
#
#   MIT License
#
#   Copyright (c) 2026 rdna2-ops contributors
#
#   Permission is hereby granted, free of charge, to any person obtaining a
#   copy of this software and associated documentation files (the
#   "Software"), to deal in the Software without restriction, including
#   without limitation the rights to use, copy, modify, merge, publish,
#   distribute, sublicense, and/or sell copies of the Software, and to permit
#   persons to whom the Software is furnished to do so, subject to the
#   following conditions:
#
#   The above copyright notice and this permission notice shall be included
#   in all copies or substantial portions of the Software.
#
#   THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS
#   OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF
#   MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN
#   NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM,
#   DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR
#   OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE
#   USE OR OTHER DEALINGS IN THE SOFTWARE.
def _shifts(order):
    s = torch.arange(8, dtype=torch.int64) * 4
    return 28 - s if order == "high" else s


def pack_int4_cpu(w, *, group_size=64, symmetric=True, layout="nk", order="low"):
    """CPU packing with ties-to-even and an explicit range
    (int4_weight_gemm_v07.py:49-82); the GPU pack_int4 must equal it."""
    if w.device.type != "cpu" or w.ndim != 2 or not w.is_floating_point():
        raise ValueError("CPU floating-point [N,K] weight required")
    n, k = w.shape
    if group_size not in _GROUPS or k % group_size or layout not in ("nk", "kn") or order not in ("low", "high"):
        raise ValueError("K must be divisible by group size 32/64/128; valid layout/order required")
    if not torch.isfinite(w).all():
        raise ValueError("Finite weight required")
    x = w.float().reshape(n, k // group_size, group_size)
    if symmetric:
        scales = x.abs().amax(-1) / 7
        scales = torch.where(scales == 0, torch.ones_like(scales), scales)
        zeros = torch.zeros_like(scales, dtype=torch.int32)
        q = torch.round(x / scales[..., None]).clamp(-7, 7).to(torch.int32)
    else:
        zero = torch.zeros((), dtype=torch.float32)
        lo = torch.minimum(x.amin(-1), zero)
        hi = torch.maximum(x.amax(-1), zero)
        scales = (hi - lo) / 15
        empty = scales == 0
        scales = torch.where(empty, torch.ones_like(scales), scales)
        zu = torch.round(-lo / scales).clamp(0, 15).to(torch.int32)
        zeros = torch.where(empty, torch.zeros_like(zu), zu - 8)
        q = (torch.round(x / scales[..., None]) + zu[..., None]).clamp(0, 15).to(torch.int32) - 8
        q = torch.where(empty[..., None], torch.zeros_like(q), q)
    sums = q.sum(-1, dtype=torch.int32)
    nib = q.reshape(n, k // 8, 8).to(torch.int64) & 15
    words = (nib << _shifts(order)).sum(-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    if layout == "kn":
        words = words.T.contiguous()
    return PackedInt4(words, scales.contiguous(), zeros.contiguous(), sums.contiguous(),
                      n, k, group_size, bool(symmetric), layout, order)


def unpack_int4_cpu(p, *, floating=True):
    """(q - zero) * scale as fp32 [N, K], or the centred integers
    (int4_weight_gemm_v07.py:85-92)."""
    words = p.data.cpu() if p.layout == "nk" else p.data.cpu().T
    nib = ((words.to(torch.int64)[..., None] >> _shifts(p.order)) & 15).to(torch.int32)
    nib = nib.reshape(p.n, p.k // p.group_size, p.group_size)
    if p.signed:
        q = torch.where(nib >= 8, nib - 16, nib)
    else:
        q = nib
    if p.zeros_packed:
        ng = p.k // p.group_size
        zw = p.zeros.cpu().to(torch.int64)
        zn = ((zw[..., None] >> (torch.arange(8, dtype=torch.int64) * 4)) & 15).reshape(p.n, -1)[:, :ng]
        z = torch.where(zn >= 8, zn - 16, zn) if p.signed else zn
        z = z.to(torch.int32)
    else:
        z = p.zeros.cpu()
    centred = q - z[..., None]
    if not floating:
        return centred.reshape(p.n, p.k)
    return (centred.float() * p.scales.cpu().float()[..., None]).reshape(p.n, p.k)


# ------------------------------------------------------------------ device API
def _eager(*tensors):
    if (torch.compiler.is_compiling() or torch.cuda.is_current_stream_capturing()
            or torch.is_autocast_enabled("cuda") or torch.jit.is_tracing()
            or torch._C._are_functorch_transforms_active()
            or torch.is_grad_enabled() and any(t.requires_grad for t in tensors)):
        raise ValueError("Explicit eager inference only")


def _storage(n, k, group_size, layout, signed, zeros_packed, scale_dtype, device):
    data = torch.empty((n, k // 8) if layout == "nk" else (k // 8, n), device=device, dtype=torch.int32)
    scales = torch.empty((n, k // group_size), device=device, dtype=scale_dtype)
    ng = k // group_size
    zeros = torch.empty((n, (ng + 7) // 8) if zeros_packed else (n, ng), device=device, dtype=torch.int32)
    sums = torch.empty((n, ng), device=device, dtype=torch.int32)
    return data, scales, zeros, sums


def _pack(w, group_size, symmetric, layout, order, signed, zeros_packed, scale_dtype):
    if w.device.type != "cuda" or w.ndim != 2 or not w.is_floating_point():
        raise ValueError("Floating [N,K] weight on gfx950 required")
    _lib.require_gfx950(w)
    _eager(w)
    n, k = w.shape
    if group_size not in _GROUPS or k % group_size or min(n, k) <= 0 or n * k >= 2 ** 31:
        raise ValueError("Nonempty bounded shape and K divisible by 32/64/128 required")
    if layout not in ("nk", "kn") or order not in ("low", "high"):
        raise ValueError("Unknown packing layout/order")
    if min(w.stride()) <= 0:
        raise ValueError("Positive strides required")
    if w.dtype not in _lib.DTYPE_CODE or _lib.DTYPE_CODE[w.dtype] not in (_lib.F32, _lib.F16, _lib.BF16):
        raise ValueError("fp32 / fp16 / bf16 weight required")
    data, scales, zeros, sums = _storage(n, k, group_size, layout, signed, zeros_packed, scale_dtype, w.device)
    p = PackedInt4(data, scales, zeros, sums, n, k, group_size, bool(symmetric), layout, order,
                   signed, zeros_packed)
    _lib.check(_lib.library().qg_w4_pack(
        _lib.ptr(w), _lib.DTYPE_CODE[w.dtype], w.stride(0), w.stride(1), n, k, group_size,
        int(bool(symmetric)), p.flags, _lib.ptr(data), _lib.ptr(scales), _lib.DTYPE_CODE[scale_dtype],
        _lib.ptr(zeros), _lib.ptr(sums), _lib.stream_of(w)), "qg_w4_pack")
    return p


def pack_int4(w, *, group_size=64, symmetric=True, layout="nk", order="low"):
    """GPU packing, equal to pack_int4_cpu (int4_weight_gemm_v07.py:413-430)."""
    return _pack(w, group_size, symmetric, layout, order, True, False, torch.float32)


def pack_uint4(w, *, group_size=128):
    """uint4 storage of benchmark configuration 2: asymmetric, unsigned nibbles (nk, low
    order), bf16 scales (the scale is rounded to bf16 before the codes are
    computed) and uint4 zero points packed 8 per int32 along the groups."""
    return _pack(w, group_size, False, "nk", "low", False, True, torch.bfloat16)


def _validate(p):
    """Contract of int4_weight_gemm_v07.py:433-447 (arch: gfx950)."""
    if not isinstance(p, PackedInt4) or p.data.device.type != "cuda":
        raise ValueError("PackedInt4 on gfx950 required")
    _lib.require_gfx950(p.data)
    if (p.group_size not in _GROUPS or min(p.n, p.k) <= 0 or p.k % p.group_size or p.n * p.k >= 2 ** 31
            or p.layout not in ("nk", "kn") or p.order not in ("low", "high")
            or p.data.dtype != torch.int32 or not p.data.is_contiguous()
            or tuple(p.data.shape) != ((p.n, p.k // 8) if p.layout == "nk" else (p.k // 8, p.n))):
        raise ValueError("Invalid packed shape/storage")
    ng = p.k // p.group_size
    zshape = (p.n, (ng + 7) // 8) if p.zeros_packed else (p.n, ng)
    scale_dtypes = (torch.float32, torch.bfloat16)
    for t, dtypes, shape in ((p.scales, scale_dtypes, (p.n, ng)), (p.zeros, (torch.int32,), zshape),
                             (p.sums, (torch.int32,), (p.n, ng))):
        if t.device != p.data.device or t.dtype not in dtypes or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError("Invalid scale/zero/sum storage")
    if p.data.data_ptr() % 16:
        raise ValueError("Packed words must be 16-byte aligned")
    _eager(p.data, p.scales)


def unpack_int4(p, *, dtype=torch.float16):
    """(q - zero) * scale rounded once to ``dtype`` (fp16 / fp32 / bf16), or the
    centred integers (int8) — int4_weight_gemm_v07.py:450-458."""
    _validate(p)
    if dtype not in (torch.float16, torch.float32, torch.bfloat16, torch.int8):
        raise TypeError(dtype)
    out = torch.empty((p.n, p.k), device=p.data.device, dtype=dtype)
    _lib.check(_lib.library().qg_w4_unpack(
        _lib.ptr(p.data), p.n, p.k, p.group_size, p.flags, _lib.ptr(p.scales),
        _lib.DTYPE_CODE[p.scales.dtype], _lib.ptr(p.zeros), _lib.ptr(out), _lib.DTYPE_CODE[dtype],
        _lib.stream_of(p.data)), "qg_w4_unpack")
    return out


def _gemv1_applies(a, p):
    """Whether the C ABI serves this call with the single-row kernel
    (k_w4_gemv1): one bf16 activation row, the benchmark's uint4 storage (nk, low
    order, bf16 scales, packed zero points), group 128, K a multiple of 512 up
    to 4096, 16-byte aligned weights and activations."""
    a = a if (a.stride(1) == 1 and a.stride(0) % 8 == 0 and a.data_ptr() % 16 == 0) else a.contiguous()
    return (a.shape[0] == 1 and a.dtype == torch.bfloat16 and p.group_size == 128
            and p.flags == _lib.W4_ZEROS_PACKED and p.scales.dtype == torch.bfloat16
            and p.k % 512 == 0 and p.k <= 4096
            and p.data.data_ptr() % 16 == 0 and a.data_ptr() % 16 == 0
            and p.scales.data_ptr() % 4 == 0 and p.zeros.data_ptr() % 4 == 0)


def w4a16_gemm(a, p, bias=None, *, out_dtype=None):
    """The fused W4A16 kernel: out = a @ dequant(p)^T (+ bias), fp32
    accumulation, one rounding to out_dtype (default: a's dtype)."""
    m, k = a.shape
    out_dtype = a.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("out_dtype must be float16, bfloat16 or float32")
    if a.stride(1) != 1 or a.stride(0) % 8 or a.data_ptr() % 16:
        a = a.contiguous()
    out = torch.empty((m, p.n), device=a.device, dtype=out_dtype)
    if m == 0:
        return out
    lib = _lib.library()
    ws_bytes = lib.qg_w4a16_gemm_workspace_bytes(m, p.n, k, p.group_size, p.flags)
    wsp, wsn = _lib.ws_ptr(_lib.workspace(ws_bytes, a.device))
    _lib.check(lib.qg_w4a16_gemm(
        _lib.ptr(a), _lib.DTYPE_CODE[a.dtype], a.stride(0), m, k, _lib.ptr(p.data), p.n, p.group_size,
        p.flags, _lib.ptr(p.scales), _lib.DTYPE_CODE[p.scales.dtype], _lib.ptr(p.zeros), _lib.ptr(bias),
        _lib.DTYPE_CODE[bias.dtype] if bias is not None else 0, _lib.ptr(out), _lib.DTYPE_CODE[out_dtype],
        wsp, wsn, _lib.stream_of(a)), "qg_w4a16_gemm")
    return out


def int4_linear_a16(a, p, *, bias=None, method="dequant", prepared=None, tile=(64, 64, 32),
                    num_warps=4, return_kernel=False):
    """fp16 (or bf16) activation and output: decode + library GEMM, prepared
    library GEMM, or the fused dot2 kernel (int4_weight_gemm_v07.py:540-564)."""
    _validate(p)
    _eager(a)
    if a.dtype not in (torch.float16, torch.bfloat16) or a.ndim != 2 or a.shape[1] != p.k or a.device != p.data.device:
        raise ValueError("Matching FP16 activation [M,K] required")
    if min(a.stride()) <= 0 or a.shape[0] * p.n >= 2 ** 31:
        raise ValueError("Unsupported shape/stride")
    if bias is not None and (bias.dtype != a.dtype or bias.shape != (p.n,) or bias.device != a.device):
        raise ValueError("FP16 bias [N] required")
    if method in ("dequant", "prepared"):
        w = unpack_int4(p, dtype=a.dtype) if method == "dequant" else prepared
        if w is None or w.shape != (p.n, p.k) or w.dtype != a.dtype or w.device != a.device:
            raise ValueError("FP16 prepared weight required")
        result = torch.nn.functional.linear(a, w, bias)
        return (result, None) if return_kernel else result
    if method not in ("dot2", "fused"):
        raise ValueError(method)
    if len(tile) != 3 or any(x not in (16, 32, 64, 128) for x in tile) or p.k % tile[2]:
        raise ValueError("Supported dot2 tile required")
    if bias is not None and not bias.is_contiguous():
        bias = bias.contiguous()
    out = w4a16_gemm(a, p, bias)
    if return_kernel:
        # the C ABI's choice: past 64 rows the dequant formulation from the
        # group's tile threshold (K a multiple of 64), else the tiled MFMA kernel
        # (K a multiple of 128); the decode kernels for up to 16 rows and K <=
        # 4096; else skinny
        m = a.shape[0]
        if _lib.library().qg_w4a16_gemm_workspace_bytes(m, p.n, p.k, p.group_size, p.flags) > 0:
            # prefill grid at or past the group's threshold of 256 x 192 tiles
            # (192 at group 128, 64 at group 64, any at group 32): W
            # dequantised into the workspace, then the 2-byte ping-pong GEMM
            # (256 x 192 tiles, K stage of 64 elements; a grid past one round
            # of the 256 CUs whose last round would be partly idle runs its
            # remaining columns as one more launch of 128 x 128 tiles)
            return out, _lib.kernel_metadata("w4a16_dequant_pingpong", (256, 192, 64), "k_h16_gemm_pp")
        if m > 64 and p.k % 128 == 0:
            # 128 x 64 tiles for group 32, and where 128 x 128 tiles would
            # leave CUs idle (the launcher's wd_w4_tile_n)
            tiles = -(-m // 128) * -(-p.n // 128)
            tbn = 64 if p.group_size == 32 or tiles < (192 if p.group_size == 64 else 256) else 128
            fmt = 0 if (p.flags == _lib.W4_ZEROS_PACKED and p.group_size == 128 and p.scales.dtype != torch.float32) else 1
            hint = "k_wd_gemmILi{}ELi{}ELb{}ELb{}ELi2ELi4ELi128ELi{}E".format(
                fmt, p.group_size, int(bool(p.flags & _lib.W4_LAYOUT_KN)), int(a.dtype == torch.float16), tbn)
            return out, _lib.kernel_metadata("w4a16_tiled_mfma", (128, tbn, 128), hint)
        if m <= 16 and -(-p.k // 128) <= 32:
            if _gemv1_applies(a, p):
                return out, _lib.kernel_metadata("w4a16_gemv1", (1, 32, 512), "k_w4_gemv1")
            rp = 1 if m == 1 else 4 if m <= 4 else 16
            # column tiles of 16 per workgroup, as launch_decode_g picks them
            ct = (4 if rp == 16 else 2) if p.group_size == 128 else 2 if p.group_size == 64 else (1 if rp > 1 else 2)
            return out, _lib.kernel_metadata("w4a16_decode", (rp, 16 * ct, 128),
                                             "k_w4_decodeILi{}ELi{}ELi{}E".format(rp, ct, p.group_size))
        fm = 1 if m <= 16 else 2 if m <= 32 else 4
        return out, _lib.kernel_metadata("w4a16_skinny", (16 * fm, 16, 128), "k_w4_skinnyILi{}E".format(fm))
    return out


# ------------------------------------------------------------------ W4A8
_A8_METHODS = ("dot4", "dot4_prepared", "dot4_split", "dot4_words", "dot8")


def prepare_dot8_activation(a, p):
    """The reference's exact A8 recoding for its dot8 kernel
    (int4_weight_gemm_v07.py:455-464, _pack_a8 :156-171): caller-owned
    (low-nibble words of (a & 15) ^ 8, high-nibble words of (a >> 4) & 15,
    per-group sums of a). Kept for interface compatibility: the gfx950 W4A8
    kernel multiplies the int8 activations directly, so int4_linear_a8 only
    validates a prepared tuple and computes from ``a``."""
    _validate(p)
    if a.dtype != torch.int8 or a.ndim != 2 or a.shape[1] != p.k or a.device != p.data.device or min(a.stride()) <= 0:
        raise ValueError("Matching positive-stride A8[M,K] required")
    m, k = a.shape
    ai = a.to(torch.int64)
    shifts = torch.arange(8, device=a.device, dtype=torch.int64) * 4
    if p.order == "high":
        shifts = 28 - shifts

    def words(nib):
        v = (nib.reshape(m, k // 8, 8) << shifts).sum(-1)
        return (((v + 2 ** 31) % 2 ** 32) - 2 ** 31).to(torch.int32)

    lo = words((ai & 15) ^ 8)
    hi = words((ai >> 4) & 15)
    sums = ai.reshape(m, k // p.group_size, p.group_size).sum(-1).to(torch.int32)
    return lo, hi, sums


def int8_activation_to_fp16(a, scale):
    """fp16 [M, K] = fp32(a) * scale[m] rounded once (int4_weight_gemm_v07.py:467-471)."""
    m, k = a.shape
    return (a.to(torch.float32) * scale.reshape(-1, 1).to(torch.float32)).to(torch.float16).reshape(m, k)


def int4_linear_a8(a, p, a_scale, *, bias=None, method="dot4", tile=(64, 64), num_warps=4,
                   prepared=None, integer=False, return_kernel=False):
    """(A8 * row scale) @ reconstructed W4^T, fp32 output (int32 with
    ``integer``) — int4_weight_gemm_v07.py:476-537, argument checks in the
    reference's order.

    Every method computes the same numbers in the reference: per K group the
    exact integer sum of a * (q - z), folded into an fp32 total as
    total = total + f32(sum) * scale[n, g] (groups ascending, separate
    roundings), then * a_scale[m], then + bias. Here all of them run one
    gfx950 kernel on the int8 MFMA (qg_w4a8_gemm) that produces those bits;
    dot4_prepared feeds the caller's centred INT8 weights instead of the
    packed words. ``tile`` / ``num_warps`` are validated, not used."""
    _validate(p)
    _eager(a)
    if (a.ndim != 2 or a.dtype != torch.int8 or a.device != p.data.device or a.shape[1] != p.k
            or min(a.stride()) <= 0 or a.shape[0] * p.n >= 2 ** 31):
        raise ValueError("Matching A8[M,K] required")
    m, k = a.shape
    if (a_scale.shape not in ((m,), (m, 1)) or a_scale.device != a.device or a_scale.dtype != torch.float32
            or not a_scale.is_contiguous()):
        raise ValueError("Contiguous FP32 per-activation-row scale required")
    if bias is not None and (bias.shape != (p.n,) or bias.device != a.device or not bias.is_contiguous()
                             or not bias.is_floating_point()):
        raise ValueError("Floating bias [N] required")
    if len(tile) != 2 or any(x not in (8, 16, 32, 64, 128) for x in tile) or num_warps not in (4, 8):
        raise ValueError("Unsupported tile/warps")
    if k * 128 * 15 >= 2 ** 31:
        raise ValueError("Integer accumulator bound exceeded")
    out = torch.empty((m, p.n), device=a.device, dtype=torch.int32 if integer else torch.float32)
    bm, bn = tile
    w8 = None
    if method == "dot8":
        # the kernel needs no recoding of A; a caller's prepared tuple is checked
        if prepared is not None:
            if not isinstance(prepared, tuple) or len(prepared) != 3:
                raise ValueError("Dot8 prepared tuple required")
            al, ah, asum = prepared
            if (any(t.device != a.device or t.dtype != torch.int32 or not t.is_contiguous() for t in prepared)
                    or al.shape != (m, k // 8) or ah.shape != al.shape or asum.shape != (m, k // p.group_size)):
                raise ValueError("Invalid prepared activation shape/dtype")
    elif method in ("dot4", "dot4_prepared"):
        if method == "dot4_prepared":
            if prepared is None or prepared.shape != (p.n, k) or prepared.dtype != torch.int8 or prepared.device != a.device:
                raise ValueError("Centered INT8 prepared weight required")
            w8 = prepared if prepared.stride(1) == 1 and prepared.stride(0) % 16 == 0 and prepared.data_ptr() % 16 == 0 \
                else prepared.contiguous()
        if bm < 16 or bn < 16:
            raise ValueError("tl.dot tile dimensions must be >=16")
    elif method == "dot4_split":
        if bm < 16 or bn < 16:
            raise ValueError("tl.dot tile dimensions must be >=16")
    elif method != "dot4_words":
        raise ValueError(method)
    if m:
        # unit-K-stride rows on 16-byte boundaries for the kernel's copies
        av = a if a.stride(1) == 1 and a.stride(0) % 16 == 0 and a.data_ptr() % 16 == 0 else a.contiguous()
        b = bias
        if b is not None and b.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            b = b.to(torch.float32)
        _lib.check(_lib.library().qg_w4a8_gemm(
            _lib.ptr(av), av.stride(0), m, k, _lib.ptr(p.data), p.n, p.group_size, p.flags,
            _lib.ptr(p.scales), _lib.DTYPE_CODE[p.scales.dtype], _lib.ptr(p.zeros), _lib.ptr(w8),
            w8.stride(0) if w8 is not None else 0, _lib.ptr(a_scale), _lib.ptr(b),
            _lib.DTYPE_CODE[b.dtype] if b is not None else 0, _lib.ptr(out), int(integer), _lib.stream_of(av)),
            "qg_w4a8_gemm")
    if return_kernel:
        # the library's choice (csrc/w4a8_gemm.hip, use_n16): 16-column waves
        # for packed weights, K a multiple of 128 and a grid of at most 128
        # tiles of 128 x 128 (256 at g32)
        tiles = -(-m // 128) * -(-p.n // 128)
        if w8 is None and k % 128 == 0 and (tiles <= 128 or (tiles <= 256 and p.group_size == 32)):
            return out, _lib.kernel_metadata("w4a8_mfma_i32_16x16x32_i8", (128, 64), "k_w4a8_n16")
        return out, _lib.kernel_metadata("w4a8_mfma_i32_32x32x32_i8", (128, 128), "6k_w4a8I")
    return out
