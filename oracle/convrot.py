"""Oracle for the ConvRot prologue and the residual epilogue (test infrastructure only).

Restates, in numpy on the CPU, the MOSS linear's optional steps around the
W8A8 product (rdna2-ops/rdna2_ops/comfy_int8.py:112-122 and :145, the same
lines as production/MOSS_RDNA2_INT8/backend.py):

  * ConvRot: every group of g consecutive K values of a row is multiplied by
    the normalised Hadamard matrix H_g / sqrt(g) before the per-row quantizer
    (Kitchen's ``_build_hadamard`` + ``_rotate_activation``; every MOSS call
    uses g = 256). Kitchen's helpers belong to comfy_kitchen 0.2.40, which is
    not vendored in the reference; its rotation is taken as the Sylvester-order
    matrix H[i][j] = (-1)^popcount(i & j), the one that both the
    Kronecker recursion and scipy.linalg.hadamard build.
  * the residual term: ``_apply_residual(y, residual, residual_scale)`` =
    y + residual (* residual_scale), after the scale and bias steps.

Kitchen's own arithmetic (dense fp32 product with H / sqrt(g)) and the gfx950
kernel (fast Walsh-Hadamard butterflies in fp32) form the same sums in a
different order. ``rotate_dense64`` is the exact-math rotation (float64);
``rotate_fwht32`` restates the kernel's fp32 butterfly order bit for bit, and
is pinned against the float64 rotation and the closed forms in
tests/test_oracle_convrot.py.
"""
from __future__ import annotations

import numpy as np

from . import int8 as o8

F32 = np.float32


def hadamard(g: int) -> np.ndarray:
    """Unnormalised Sylvester Hadamard matrix of order g (a power of two), float64,
    built from the entry formula H[i][j] = (-1)^popcount(i & j)."""
    if g < 1 or g & (g - 1):
        raise ValueError("g must be a power of two")
    i = np.arange(g, dtype=np.uint32)
    bits = i[:, None] & i[None, :]
    pop = np.zeros_like(bits)
    for s in range(max(1, g.bit_length())):
        pop += (bits >> np.uint32(s)) & np.uint32(1)
    return np.where(pop & 1, -1.0, 1.0)


def rotate_dense64(x, g: int) -> np.ndarray:
    """Exact-math ConvRot: each group of g values times H_g / sqrt(g), in float64."""
    x = np.asarray(x, dtype=np.float64)
    m, k = x.shape
    if k % g:
        raise ValueError("g must divide K")
    h = hadamard(g) / np.sqrt(g)
    return (x.reshape(m, k // g, g) @ h).reshape(m, k)


def rotate_fwht32(x, g: int) -> np.ndarray:
    """ConvRot in the gfx950 kernel's fp32 order: log2(g) butterfly stages
    h = 1, 2, 4, ..., g/2, each replacing (v[i], v[i + h]) by (v[i] + v[i + h],
    v[i] - v[i + h]) for every i whose bit h is clear, every operation rounded
    to fp32; then every value times fp32(1 / sqrt(g))."""
    v = np.array(x, dtype=np.float32, copy=True)
    m, k = v.shape
    if k % g or g & (g - 1):
        raise ValueError("g must be a power of two dividing K")
    h = 1
    while h < g:
        blocks = v.reshape(m, k // (2 * h), 2, h)
        a = blocks[:, :, 0, :].copy()
        c = blocks[:, :, 1, :].copy()
        blocks[:, :, 0, :] = (a + c).astype(np.float32)
        blocks[:, :, 1, :] = (a - c).astype(np.float32)
        h *= 2
    inv = F32(1.0 / np.sqrt(np.float64(g)))
    return (v * inv).astype(np.float32)


def rot_quant_rows(x, g: int, rounding="half_even"):
    """ConvRot (kernel order) then the per-row INT8 quantizer: (codes [M, K], steps [M])."""
    return o8.quant_rows(rotate_fwht32(x, g), rounding)


def residual_term(residual, residual_scale, n: int) -> np.ndarray:
    """f32(residual) times the fp32 residual scale (one value or [N]), rounded to fp32."""
    r = np.asarray(residual, dtype=np.float32)
    if residual_scale is None:
        return r
    s = np.asarray(residual_scale, dtype=np.float32).reshape(-1)
    if s.size not in (1, n):
        raise ValueError("residual_scale must hold 1 or N values")
    return (r * s.reshape(1, -1)).astype(np.float32)


def epilogue_f_residual(acc, a_scale, b_scale, bias=None, residual=None, residual_scale=None, *, out="f32",
                        fused=False, activation=None):
    """Order-F epilogue (oracle.int8.epilogue_f) with the residual term added in
    fp32 after the scale, bias and activation steps, then one rounding to
    ``out``. For out="f32" this is Kitchen's fp32 sequence scale -> + bias ->
    + residual (* residual_scale) (comfy_int8.py:135-145)."""
    v = o8.epilogue_f(acc, a_scale, b_scale, bias, out="f32", fused=fused, activation=activation)
    if residual is not None:
        v = (v + residual_term(residual, residual_scale, v.shape[1])).astype(np.float32)
    return o8.round_to(v, out)


def moss_linear(x, w_q, w_scale, bias=None, *, g=None, residual=None, residual_scale=None, out="f32",
                rounding="half_even"):
    """The MOSS INT8 linear with the optional steps: ConvRot (kernel order) ->
    per-row quantizer -> exact INT8 product -> order F -> residual."""
    x = np.asarray(x, dtype=np.float32)
    xr = rotate_fwht32(x, g) if g else x
    xq, xs = o8.quant_rows(xr, rounding)
    acc = o8.int8_matmul(xq, np.ascontiguousarray(np.asarray(w_q).T))
    y = epilogue_f_residual(acc, xs, w_scale, bias, residual, residual_scale, out=out)
    return y, xq, xs, acc
