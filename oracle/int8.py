"""Oracle for the W8A8 INT8 GEMM path (test infrastructure only).

Restates, in numpy on the CPU:
  * the exact INT8 x INT8 -> INT32 product of _int8_dot_dequant
    (rdna2-ops/rdna2_ops/int8_gemm.py:41-52) — the reference's own oracle is
    ``a.to(int64) @ b.to(int64)`` (rdna2-ops/bench_int8_gemm.py:189);
  * epilogue order F, int8_gemm.py:53-63 with enable_fp_fusion=False (:191):
    value = f32(acc) * (sa[m] * sb[n]); value = value + f32(bias[n]);
    then one RNE rounding to the output dtype (fp8_weight_gemm_v06.py:193);
  * the rounding="fused" epilogue (FMA of f32(acc), scale, bias; :191);
  * epilogue order E, the Kitchen eager chunk loop
    (rdna2-ops/rdna2_ops/comfy_int8.py:128-143): t = out(f32(acc) * (sa*sw));
    t = out(f32(t) + f32(out(bias)));
  * the per-row quantizer of fp8_weight_gemm_v06.py:76-92 (half away from zero)
    and the per-token rule of the benchmark (absmax / 127, round half to even);
  * GELU tanh approximation in the operation order of ATen's CPU kernel.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


# --------------------------------------------------------------------------- dtypes
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even; NaN -> quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def round_to(x: np.ndarray, out: str) -> np.ndarray:
    """Round fp32 values to ``out`` ("f32", "f16", "bf16") and return them as fp32."""
    x = np.asarray(x, dtype=np.float32)
    if out == "f32":
        return x
    if out == "f16":
        return x.astype(np.float16).astype(np.float32)
    if out == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    raise ValueError(out)


def encode(x: np.ndarray, out: str) -> np.ndarray:
    """fp32 values -> storage of ``out`` (float32 / float16 / uint16 bf16 bits)."""
    if out == "f32":
        return np.asarray(x, dtype=np.float32)
    if out == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16)
    if out == "bf16":
        return f32_to_bf16_bits(x)
    raise ValueError(out)


# --------------------------------------------------------------------------- GEMM
def int8_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact int8 [M,K] @ int8 [K,N] -> int32 (int8_gemm.py:41-52).

    Computed in float64 BLAS: every product is an integer <= 2^14 in magnitude
    and every partial sum an integer <= K * 2^14 <= 2^31 < 2^53, so all
    intermediate values are exact whatever the summation order.
    """
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype != np.int8 or b.dtype != np.int8 or a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("int8 [M,K] @ [K,N] required")
    if a.shape[1] > 131071:
        raise ValueError("K bound (int8_gemm.py:142-143)")
    acc = a.astype(np.float64) @ b.astype(np.float64)
    return acc.astype(np.int64).astype(np.int32)


def int8_matmul_bruteforce(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Pure-Python triple loop, for tiny inputs only (pins int8_matmul)."""
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), dtype=np.int64)
    for i in range(m):
        for j in range(n):
            s = 0
            for t in range(k):
                s += int(a[i, t]) * int(b[t, j])
            out[i, j] = s
    return out.astype(np.int32)


# --------------------------------------------------------------------------- FMA
def fma_f32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Correctly rounded fp32 fma(a, b, c), vectorised.

    a*b is exact in float64 (24+24 significand bits). s = p + c is computed in
    float64 with its exact error e (TwoSum); rounding s to fp32 differs from
    rounding the exact value s + e only when s lies exactly halfway between two
    fp32 neighbours (or is exactly representable while e != 0 cannot move it
    past a midpoint) — that case is resolved by the sign of e.
    """
    a = np.asarray(a, np.float32).astype(np.float64)
    b = np.asarray(b, np.float32).astype(np.float64)
    c = np.asarray(c, np.float32).astype(np.float64)
    p = a * b
    s = p + c
    bb = s - p
    e = (p - (s - bb)) + (c - bb)
    r = s.astype(np.float32)
    # Detect s exactly at an fp32 rounding midpoint: s differs from r by half an ulp.
    r64 = r.astype(np.float64)
    up = np.nextafter(r, np.float32(np.inf)).astype(np.float64)
    dn = np.nextafter(r, np.float32(-np.inf)).astype(np.float64)
    mid_up = (s - r64) == (up - r64) / 2
    mid_dn = (r64 - s) == (r64 - dn) / 2
    fix_up = mid_up & (e > 0)
    fix_dn = mid_dn & (e < 0)
    # s at a midpoint rounded to even r; the exact value is beyond the midpoint
    r = np.where(fix_up, np.nextafter(r, np.float32(np.inf)), r)
    r = np.where(fix_dn, np.nextafter(r, np.float32(-np.inf)), r)
    # s at a midpoint rounded away from r toward the other neighbour is impossible
    # (r is the nearest-even of s); e of the opposite sign keeps r. Values of s
    # that are exactly representable in fp32 with e != 0 round to r as well.
    return r.astype(np.float32)


# --------------------------------------------------------------------------- epilogues
def gelu_tanh(v: np.ndarray) -> np.ndarray:
    """0.5*x*(1+tanh(sqrt(2/pi)*(x+0.044715*x^3))) in fp32, ATen CPU op order."""
    x = np.asarray(v, dtype=np.float32)
    k_beta = F32(0.7978845608028654)
    k_kappa = F32(0.044715)
    x_cube = x * x * x
    inner = k_beta * (x + k_kappa * x_cube)
    return (F32(0.5) * x * (F32(1.0) + np.tanh(inner))).astype(np.float32)


def epilogue_f(acc, a_scale, b_scale, bias=None, *, out="f32", fused=False, activation=None):
    """Order F (int8_gemm.py:53-63); fused=True is the rounding="fused" FMA form.

    Returns the output values as fp32 (already rounded to ``out``).
    """
    acc = np.asarray(acc, dtype=np.int32)
    m, n = acc.shape
    sa = np.asarray(a_scale, dtype=np.float32).reshape(m, 1)
    sb = np.asarray(b_scale, dtype=np.float32).reshape(1, -1)
    scale = (sa * sb).astype(np.float32)  # sa[:, None] * sb[None, :]
    accf = acc.astype(np.float32)          # RNE int32 -> fp32
    if bias is not None:
        bv = np.asarray(bias, dtype=np.float32).reshape(1, n)
        if fused:
            v = fma_f32(accf, np.broadcast_to(scale, (m, n)), np.broadcast_to(bv, (m, n)))
        else:
            v = (accf * scale).astype(np.float32)
            v = (v + bv).astype(np.float32)
    else:
        v = (accf * scale).astype(np.float32)
    if activation == "gelu_tanh":
        v = gelu_tanh(v)
    elif activation is not None:
        raise ValueError(activation)
    return round_to(v, out)


def epilogue_e(acc, a_scale, w_scale, bias=None, *, out="f32"):
    """Order E, the Kitchen eager chunk loop (comfy_int8.py:128-143)."""
    acc = np.asarray(acc, dtype=np.int32)
    m, n = acc.shape
    sa = np.asarray(a_scale, dtype=np.float32).reshape(m, 1)
    sw = np.asarray(w_scale, dtype=np.float32).reshape(1, -1)
    t = round_to((acc.astype(np.float32) * (sa * sw).astype(np.float32)).astype(np.float32), out)
    if bias is not None:
        t = round_to((t + round_to(np.asarray(bias, np.float32).reshape(1, n), out)).astype(np.float32), out)
    return t


# --------------------------------------------------------------------------- quantizer
def quant_rows(x, rounding="half_even"):
    """Per-row INT8 quantization; returns (int8 codes [M,K], fp32 steps [M]).

    step = max(absmax / 127, 1e-20) and z = x / step, both IEEE fp32
    (fp8_weight_gemm_v06.py:87-88). half_away: q = floor(z + 0.5) if z >= 0
    else ceil(z - 0.5), with z +/- 0.5 rounded in fp32 (:89); half_even:
    q = rint(z). Then clamp to [-127, 127] (:90).
    """
    x = np.asarray(x, dtype=np.float32)
    if x.ndim != 2:
        raise ValueError("2-D input required")
    amax = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    step = np.maximum((amax / F32(127.0)).astype(np.float32), F32(1e-20)).astype(np.float32)
    z = (x / step[:, None]).astype(np.float32)
    if rounding == "half_even":
        q = np.rint(z)
    elif rounding == "half_away":
        q = np.where(z >= 0, np.floor((z + F32(0.5)).astype(np.float32)),
                     np.ceil((z - F32(0.5)).astype(np.float32)))
    else:
        raise ValueError(rounding)
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, step


def quantize_weight_per_channel(w, rounding="half_even"):
    """Symmetric per-output-channel int8 weight quantization (scale = absmax/127),
    the benchmark's weight preparation; identical arithmetic to quant_rows."""
    return quant_rows(w, rounding)


def w8a8_linear(x, w_q, w_scale, bias=None, *, out="f16", rounding="half_even", activation=None):
    """quant(x) -> int8 GEMM -> order-F epilogue (the fused W8A8 linear)."""
    xq, xs = quant_rows(x, rounding)
    acc = int8_matmul(xq, np.ascontiguousarray(np.asarray(w_q).T))
    return epilogue_f(acc, xs, w_scale, bias, out=out, activation=activation), xq, xs, acc
