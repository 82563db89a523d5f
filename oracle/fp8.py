"""Oracle for the FP8 weight-only GEMM path (test infrastructure only).

Restates, in numpy on the CPU:
  * _decode_bits (rdna2-ops/rdna2_ops/fp8_weight_gemm_v06.py:21-37): e4m3fn
    exponent 0 -> m * 2^-9, 0x7f / 0xff -> NaN, else (e + 120) << 23 | m << 20;
    e5m2 exponent 0 -> m * 2^-16, exponent 31 -> inf / NaN, else
    (e + 112) << 23 | m << 21; the sign bit on top;
  * the weight encoding of benchmark configuration 3: per output channel
    s = absmax / 448, w / s saturated to +-448, round to nearest even e4m3fn;
  * the weight-only product y = (A @ decode(W)^T) * s[n] (+ bias) in float64;
    the reference's own formulation has s = 1 and fp16 activations
    (fp8_weight_gemm_v06.py:49-73, "unscaled").

Pinned by tests/test_oracle_fp8.py: all 256 byte patterns against torch's own
float8_e4m3fn / float8_e5m2 -> float32 casts (a library routine, the
reference's known-answer test bench_dtype_gemm_v06.py:232-245), the encoder
against torch's RNE cast on random values and on every exact tie between two
neighbouring e4m3 values, and brute-force float64 loops for the product.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
E4M3_MAX = 448.0


def decode_bits(raw: np.ndarray, e5: bool = False) -> np.ndarray:
    """uint8 storage -> float32 values, bit for bit _decode_bits."""
    u = np.asarray(raw, dtype=np.uint8).astype(np.uint32)
    sign = (u & 128) << 24
    if e5:
        e, m = (u >> 2) & 31, u & 3
        normal = ((e + 112) << 23) | (m << 21)
        small = (m.astype(F32) * F32(0.0000152587890625)).view(np.uint32)
        bits = np.where(e == 0, small, normal)
        bits = np.where(e == 31, np.uint32(0x7F800000) | (m << 21), bits)
    else:
        e, m = (u >> 3) & 15, u & 7
        normal = ((e + 120) << 23) | (m << 20)
        small = (m.astype(F32) * F32(0.001953125)).view(np.uint32)
        bits = np.where(e == 0, small, normal)
        bits = np.where((e == 15) & (m == 7), np.uint32(0x7FC00000), bits)
    return (bits.astype(np.uint32) | sign).view(F32)


def _e4m3_table():
    vals = decode_bits(np.arange(128, dtype=np.uint8))  # non-negative half
    finite = np.isfinite(vals)
    codes = np.arange(128, dtype=np.uint8)[finite]
    return vals[finite].astype(np.float64), codes


def encode_e4m3(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn storage, saturating at +-448, round to nearest even
    (ties go to the code with an even mantissa, i.e. an even code)."""
    x = np.asarray(x, dtype=F32).astype(np.float64)
    if not np.isfinite(x).all():
        raise ValueError("finite input required")
    vals, codes = _e4m3_table()
    a = np.minimum(np.abs(x), E4M3_MAX)
    idx = np.searchsorted(vals, a)  # vals[idx-1] < a <= vals[idx]
    idx = np.clip(idx, 1, len(vals) - 1)
    lo_v, hi_v = vals[idx - 1], vals[idx]
    lo_c, hi_c = codes[idx - 1], codes[idx]
    d_lo, d_hi = a - lo_v, hi_v - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi_c % 2 == 0))
    code = np.where(pick_hi, hi_c, lo_c).astype(np.uint8)
    code = np.where(a == 0, np.uint8(0), code)
    return (code | np.where(np.signbit(x), np.uint8(128), np.uint8(0))).astype(np.uint8)


def quantize_weight_per_channel(w: np.ndarray):
    """Benchmark configuration 3: s[n] = absmax_n / 448 (1 for a zero row),
    codes = e4m3fn(sat(w / s)). Returns (uint8 codes [N, K], fp32 s [N])."""
    w = np.asarray(w, dtype=F32)
    s = (np.abs(w).max(1) / F32(E4M3_MAX)).astype(F32)
    s = np.where(s == 0, F32(1), s).astype(F32)
    return encode_e4m3((w / s[:, None]).astype(F32)), s


def fp8_linear(a, w_codes, w_scale=None, bias=None, e5=False):
    """float64 y = (a @ decode(w)^T) * s[n] + bias[n]."""
    w = decode_bits(w_codes, e5).astype(np.float64)
    y = np.asarray(a, np.float64) @ w.T
    if w_scale is not None:
        y = y * np.asarray(w_scale, np.float64)[None, :]
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y


def fp8_linear_bruteforce(a, w_codes, w_scale=None, bias=None, e5=False):
    w = decode_bits(w_codes, e5)
    m, k = np.asarray(a).shape
    n = w.shape[0]
    y = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            acc = sum(float(a[i, kk]) * float(w[j, kk]) for kk in range(k))
            if w_scale is not None:
                acc *= float(w_scale[j])
            y[i, j] = acc + (float(bias[j]) if bias is not None else 0.0)
    return y
