"""Oracle for the W4A16 group-dequant GEMM path (test infrastructure only).

Restates, in numpy on the CPU:
  * pack_int4_cpu / unpack_int4_cpu of the reference's PackedInt4 format
    (rdna2-ops/rdna2_ops/int4_weight_gemm_v07.py:49-92): per K-group affine
    quantisation with fp32 division and round-half-to-even, signed nibbles
    q & 15 with q in [-8, 7], int32 zero points in the same signed coordinates,
    "nk"/"kn" word layouts and "low"/"high" nibble order;
  * the uint4 storage of benchmark configuration 2 (this build's definition of "uint4
    packed 8 per int32, asymmetric, group 128, bf16 scales, uint4 zero
    points"): the same affine rule evaluated with the bf16-rounded scale,
    unsigned nibbles, low order, zero points packed 8 per int32 along groups;
  * the W4A16 product y = A @ ((q - z) * s)^T (+ bias) in float64, the closed
    form that int4_linear_a16 approximates (int4_weight_gemm_v07.py:365-387,
    :540-564; its fp16 rounding of each weight is not part of the oracle);
  * the grouped form of int4_model_switches_v07.py:19-34: per group an exact
    integer dot product, then the group scale;
  * W4A8 (int4_linear_a8, int4_weight_gemm_v07.py:476-537): the exact integer
    product and the fp32 group-scale accumulation in the reference's order.

Pinned by tests/test_oracle_int4.py: the reference's smoke patterns
(bench_int4_v07.py:89-95: an all-zero row, the 16 integer levels -8..7 and the
15 levels -7..7, which must round-trip exactly), hand-written words for every
nibble position in both orders, the rounding-error bound |w - dequant| <= s/2
for unclipped elements, signed/unsigned storage equivalence and brute-force
float64 loops for the product; W4A8 by scalar loops with one float32 rounding
per operation, a torch CPU formulation of the reference's grouped reference,
closed forms and planted mistakes.
"""
from __future__ import annotations

import numpy as np

from .int8 import bf16_bits_to_f32, f32_to_bf16_bits

F32 = np.float32
GROUPS = (32, 64, 128)


def _shifts(order: str) -> np.ndarray:
    s = np.arange(8, dtype=np.uint32) * np.uint32(4)
    return np.uint32(28) - s if order == "high" else s


def pack_words(q_nib: np.ndarray, order: str = "low") -> np.ndarray:
    """[N, K] nibbles (0..15) -> [N, K/8] int32 words, nibble e of a word at
    bits 4e ("low") or 28 - 4e ("high") (int4_weight_gemm_v07.py:76-80)."""
    n, k = q_nib.shape
    q8 = (q_nib.astype(np.uint32) & np.uint32(15)).reshape(n, k // 8, 8)
    words = np.bitwise_or.reduce(q8 << _shifts(order), axis=-1).astype(np.uint32)
    return words.view(np.int32)


def unpack_words(words: np.ndarray, k: int, order: str = "low") -> np.ndarray:
    """[N, K/8] int32 words -> [N, K] nibbles 0..15 (int32)."""
    w = np.ascontiguousarray(words).view(np.uint32)
    q = (w[..., None] >> _shifts(order)) & np.uint32(15)
    return q.reshape(w.shape[0], k).astype(np.int32)


def pack_int4_ref(w, *, group_size=64, symmetric=True, layout="nk", order="low"):
    """pack_int4_cpu (int4_weight_gemm_v07.py:49-82) in numpy.

    Returns dict(data int32, scales f32 [N, K/G], zeros int32 [N, K/G],
    sums int32 [N, K/G]); data is [N, K/8] ("nk") or [K/8, N] ("kn").
    """
    w = np.asarray(w)
    if w.ndim != 2:
        raise ValueError("[N,K] weight required")
    n, k = w.shape
    if group_size not in GROUPS or k % group_size or layout not in ("nk", "kn") or order not in ("low", "high"):
        raise ValueError("K must be divisible by group size 32/64/128; valid layout/order required")
    x = w.astype(F32).reshape(n, k // group_size, group_size)
    if not np.isfinite(x).all():
        raise ValueError("Finite weight required")
    if symmetric:
        scales = (np.abs(x).max(-1) / F32(7)).astype(F32)
        scales = np.where(scales == 0, F32(1), scales).astype(F32)
        zeros = np.zeros(scales.shape, np.int32)
        q = np.clip(np.rint(x / scales[..., None]), -7, 7).astype(np.int32)
    else:
        lo = np.minimum(x.min(-1), F32(0)).astype(F32)
        hi = np.maximum(x.max(-1), F32(0)).astype(F32)
        scales = ((hi - lo) / F32(15)).astype(F32)
        empty = scales == 0
        scales = np.where(empty, F32(1), scales).astype(F32)
        zu = np.clip(np.rint(-lo / scales), 0, 15).astype(np.int32)
        zeros = np.where(empty, 0, zu - 8).astype(np.int32)
        qf = np.rint(x / scales[..., None]).astype(F32) + zu[..., None].astype(F32)
        q = np.clip(qf, 0, 15).astype(np.int32) - 8
        q = np.where(empty[..., None], 0, q).astype(np.int32)
    sums = q.sum(-1, dtype=np.int64).astype(np.int32)
    words = pack_words(q.reshape(n, k) & 15, order)
    if layout == "kn":
        words = np.ascontiguousarray(words.T)
    return dict(data=words, scales=np.ascontiguousarray(scales), zeros=np.ascontiguousarray(zeros),
                sums=np.ascontiguousarray(sums), n=n, k=k, group_size=group_size,
                symmetric=bool(symmetric), layout=layout, order=order)


def unpack_int4_ref(p, *, floating=True):
    """unpack_int4_cpu (int4_weight_gemm_v07.py:85-92): (q - zero) * scale as
    fp32 [N, K], or the centred integers q - zero."""
    words = p["data"] if p["layout"] == "nk" else np.ascontiguousarray(p["data"].T)
    nib = unpack_words(words, p["k"], p["order"])
    q = np.where(nib >= 8, nib - 16, nib).reshape(p["n"], p["k"] // p["group_size"], p["group_size"])
    centred = q - p["zeros"][..., None]
    if not floating:
        return centred.reshape(p["n"], p["k"]).astype(np.int32)
    return (centred.astype(F32) * p["scales"][..., None]).reshape(p["n"], p["k"]).astype(F32)


# ----------------------------------------------------------------- uint4 storage, packed zero points
def pack_uint4_baseline(w, *, group_size=128):
    """Asymmetric uint4 storage of benchmark configuration 2.

    Per [N, group]: lo = min(min x, 0), hi = max(max x, 0),
    s = bf16((hi - lo) / 15) (1 for an all-zero group), zu = clip(rint(-lo/s), 0, 15),
    q = clip(rint(x/s) + zu, 0, 15); every division is fp32 with the bf16-rounded
    scale, every rounding half to even. Returns dict(data int32 [N, K/8] (low
    order), scales uint16 bf16 bits [N, K/G], zeros int32 [N, ceil(K/G/8)] with
    zero point g at bits 4*(g%8) of word g//8, q uint8 [N, K], zu uint8 [N, K/G]).
    """
    w = np.asarray(w)
    n, k = w.shape
    if group_size not in GROUPS or k % group_size:
        raise ValueError("K must be divisible by the group size")
    ng = k // group_size
    x = w.astype(F32).reshape(n, ng, group_size)
    lo = np.minimum(x.min(-1), F32(0)).astype(F32)
    hi = np.maximum(x.max(-1), F32(0)).astype(F32)
    s32 = ((hi - lo) / F32(15)).astype(F32)
    sbits = f32_to_bf16_bits(s32)
    s = bf16_bits_to_f32(sbits)
    empty = s == 0
    sbits = np.where(empty, f32_to_bf16_bits(np.ones_like(s)), sbits).astype(np.uint16)
    s = bf16_bits_to_f32(sbits)
    zu = np.clip(np.rint(-lo / s), 0, 15).astype(np.int32)
    q = np.clip(np.rint(x / s[..., None]).astype(F32) + zu[..., None].astype(F32), 0, 15).astype(np.int32)
    data = pack_words(q.reshape(n, k), "low")
    nzw = (ng + 7) // 8
    zpad = np.zeros((n, nzw * 8), np.int32)
    zpad[:, :ng] = zu
    zeros = pack_words(zpad, "low")
    return dict(data=data, scales=sbits, zeros=zeros, q=q.reshape(n, k).astype(np.uint8),
                zu=zu.astype(np.uint8), n=n, k=k, group_size=group_size)


def unpack_zeros_packed(zwords: np.ndarray, ngroups: int) -> np.ndarray:
    nib = unpack_words(zwords, zwords.shape[1] * 8, "low")
    return nib[:, :ngroups]


def dequant_baseline(p, *, floating=True):
    """(q - zu) * s as fp32 [N, K] (or the centred integers)."""
    n, k, g = p["n"], p["k"], p["group_size"]
    q = unpack_words(p["data"], k, "low").reshape(n, k // g, g)
    zu = unpack_zeros_packed(p["zeros"], k // g)
    centred = q - zu[..., None]
    if not floating:
        return centred.reshape(n, k).astype(np.int32)
    s = bf16_bits_to_f32(p["scales"])
    return (centred.astype(F32) * s[..., None]).reshape(n, k).astype(F32)


# ----------------------------------------------------------------- products
def w4a16_linear(a, centred, scales, group_size, bias=None):
    """float64 y[m, n] = sum_k a[m,k] * centred[n,k] * scales[n, k // G] (+ bias[n]).

    ``a`` holds the activation values (from fp16 / bf16 storage), ``centred``
    the integers q - zero, ``scales`` the fp32 values of the group scales."""
    a64 = np.asarray(a, np.float64)
    n, k = centred.shape
    w64 = centred.astype(np.float64) * np.repeat(np.asarray(scales, np.float64), group_size, axis=1)
    y = a64 @ w64.T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y


def grouped_reference(a, centred, scales, group_size, bias=None):
    """int4_model_switches_v07.py:19-34 in float64: per group the exact dot
    product sum_k a * (q - z), times the group scale, summed over groups."""
    a64 = np.asarray(a, np.float64)
    n, k = centred.shape
    total = np.zeros((a64.shape[0], n))
    for g in range(k // group_size):
        sl = slice(g * group_size, (g + 1) * group_size)
        total += (a64[:, sl] @ centred[:, sl].astype(np.float64).T) * np.asarray(scales, np.float64)[:, g][None, :]
    if bias is not None:
        total = total + np.asarray(bias, np.float64)[None, :]
    return total


def w4a16_linear_bruteforce(a, centred, scales, group_size, bias=None):
    """Scalar loops; tiny inputs only."""
    m, k = np.asarray(a).shape
    n = centred.shape[0]
    y = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                acc += float(a[i, kk]) * int(centred[j, kk]) * float(scales[j, kk // group_size])
            y[i, j] = acc + (float(bias[j]) if bias is not None else 0.0)
    return y


# ----------------------------------------------------------------- W4A8
def w4a8_integer(a, centred):
    """The integer=True result of int4_linear_a8 (int4_weight_gemm_v07.py:476-537):
    exact int64 [M, N] = sum_k a[m, k] (q - z)[n, k] (float64 BLAS is exact:
    |sum| <= 128 * 15 * K < 2^53)."""
    return np.rint(np.asarray(a, np.float64) @ np.asarray(centred, np.float64).T).astype(np.int64)


def w4a8_linear(a, centred, scales, a_scale, group_size, bias=None):
    """The float result of int4_linear_a8 in the reference's declared order
    (_linear_dot4 int4_weight_gemm_v07.py:200-217, grouped_integer_reference
    int4_model_switches_v07.py:19-34): per group g the exact integer dot
    acc_g (exact in fp32: |acc_g| <= 128 * 15 * 128 < 2^24), then in fp32 with
    a rounding after every operation
        total = 0; for g ascending: total = total + f32(acc_g) * scale[n, g]
        y = total * a_scale[m]; y = y + f32(bias[n]).
    a int8 [M, K]; centred int [N, K] = q - zero; scales [N, K/G] (fp32
    values); returns fp32 [M, N]."""
    a64 = np.asarray(a, np.float64)
    c64 = np.asarray(centred, np.float64)
    m, k = a64.shape
    n = c64.shape[0]
    s = np.asarray(scales, F32)
    total = np.zeros((m, n), F32)
    for g in range(k // group_size):
        sl = slice(g * group_size, (g + 1) * group_size)
        acc = (a64[:, sl] @ c64[:, sl].T).astype(F32)  # exact
        total = (total + (acc * s[:, g][None, :]).astype(F32)).astype(F32)
    y = (total * np.asarray(a_scale, F32).reshape(-1)[:, None]).astype(F32)
    if bias is not None:
        y = (y + np.asarray(bias, F32).reshape(1, -1)).astype(F32)
    return y


def w4a8_linear_bruteforce(a, centred, scales, a_scale, group_size, bias=None):
    """Scalar loops with np.float32 scalars, one rounding per operation; tiny
    inputs only."""
    m, k = np.asarray(a).shape
    n = np.asarray(centred).shape[0]
    y = np.zeros((m, n), F32)
    for i in range(m):
        for j in range(n):
            total = F32(0)
            for g in range(k // group_size):
                acc = 0
                for kk in range(g * group_size, (g + 1) * group_size):
                    acc += int(a[i, kk]) * int(centred[j, kk])
                total = F32(total + F32(F32(acc) * F32(scales[j, g])))
            v = F32(total * F32(np.asarray(a_scale).reshape(-1)[i]))
            if bias is not None:
                v = F32(v + F32(bias[j]))
            y[i, j] = v
    return y
