"""Pins of oracle/int4.py (CPU only).

Every check here is independent of the formula it tests: known-answer patterns
from the reference's own smoke test (rdna2-ops/bench_int4_v07.py:89-95),
hand-written bit layouts, error bounds that any correct affine quantiser must
meet, and brute-force loops for the product.
"""
import numpy as np
import pytest

from oracle import int4 as o4
from oracle.int8 import bf16_bits_to_f32



def smoke_weight(n=19, k=384, seed=20261107):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.2).astype(np.float32)
    w[0] = 0
    w[1] = (np.arange(k) % 16) - 8
    w[2] = (np.arange(k) % 15) - 7
    return w


@pytest.mark.parametrize("g", o4.GROUPS)
@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("order", ["low", "high"])
def test_smoke_patterns_known_answers(g, sym, layout, order):
    w = smoke_weight()
    p = o4.pack_int4_ref(w, group_size=g, symmetric=sym, layout=layout, order=order)
    n, k = w.shape
    assert p["data"].shape == ((n, k // 8) if layout == "nk" else (k // 8, n))
    assert p["data"].dtype == np.int32 and p["scales"].dtype == np.float32
    # row 0 is all zero: scale 1, zero point 0, every code 0
    assert (p["scales"][0] == 1).all() and (p["zeros"][0] == 0).all()
    deq = o4.unpack_int4_ref(p)
    assert (deq[0] == 0).all()
    # row 2 holds the 15 integers -7..7: symmetric scale 7/7 = 1 -> exact
    if sym:
        assert (p["scales"][2] == 1).all()
        assert np.array_equal(deq[2], w[2])
    else:
        # row 1 holds -8..7 in every group: lo=-8, hi=7 -> s=1, zu=8 -> exact
        assert (p["scales"][1] == 1).all() and (p["zeros"][1] == 0).all()
        assert np.array_equal(deq[1], w[1])
        assert np.array_equal(o4.unpack_int4_ref(p, floating=False)[1], w[1].astype(np.int32))
    # sums are the per-group sums of the signed codes
    nib = o4.unpack_words(p["data"] if layout == "nk" else np.ascontiguousarray(p["data"].T), k, order)
    q = np.where(nib >= 8, nib - 16, nib)
    assert np.array_equal(p["sums"], q.reshape(n, k // g, g).sum(-1))


@pytest.mark.parametrize("order,expect", [("low", 0x76543210), ("high", 0x01234567)])
def test_nibble_positions_by_hand(order, expect):
    q = np.arange(16, dtype=np.int32).reshape(2, 8)  # all 16 levels
    words = o4.pack_words(q, order).view(np.uint32)
    hi = 0xFEDCBA98 if order == "low" else 0x89ABCDEF
    assert words[0, 0] == expect and words[1, 0] == hi
    assert np.array_equal(o4.unpack_words(words.view(np.int32), 8, order), q)


def test_signed_levels_store_q_and_15():
    # signed q in [-8, 7] is stored as q & 15 (int4_weight_gemm_v07.py:76)
    q = np.array([[-8, -7, -1, 0, 1, 6, 7, -2]], np.int32)
    words = o4.pack_words(q & 15, "low").view(np.uint32)
    assert words[0, 0] == 0xE7610F98


@pytest.mark.parametrize("g", o4.GROUPS)
@pytest.mark.parametrize("sym", [True, False])
def test_rounding_error_bound(g, sym):
    rng = np.random.default_rng(g + sym)
    w = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    p = o4.pack_int4_ref(w, group_size=g, symmetric=sym)
    deq = o4.unpack_int4_ref(p).reshape(8, -1, g)
    s = p["scales"][..., None]
    err = np.abs(deq - w.reshape(8, -1, g))
    # asymmetric: lo..hi is covered, so every element rounds to within s/2
    # (plus the fp32 rounding of x/s); symmetric: +-7 s covers +-absmax.
    assert (err <= s * (0.5 + 1e-5)).all()
    cen = o4.unpack_int4_ref(p, floating=False)
    assert cen.min() >= -15 and cen.max() <= 15
    if sym:
        assert (p["zeros"] == 0).all() and np.abs(cen).max() <= 7


def test_reference_and_baseline_storage_agree_on_centred_values():
    # (q - zero) in signed coordinates equals (q_u - z_u) in unsigned ones
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    p = o4.pack_int4_ref(w, group_size=128, symmetric=False)
    nib = o4.unpack_words(p["data"], 256, "low")
    q_signed = np.where(nib >= 8, nib - 16, nib)
    q_u = nib ^ 8  # unsigned nibble of the same level
    z_u = p["zeros"] + 8
    assert np.array_equal(q_u, q_signed + 8)
    cen_u = q_u.reshape(16, 2, 128) - z_u[..., None]
    assert np.array_equal(cen_u.reshape(16, 256), o4.unpack_int4_ref(p, floating=False))


def test_baseline_format_layout_and_bounds():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((32, 1024)) * 0.02).astype(np.float32)
    w[3] = 0
    p = o4.pack_uint4_baseline(w, group_size=128)
    assert p["data"].shape == (32, 128) and p["scales"].shape == (32, 8) and p["zeros"].shape == (32, 1)
    # zero points: group g at bits 4*(g%8) of word g//8
    z = p["zeros"].view(np.uint32)[:, 0]
    for g in range(8):
        assert np.array_equal((z >> (4 * g)) & 15, p["zu"][:, g])
    s = bf16_bits_to_f32(p["scales"])
    assert (s[3] == 1).all() and (p["zu"][3] == 0).all()
    deq = o4.dequant_baseline(p)
    assert (deq[3] == 0).all()
    err = np.abs(deq - w).reshape(32, 8, 128)
    # with the bf16-rounded scale the grid still spans [lo, hi] up to one
    # bf16 rounding of s (relative 2^-9) times 15 steps
    assert (err <= s[..., None] * (0.5 + 15 * 2.0 ** -8)).all()
    assert np.array_equal(o4.unpack_words(p["data"], 1024, "low"), p["q"].astype(np.int32))


def test_baseline_zero_words_pad_partial_groups():
    w = np.ones((2, 96 * 4), np.float32)  # 12 groups of 32 -> 2 zero words
    p = o4.pack_uint4_baseline(w, group_size=32)
    assert p["zeros"].shape == (2, 2)
    assert (p["zeros"].view(np.uint32)[:, 1] >> 16 == 0).all()


@pytest.mark.parametrize("g", [32, 64])
def test_product_bruteforce_and_grouped_form(g):
    rng = np.random.default_rng(11)
    m, n, k = 3, 5, 2 * g
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    p = o4.pack_int4_ref(w, group_size=g, symmetric=False)
    cen = o4.unpack_int4_ref(p, floating=False)
    bias = rng.standard_normal(n).astype(np.float32)
    y = o4.w4a16_linear(a, cen, p["scales"], g, bias)
    yb = o4.w4a16_linear_bruteforce(a, cen, p["scales"], g, bias)
    yg = o4.grouped_reference(a, cen, p["scales"], g, bias)
    np.testing.assert_allclose(y, yb, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(yg, yb, rtol=1e-12, atol=1e-12)
    # and equals the dense product with the dequantised fp32 weight
    deq = o4.unpack_int4_ref(p).astype(np.float64)
    np.testing.assert_allclose(y, a.astype(np.float64) @ deq.T + bias, rtol=1e-6, atol=1e-6)


def test_pack_rejects_bad_arguments():
    with pytest.raises(ValueError):
        o4.pack_int4_ref(np.zeros((2, 100), np.float32), group_size=32)
    with pytest.raises(ValueError):
        o4.pack_int4_ref(np.zeros((2, 128), np.float32), group_size=16)
    w = np.zeros((2, 128), np.float32)
    w[0, 0] = np.inf
    with pytest.raises(ValueError):
        o4.pack_int4_ref(w, group_size=32)


# ----------------------------------------------------------------- W4A8
def _a8_case(seed, m, n, k, g, sym=False):
    rng = np.random.default_rng(seed)
    a = rng.integers(-128, 128, (m, k)).astype(np.int8)
    w = (rng.standard_normal((n, k)) * 0.01).astype(np.float32)
    p = o4.pack_int4_ref(w, group_size=g, symmetric=sym)
    centred = o4.unpack_int4_ref(p, floating=False)
    sa = (rng.random(m) * 0.02 + 0.001).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
    return a, centred, p["scales"], sa, bias


@pytest.mark.parametrize("g", [32, 64, 128])
def test_w4a8_oracle_matches_scalar_loops(g):
    """The vectorised oracle equals scalar loops with one float32 rounding per
    operation, bit for bit (float and integer results)."""
    a, c, s, sa, bias = _a8_case(g, 3, 5, 2 * g, g)
    assert np.array_equal(o4.w4a8_linear(a, c, s, sa, g, bias), o4.w4a8_linear_bruteforce(a, c, s, sa, g, bias))
    assert np.array_equal(o4.w4a8_linear(a, c, s, sa, g), o4.w4a8_linear_bruteforce(a, c, s, sa, g))
    ref = np.array([[sum(int(a[i, kk]) * int(c[j, kk]) for kk in range(a.shape[1])) for j in range(5)]
                    for i in range(3)])
    assert np.array_equal(o4.w4a8_integer(a, c), ref)


def test_w4a8_oracle_matches_torch_grouped_reference():
    """The reference's own grouped reference (int4_model_switches_v07.py:19-34:
    torch fp32 mm per group, which is exact here, then torch mul / add in
    the declared order), formulated with torch on the CPU, is bit-identical."""
    import torch
    a, c, s, sa, bias = _a8_case(7, 37, 53, 384, 32)
    at, ct = torch.from_numpy(a), torch.from_numpy(c.astype(np.int8))
    st = torch.from_numpy(s)
    total = torch.zeros((37, 53), dtype=torch.float32)
    for gi in range(384 // 32):
        exact = torch.mm(at[:, gi * 32:(gi + 1) * 32].float(), ct[:, gi * 32:(gi + 1) * 32].float().T)
        total = total + exact * st[:, gi][None, :]
    y = total * torch.from_numpy(sa).reshape(-1, 1) + torch.from_numpy(bias).reshape(1, -1)
    assert np.array_equal(o4.w4a8_linear(a, c, s, sa, 32, bias), y.numpy())


def test_w4a8_closed_forms():
    """Unit scales and no bias: the float result is the exact integer product
    (|sum| < 2^24); a = 1 everywhere: column sums of q - z."""
    a, c, s, sa, _ = _a8_case(3, 6, 7, 256, 64)
    ones_s = np.ones_like(s)
    ones_a = np.ones(6, np.float32)
    assert np.array_equal(o4.w4a8_linear(a, c, ones_s, ones_a, 64), o4.w4a8_integer(a, c).astype(np.float32))
    a1 = np.ones((2, 256), np.int8)
    assert np.array_equal(o4.w4a8_integer(a1, c), np.repeat(c.sum(1)[None, :], 2, 0))


def test_w4a8_planted_mistakes_are_caught():
    """Plausible slips — the zero point dropped, the row scale applied per
    group before the sum, the groups summed in reverse, one fused multiply-add
    instead of two roundings — each change the result."""
    a, c, s, sa, bias = _a8_case(11, 16, 24, 512, 32)
    good = o4.w4a8_linear(a, c, s, sa, 32, bias)
    # zero point dropped: q instead of q - z
    p = o4.pack_int4_ref((np.random.default_rng(11).standard_normal((24, 512)) * 0.01).astype(np.float32),
                         group_size=32, symmetric=False)
    assert (p["zeros"] != 0).any()
    c2 = o4.unpack_int4_ref(p, floating=False)
    q = c2 + np.repeat(p["zeros"], 32, axis=1)
    assert not np.array_equal(o4.w4a8_linear(a, q, p["scales"], sa, 32, bias),
                              o4.w4a8_linear(a, c2, p["scales"], sa, 32, bias))
    # row scale inside the group loop
    a64, c64 = a.astype(np.float64), c.astype(np.float64)
    t1 = np.zeros((16, 24), np.float32)
    t2 = np.zeros((16, 24), np.float32)
    t3 = np.zeros((16, 24), np.float32)
    for gi in range(16):
        sl = slice(gi * 32, gi * 32 + 32)
        acc = (a64[:, sl] @ c64[:, sl].T).astype(np.float32)
        t1 = (t1 + ((acc * s[:, gi][None, :]).astype(np.float32) * sa[:, None]).astype(np.float32)).astype(np.float32)
        t3 = (acc.astype(np.float64) * s[:, gi][None, :].astype(np.float64) + t3.astype(np.float64)).astype(np.float32)
    for gi in reversed(range(16)):
        sl = slice(gi * 32, gi * 32 + 32)
        acc = (a64[:, sl] @ c64[:, sl].T).astype(np.float32)
        t2 = (t2 + (acc * s[:, gi][None, :]).astype(np.float32)).astype(np.float32)
    assert not np.array_equal((t1 + bias[None, :]).astype(np.float32), good)
    assert not np.array_equal(((t2 * sa[:, None]).astype(np.float32) + bias[None, :]).astype(np.float32), good)
    assert not np.array_equal(((t3 * sa[:, None]).astype(np.float32) + bias[None, :]).astype(np.float32), good)
