"""Pins of the INT8 oracle (CPU only).

Each check is chosen so that a plausible mistake in oracle/int8.py (a
transposed operand, a dropped bias, half-away instead of half-even, float64
instead of fp32 arithmetic, FMA instead of separate rounding) fails one of
them; none of them restates the oracle's own formula.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import int8 as o

GOLDEN = __import__("pathlib").Path(__file__).parent / "golden"


def test_int8_matmul_bruteforce_nonsquare():
    rng = np.random.default_rng(1)
    a = rng.integers(-128, 128, (5, 7), dtype=np.int8)
    b = rng.integers(-128, 128, (7, 9), dtype=np.int8)
    assert np.array_equal(o.int8_matmul(a, b), o.int8_matmul_bruteforce(a, b))


def test_int8_matmul_matches_torch_int_mm():
    g = torch.Generator().manual_seed(3)
    a = torch.randint(-128, 128, (64, 200), generator=g, dtype=torch.int8)
    b = torch.randint(-128, 128, (200, 48), generator=g, dtype=torch.int8)
    assert np.array_equal(o.int8_matmul(a.numpy(), b.numpy()), torch._int_mm(a, b).numpy())


def test_int8_matmul_closed_forms():
    # identity picks the other operand
    b = np.arange(-64, 64, dtype=np.int8).reshape(16, 8)
    assert np.array_equal(o.int8_matmul(np.eye(16, dtype=np.int8), b), b.astype(np.int32))
    # the int32 bound of int8_gemm.py:142-143: K = 131071 rows of -128 * -128
    k = 131071
    a = np.full((1, k), -128, dtype=np.int8)
    acc = o.int8_matmul(a, np.full((k, 1), -128, dtype=np.int8))
    assert acc[0, 0] == 131071 * 16384 == 2147467264
    with pytest.raises(ValueError):
        o.int8_matmul(np.zeros((1, k + 1), np.int8), np.zeros((k + 1, 1), np.int8))


def test_epilogue_hand_values():
    acc = np.array([[3, -8]], dtype=np.int32)
    out = o.epilogue_f(acc, [0.5], [0.25, 0.5], [1.0, -1.0])
    assert out.tolist() == [[1.375, -3.0]]
    assert o.epilogue_f(acc, [0.5], [0.25, 0.5], None).tolist() == [[0.375, -2.0]]
    # scalar weight scale broadcasts
    assert o.epilogue_f(acc, [2.0], [0.25], None).tolist() == [[1.5, -4.0]]


def test_epilogue_separate_vs_fused_rounding():
    # acc * scale = (2^23 + 1)(1 + 2^-23) = 2^23 + 2 + 2^-23: fp32 rounds the
    # product to 2^23 + 2, so the separate order returns exactly 0 while the
    # single-rounding FMA keeps 2^-23 (int8_gemm.py:191).
    acc = np.array([[2 ** 23 + 1]], dtype=np.int32)
    scale = np.float32(1 + 2 ** -23)
    bias = np.array([-(2.0 ** 23 + 2)], np.float32)
    assert o.epilogue_f(acc, [scale], [1.0], bias)[0, 0] == 0.0
    assert o.epilogue_f(acc, [scale], [1.0], bias, fused=True)[0, 0] == np.float32(2 ** -23)


def test_fma_emulation_against_exact_rationals():
    rng = np.random.default_rng(5)
    a = rng.standard_normal(4000).astype(np.float32) * 1e3
    b = rng.standard_normal(4000).astype(np.float32)
    c = -(a.astype(np.float64) * b).astype(np.float32)  # heavy cancellation
    c[::3] = rng.standard_normal(c[::3].size).astype(np.float32)
    got = o.fma_f32(a, b, c)
    for i in range(0, 4000, 7):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        # correctly rounded fp32 of the exact rational, ties to even
        lo = np.float32(float(exact))
        cand = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
        best = min(cand, key=lambda v: (abs(Fraction(float(v)) - exact),
                                        int(np.array(v, np.float32).view(np.uint32)) & 1))
        assert got[i] == best, i


def test_epilogue_order_e_differs_from_f_in_fp16():
    # order E rounds acc*scale to fp16 before adding the fp16-rounded bias
    acc = np.array([[1]], dtype=np.int32)
    e = o.epilogue_e(acc, [1.0], [1.0004883], [0.0004883], out="f16")
    f = o.epilogue_f(acc, [1.0], [1.0004883], [0.0004883], out="f16")
    assert e[0, 0] != f[0, 0]


def test_bf16_rounding_matches_torch():
    x = torch.randn(100000) * 3
    x[:4] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 65504.0])
    bits = o.f32_to_bf16_bits(x.numpy())
    assert np.array_equal(bits, x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


def test_quant_ties_and_rounding_rules():
    x = np.array([[127.0, -2.5, 2.5, 0.5, -0.5, 1.5, 126.5, -126.5]], np.float32)
    q_even, step = o.quant_rows(x, "half_even")
    q_away, _ = o.quant_rows(x, "half_away")
    assert step.tolist() == [1.0]
    assert q_even.tolist() == [[127, -2, 2, 0, 0, 2, 126, -126]]
    assert q_away.tolist() == [[127, -3, 3, 1, -1, 2, 127, -127]]


def test_quant_half_away_uses_fp32_add():
    # z = 0.49999997: z + 0.5 rounds to 1.0 in fp32, so the reference's
    # floor(z + 0.5) (fp8_weight_gemm_v06.py:89) yields 1, not 0.
    x = np.array([[127.0, 0.49999997]], np.float32)
    assert o.quant_rows(x, "half_away")[0][0, 1] == 1
    assert o.quant_rows(x, "half_even")[0][0, 1] == 0


def test_quant_zero_row_and_clamp():
    q, step = o.quant_rows(np.zeros((1, 5), np.float32))
    assert step[0] == np.float32(1e-20) and not q.any()
    # |x| / step can exceed 127 by rounding of step; the clamp keeps 127
    q, _ = o.quant_rows(np.array([[1.0, -1.0, 0.3]], np.float32))
    assert q[0, :2].tolist() == [127, -127]


def test_quant_matches_torch_division_and_round():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(64, 3072, generator=g).to(torch.float16).float()
    q, step = o.quant_rows(x.numpy())
    st = torch.clamp(x.abs().amax(1) / 127.0, min=1e-20)
    assert np.array_equal(step, st.numpy())
    assert np.array_equal(q, torch.round(x / st[:, None]).clamp(-127, 127).to(torch.int8).numpy())


def test_gelu_tanh_close_to_torch():
    x = torch.randn(200000) * 4
    ref = torch.nn.functional.gelu(x, approximate="tanh").numpy()
    assert np.abs(o.gelu_tanh(x.numpy()) - ref).max() <= 1e-6


@pytest.mark.parametrize("name", ["int8_small", "int8_layout", "quant_small"])
def test_golden_fixtures_reproduce(name):
    d = np.load(GOLDEN / f"{name}.npz")
    if name == "int8_small":
        a = d["a_store"][1:38, 1:80]
        acc = o.int8_matmul(a, np.ascontiguousarray(d["w"].T))
        assert np.array_equal(acc, d["acc"])
        for label, sb in (("vec", d["sb"]), ("scalar", d["sb1"])):
            f32 = o.epilogue_f(acc, d["sa"], sb, d["bias"])
            assert np.array_equal(f32.view(np.uint32), d[f"f32_{label}"].view(np.uint32))
            assert np.array_equal(o.encode(f32, "f16"), d[f"f16_{label}"])
    elif name == "int8_layout":
        assert np.array_equal(o.int8_matmul(d["a"], np.ascontiguousarray(d["w"].T)), d["acc"])
    else:
        q, step = o.quant_rows(d["x_f32"], "half_even")
        assert np.array_equal(q, d["q_f32_half_even"]) and np.array_equal(step, d["step_f32_half_even"])
