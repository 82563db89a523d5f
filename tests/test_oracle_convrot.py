"""Pins of the ConvRot / residual oracle (CPU only).

Each check is chosen so that a plausible mistake in oracle/convrot.py (a
missing or wrong normalisation, the butterfly's difference on the wrong side,
another row order of H such as Walsh / sequency order, the residual scale
applied to the product instead of the residual, the residual added after the
rounding) fails one of them; none of them restates the oracle's formula.
"""
import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import convrot as cr
from oracle import int8 as o8

GROUPS = (2, 4, 16, 128, 256, 1024)


@pytest.mark.parametrize("g", GROUPS)
def test_hadamard_is_sylvester_and_orthogonal(g):
    h = cr.hadamard(g)
    # Sylvester's recursion H_2g = [[H, H], [H, -H]], built independently
    ref = np.ones((1, 1))
    while ref.shape[0] < g:
        ref = np.block([[ref, ref], [ref, -ref]])
    assert np.array_equal(h, ref)
    assert np.array_equal(h, scipy.linalg.hadamard(g).astype(np.float64))
    assert np.array_equal(h @ h.T, g * np.eye(g))
    assert np.array_equal(h, h.T)


def test_hadamard_rejects_non_power_of_two():
    with pytest.raises(ValueError):
        cr.hadamard(12)


@pytest.mark.parametrize("g", (16, 256))
def test_dense_rotation_closed_forms(g):
    rng = np.random.default_rng(g)
    x = rng.standard_normal((3, 4 * g))
    r = cr.rotate_dense64(x, g)
    # orthonormal: Parseval per group, and the rotation is an involution
    assert np.allclose(np.linalg.norm(r.reshape(3, 4, g), axis=2), np.linalg.norm(x.reshape(3, 4, g), axis=2),
                       rtol=1e-13)
    assert np.allclose(cr.rotate_dense64(r, g), x, atol=1e-12)
    # unit vector e_j -> row j of H / sqrt(g); constant group -> sqrt(g) e_0
    e = np.zeros((1, g))
    e[0, 5] = 1.0
    assert np.array_equal(cr.rotate_dense64(e, g)[0] * np.sqrt(g), cr.hadamard(g)[5])
    ones = np.ones((1, g))
    want = np.zeros(g)
    want[0] = np.sqrt(g)
    assert np.allclose(cr.rotate_dense64(ones, g)[0], want, atol=1e-12)


@pytest.mark.parametrize("g", GROUPS)
def test_fwht32_agrees_with_exact_rotation(g):
    rng = np.random.default_rng(7 + g)
    x = (rng.standard_normal((5, 2 * g)) * np.array([[1e-3], [1.0], [30.0], [1.0], [1e4]])).astype(np.float32)
    got = cr.rotate_fwht32(x, g).astype(np.float64)
    exact = cr.rotate_dense64(x.astype(np.float64), g)
    # every butterfly stage rounds once: |error| <= log2(g) * 2^-24 * sum|x| / sqrt(g) (+ the final scale)
    bound = (np.log2(g) + 1) * 2.0 ** -24 * np.abs(x.reshape(5, 2, g)).sum(axis=2, keepdims=True) / np.sqrt(g)
    err = np.abs(got - exact).reshape(5, 2, g)
    assert np.all(err <= bound + 1e-30)


def test_fwht32_exact_special_cases():
    g = 256
    # 1 / sqrt(256) = 1/16 exactly: e_0 -> all 1/16, a constant group -> 16 e_0, bit for bit
    e0 = np.zeros((1, g), np.float32)
    e0[0, 0] = 1.0
    assert np.array_equal(cr.rotate_fwht32(e0, g), np.full((1, g), 1.0 / 16, np.float32))
    want = np.zeros((1, g), np.float32)
    want[0, 0] = 16.0
    assert np.array_equal(cr.rotate_fwht32(np.ones((1, g), np.float32), g), want)
    # small integers: every partial sum is exact, so the result equals the exact rotation
    rng = np.random.default_rng(3)
    xi = rng.integers(-50, 50, (4, 3 * g)).astype(np.float32)
    assert np.array_equal(cr.rotate_fwht32(xi, g).astype(np.float64), cr.rotate_dense64(xi, g))


def _fwht_planted(x, g, *, swap=False, normalise=True):
    """A deliberately wrong variant of the oracle's rotation (planted on the CPU)."""
    v = np.array(x, dtype=np.float32, copy=True)
    m, k = v.shape
    h = 1
    while h < g:
        b = v.reshape(m, k // (2 * h), 2, h)
        a, c = b[:, :, 0, :].copy(), b[:, :, 1, :].copy()
        b[:, :, 0, :] = a + c
        b[:, :, 1, :] = (c - a) if swap else (a - c)
        h *= 2
    return v / np.float32(np.sqrt(g)) if normalise else v


def test_planted_mistakes_are_caught():
    g = 16
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 2 * g)).astype(np.float32)
    exact = cr.rotate_dense64(x, g)
    assert np.allclose(_fwht_planted(x, g), exact, atol=1e-5)  # the faithful variant passes
    assert not np.allclose(_fwht_planted(x, g, swap=True), exact, atol=1e-3)
    assert not np.allclose(_fwht_planted(x, g, normalise=False), exact, atol=1e-3)
    # Walsh (sequency) order is another Hadamard matrix with the same rows permuted
    walsh = cr.hadamard(g)[np.argsort([bin(i ^ (i >> 1)).count("1") for i in range(g)], kind="stable")]
    assert not np.allclose(x.astype(np.float64).reshape(2, 2, g) @ walsh / 4.0, exact.reshape(2, 2, g), atol=1e-3)


def test_rotation_matches_torch_dense_fp32_up_to_ulps():
    """Kitchen's arithmetic, a dense fp32 product with H / sqrt(g), versus the
    butterfly order: the values agree to a few ulps and the codes to +-1 at
    near-ties only."""
    g = 256
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(64, 3072, generator=gen)
    h = torch.from_numpy(cr.hadamard(g) / 16.0).float()
    dense = (x.reshape(64, -1, g) @ h).reshape(64, 3072).numpy()
    fwht = cr.rotate_fwht32(x.numpy(), g)
    scale = np.abs(x.numpy().reshape(64, -1, g)).sum(axis=2, keepdims=True) / 16.0
    assert np.all(np.abs(dense - fwht).reshape(64, -1, g) <= 16 * 2.0 ** -24 * scale)
    qd, sd = o8.quant_rows(dense)
    qf, sf = o8.quant_rows(fwht)
    # the steps inherit the rotated absmax's few-ulp difference (measured <= 8 ulps here)
    assert np.all(np.abs(sd - sf) <= 2.0 ** -18 * sd)
    diff = qd.astype(np.int32) - qf.astype(np.int32)
    assert np.abs(diff).max() <= 1
    assert np.count_nonzero(diff) <= 1e-3 * diff.size


def test_residual_epilogue_hand_values():
    acc = np.array([[3, -2]], np.int32)
    sa = np.array([0.5], np.float32)
    sb = np.array([2.0, 4.0], np.float32)
    bias = np.array([1.0, -1.0], np.float32)
    res = np.array([[0.25, 8.0]], np.float32)
    # 3*1 + 1 + 0.25*4 = 5 ; -2*2 - 1 + 8*0.5 = -1
    got = cr.epilogue_f_residual(acc, sa, sb, bias, res, np.array([4.0, 0.5], np.float32))
    assert np.array_equal(got, np.array([[5.0, -1.0]], np.float32))
    # scalar scale, and no scale
    assert np.array_equal(cr.epilogue_f_residual(acc, sa, sb, bias, res, np.float32(2.0)), [[4.5, 11.0]])
    assert np.array_equal(cr.epilogue_f_residual(acc, sa, sb, bias, res), [[4.25, 3.0]])


def test_residual_epilogue_matches_torch_kitchen_order():
    """fp32 out: torch CPU fp32 ops in Kitchen's order, scale -> + bias -> + residual * scale."""
    gen = torch.Generator().manual_seed(9)
    acc = torch.randint(-2 ** 20, 2 ** 20, (33, 47), generator=gen, dtype=torch.int32)
    sa = torch.rand(33, 1, generator=gen) * 1e-3
    sw = torch.rand(47, generator=gen) * 1e-2
    bias = torch.randn(47, generator=gen)
    res = torch.randn(33, 47, generator=gen)
    rscale = torch.rand(47, generator=gen)
    want = acc.float() * (sa * sw.reshape(1, -1))
    want = want + bias.reshape(1, -1)
    want = want + res * rscale
    got = cr.epilogue_f_residual(acc.numpy(), sa.numpy(), sw.numpy(), bias.numpy(), res.numpy(), rscale.numpy())
    assert np.array_equal(got, want.numpy())
    # fp16 / bf16 out: one rounding of the fp32 value (not the rounded sum of rounded parts)
    for out, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        got = cr.epilogue_f_residual(acc.numpy(), sa.numpy(), sw.numpy(), bias.numpy(), res.numpy(),
                                     rscale.numpy(), out=out)
        assert np.array_equal(got, want.to(dt).float().numpy())


def test_convrot_invariance_of_the_linear():
    """ConvRot is exact in real arithmetic: with the weight rotated by the same
    H, Q(xH) (WH)^T approximates x W^T to the quantizers' error."""
    g = 256
    rng = np.random.default_rng(21)
    x = rng.standard_normal((8, 1024)).astype(np.float32)
    w = (rng.standard_normal((96, 1024)) * 0.02).astype(np.float32)
    w_rot = cr.rotate_fwht32(w, g)
    wq, ws = o8.quant_rows(w_rot)
    y, _, _, _ = cr.moss_linear(x, wq, ws, g=g)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    rel = np.linalg.norm(y - exact) / np.linalg.norm(exact)
    assert rel < 0.02
    # without the activation rotation the product is wrong (the weight alone is rotated)
    y_bad, _, _, _ = cr.moss_linear(x, wq, ws, g=None)
    assert np.linalg.norm(y_bad - exact) / np.linalg.norm(exact) > 0.5
