"""W4A8 GPU parity (int4_linear_a8, int4_weight_gemm_v07.py:476-537): every
method, integer and float results bit-identical to oracle/int4.w4a8_integer /
w4a8_linear (the reference's own bar: byte-equal to grouped_integer_reference,
bench_int4_v07.py:149-171), over group sizes, symmetric / affine packing,
both word layouts and nibble orders, uint4 storage, prepared centred weights,
K not a multiple of 128, M / N tails and the reference's check shapes."""
import numpy as np
import pytest
import torch

from conftest import case
from oracle import int4 as o4

pytestmark = pytest.mark.gpu


def w4():
    from rdna2_ops import int4_weight_gemm_v07 as mod
    return mod


def _np(t):
    return t.detach().cpu().numpy()


def make(cuda, m, n, k, g, sym=False, layout="nk", order="low", seed=0, uint4=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.01).astype(np.float32)
    if uint4:
        p = w4().pack_uint4(torch.from_numpy(w).to(cuda), group_size=g)
        centred = _np(w4().unpack_int4(p, dtype=torch.int8)).astype(np.int32)
        r = o4.pack_uint4_baseline(w, group_size=g)
        assert np.array_equal(centred, o4.dequant_baseline(r, floating=False))
        scales = _np(p.scales.float())
    else:
        p = w4().pack_int4(torch.from_numpy(w).to(cuda), group_size=g, symmetric=sym, layout=layout, order=order)
        r = o4.pack_int4_ref(w, group_size=g, symmetric=sym, layout=layout, order=order)
        centred = o4.unpack_int4_ref(r, floating=False)
        scales = r["scales"]
    a = rng.integers(-128, 128, (m, k)).astype(np.int8)
    sa = (rng.random(m) * 0.02 + 0.001).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
    return p, centred, scales, a, sa, bias


def run(cuda, p, a, sa, bias=None, **kw):
    bt = None if bias is None else torch.from_numpy(bias).to(cuda)
    return w4().int4_linear_a8(torch.from_numpy(a).to(cuda), p, torch.from_numpy(sa).to(cuda), bias=bt, **kw)


def check(cuda, p, centred, scales, a, sa, bias, g, label, methods=("dot4", "dot8", "dot4_words", "dot4_split")):
    ref_i = o4.w4a8_integer(a, centred)
    ref_f = o4.w4a8_linear(a, centred, scales, sa, g, bias)
    ref_nb = o4.w4a8_linear(a, centred, scales, sa, g)
    for method in methods:
        yi = run(cuda, p, a, sa, method=method, integer=True)
        assert yi.dtype == torch.int32 and np.array_equal(_np(yi).astype(np.int64), ref_i), (label, method, "integer")
        yf = run(cuda, p, a, sa, bias, method=method)
        assert yf.dtype == torch.float32
        assert np.array_equal(_np(yf).view(np.uint32), ref_f.view(np.uint32)), (label, method, "float")
    y0 = run(cuda, p, a, sa, method=methods[0])
    assert np.array_equal(_np(y0).view(np.uint32), ref_nb.view(np.uint32)), (label, "no bias")


@pytest.mark.parametrize("g", o4.GROUPS)
@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("layout,order", [("nk", "low"), ("nk", "high"), ("kn", "low"), ("kn", "high")])
def test_w4a8_formats(cuda, g, sym, layout, order):
    case(f"w4a8 g{g} sym={sym} {layout} {order}")
    p, c, s, a, sa, bias = make(cuda, 40, 72, 2 * max(g, 128), g, sym, layout, order, seed=g + sym)
    check(cuda, p, c, s, a, sa, bias, g, f"g{g} {layout} {order}", methods=("dot4", "dot4_words"))


@pytest.mark.parametrize("m,n,k,g", [(37, 53, 384, 32), (129, 130, 256, 64), (1, 7, 96, 32), (65, 200, 192, 64),
                                     (300, 140, 320, 64), (5, 129, 640, 128), (33, 70, 352, 32), (17, 90, 160, 32)])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_w4a8_shapes_and_tails(cuda, m, n, k, g, layout):
    """Row / column tails, a single row, K = 96, 160, 192, 320, 352, 640 (last
    stage of 128 K filled by 1, 2 or 3 of its 4 k-steps, or whole): K a
    multiple of 128 takes the 16-column form (these grids are small), other K
    the 32-column guarded body (nk words as 16-byte loads, kn as 4-byte)."""
    case(f"w4a8 shape {m}x{n}x{k} g{g} {layout}")
    p, c, s, a, sa, bias = make(cuda, m, n, k, g, layout=layout, seed=m + n)
    check(cuda, p, c, s, a, sa, bias, g, f"{m}x{n}x{k}")


def test_w4a8_reference_check_shapes(cuda):
    """The reference's own check (bench_int4_v07.py:149-171): g32 affine, kn,
    low order, bias, methods dot4 / dot8 / dot4_words, byte-equal on every
    output, the 1061 x 3072 x 3072 case included."""
    for m, n, k in ((37, 53, 384), (19, 3072, 3072), (1061, 3072, 3072)):
        case(f"w4a8 reference check {m}x{n}x{k}")
        p, c, s, a, sa, bias = make(cuda, m, n, k, 32, layout="kn", seed=20261107)
        ref = o4.w4a8_linear(a, c, s, sa, 32, bias)
        for method in ("dot4", "dot8", "dot4_words"):
            y = _np(run(cuda, p, a, sa, bias, method=method))
            assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), (m, n, k, method)


def test_w4a8_prepared_and_uint4(cuda):
    """dot4_prepared with the centred INT8 weights of unpack_int4; benchmark
    uint4 storage (bf16 scales, packed uint4 zero points)."""
    case("w4a8 prepared and uint4")
    p, c, s, a, sa, bias = make(cuda, 96, 160, 512, 64, seed=5)
    prep = w4().unpack_int4(p, dtype=torch.int8)
    for integer in (True, False):
        y = run(cuda, p, a, sa, None if integer else bias, method="dot4_prepared", prepared=prep, integer=integer)
        ref = o4.w4a8_integer(a, c) if integer else o4.w4a8_linear(a, c, s, sa, 64, bias)
        if integer:
            assert np.array_equal(_np(y).astype(np.int64), ref)
        else:
            assert np.array_equal(_np(y).view(np.uint32), ref.view(np.uint32))
    p, c, s, a, sa, bias = make(cuda, 70, 96, 1024, 128, uint4=True, seed=6)
    check(cuda, p, c, s, a, sa, bias, 128, "uint4", methods=("dot4",))


def test_w4a8_bias_dtypes_and_strided_activation(cuda):
    case("w4a8 bias dtypes, strided A")
    p, c, s, a, sa, bias = make(cuda, 50, 64, 256, 32, seed=8)
    for dt in (torch.float16, torch.bfloat16, torch.float64):
        bt = torch.from_numpy(bias).to(dt)
        y = w4().int4_linear_a8(torch.from_numpy(a).to(cuda), p, torch.from_numpy(sa).to(cuda), bias=bt.to(cuda))
        ref = o4.w4a8_linear(a, c, s, sa, 32, bt.to(torch.float32).numpy())
        assert np.array_equal(_np(y).view(np.uint32), ref.view(np.uint32)), dt
    wide = torch.zeros(50, 256 + 48, dtype=torch.int8)
    wide[:, 16:16 + 256] = torch.from_numpy(a)
    av = wide.to(cuda)[:, 16:16 + 256]  # row stride 304, base offset 16
    y = w4().int4_linear_a8(av, p, torch.from_numpy(sa).to(cuda).reshape(-1, 1))
    assert np.array_equal(_np(y).view(np.uint32), o4.w4a8_linear(a, c, s, sa, 32).view(np.uint32))


def test_w4a8_extreme_values(cuda):
    """a = -128 everywhere against the extreme codes; K = 12288 with g32."""
    case("w4a8 extreme values K=12288")
    p, c, s, a, sa, bias = make(cuda, 16, 96, 12288, 32, seed=9)
    a[:] = -128
    a[3, ::2] = 127
    ref_i = o4.w4a8_integer(a, c)
    y = run(cuda, p, a, sa, method="dot4", integer=True)
    assert np.array_equal(_np(y).astype(np.int64), ref_i)
    yf = run(cuda, p, a, sa, bias)
    assert np.array_equal(_np(yf).view(np.uint32), o4.w4a8_linear(a, c, s, sa, 32, bias).view(np.uint32))


@pytest.mark.parametrize("m,n,k,g,layout,form", [
    (300, 2100, 256, 128, "nk", "k_w4a8_n16"),   # 51 tiles: 16-column waves
    (1100, 2200, 256, 32, "kn", "k_w4a8_n16"),   # 162 tiles at g32: 16-column waves
    (2048, 1152, 256, 128, "nk", "6k_w4a8I"),    # 144 tiles: 32-column waves, full-K body
    (1100, 2200, 384, 64, "kn", "6k_w4a8I"),     # 162 tiles at g64: 32-column waves, full-K body
    (1100, 2200, 320, 64, "nk", "6k_w4a8I"),     # K not a multiple of 128: guarded body
])
def test_w4a8_kernel_forms(cuda, m, n, k, g, layout, form):
    """Every kernel form the library chooses by grid size, group and K,
    byte-equal to the oracle (integer and float, ragged M and N)."""
    case(f"w4a8 form {form} {m}x{n}x{k} g{g} {layout}")
    p, c, s, a, sa, bias = make(cuda, m, n, k, g, layout=layout, seed=m + n + k)
    y, meta = run(cuda, p, a, sa, bias, return_kernel=True)
    assert form in (meta["symbol"] or ""), meta
    assert np.array_equal(_np(y).view(np.uint32), o4.w4a8_linear(a, c, s, sa, g, bias).view(np.uint32))
    yi = run(cuda, p, a, sa, integer=True)
    assert np.array_equal(_np(yi).astype(np.int64), o4.w4a8_integer(a, c))


def test_w4a8_random_shapes(cuda):
    """24 seeded random cases over M, N, K (K a multiple of 128 or not), group
    size, word layout, nibble order and symmetric / affine packing: integer
    and float outputs byte-equal to the oracle, whichever form the grid takes."""
    rng = np.random.default_rng(20261202)
    for i in range(24):
        g = int(rng.choice(o4.GROUPS))
        k = g * int(rng.integers(1, 1536 // g + 1))
        m, n = int(rng.integers(1, 700)), int(rng.integers(1, 900))
        layout = str(rng.choice(["nk", "kn"]))
        order = str(rng.choice(["low", "high"]))
        sym = bool(rng.integers(0, 2))
        case(f"w4a8 random {i}: {m}x{n}x{k} g{g} {layout} {order} sym={sym}")
        p, c, s, a, sa, bias = make(cuda, m, n, k, g, sym, layout, order, seed=1000 + i)
        yf = run(cuda, p, a, sa, bias)
        assert np.array_equal(_np(yf).view(np.uint32), o4.w4a8_linear(a, c, s, sa, g, bias).view(np.uint32)), i
        yi = run(cuda, p, a, sa, integer=True)
        assert np.array_equal(_np(yi).astype(np.int64), o4.w4a8_integer(a, c)), i


def test_w4a8_argument_checks(cuda):
    case("w4a8 argument checks")
    p, c, s, a, sa, bias = make(cuda, 8, 64, 256, 32)
    at, sat = torch.from_numpy(a).to(cuda), torch.from_numpy(sa).to(cuda)
    with pytest.raises(ValueError, match="Matching A8"):
        w4().int4_linear_a8(at.float(), p, sat)
    with pytest.raises(ValueError, match="per-activation-row scale"):
        w4().int4_linear_a8(at, p, sat.double())
    with pytest.raises(ValueError, match="Floating bias"):
        w4().int4_linear_a8(at, p, sat, bias=torch.zeros(64, dtype=torch.int32, device=cuda))
    with pytest.raises(ValueError, match="tile"):
        w4().int4_linear_a8(at, p, sat, tile=(48, 64))
    with pytest.raises(ValueError, match=">=16"):
        w4().int4_linear_a8(at, p, sat, tile=(8, 64))
    with pytest.raises(ValueError, match="Centered INT8"):
        w4().int4_linear_a8(at, p, sat, method="dot4_prepared")
    with pytest.raises(ValueError, match="Dot8 prepared tuple"):
        w4().int4_linear_a8(at, p, sat, method="dot8", prepared=[1, 2, 3])
    with pytest.raises(ValueError):
        w4().int4_linear_a8(at, p, sat, method="nope")
    lo, hi, sums = w4().prepare_dot8_activation(at, p)
    assert lo.shape == (8, 32) and hi.shape == (8, 32) and sums.shape == (8, 8)
    assert np.array_equal(_np(sums), a.astype(np.int64).reshape(8, 8, 32).sum(-1))
    y = w4().int4_linear_a8(at, p, sat, method="dot8", prepared=(lo, hi, sums))
    assert np.array_equal(_np(y).view(np.uint32), o4.w4a8_linear(a, c, s, sa, 32).view(np.uint32))
    h = w4().int8_activation_to_fp16(at, sat)
    assert h.dtype == torch.float16 and np.array_equal(_np(h), (a.astype(np.float32) * sa[:, None]).astype(np.float16))
