"""GPU parity of the opt-in MOSS steps: the ConvRot prologue and the residual epilogue.

The gfx950 rotation runs the fast Walsh-Hadamard butterflies in fp32, the order
oracle/convrot.py's rotate_fwht32 restates: codes and steps are bit-exact
against it. Against Kitchen's arithmetic (a dense fp32 product with H / 16 on
the GPU) the codes differ by at most one, on at most 0.1 % of the elements
(near-ties), and the steps by at most 2^-18 relative. The residual epilogue is
bit-exact against oracle.convrot.epilogue_f_residual on small grids and, at the
MOSS shape, against the library's own plain linear plus the residual added by
torch in fp32 (the fused value is rounded once).
"""
import numpy as np
import pytest
import torch

from conftest import case
from oracle import convrot as cr
from oracle import int8 as o8

pytestmark = pytest.mark.gpu

FLOATS = (torch.float32, torch.float16, torch.bfloat16)
OUT_NAME = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def bits(t):
    t = t.detach().cpu()
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    return t.view(torch.int16).numpy()


def _rows(shape, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * 2
    x[torch.rand(*shape, generator=g) < 0.002] *= 25
    if shape[0] > 2:
        x[1] = 0  # a zero row: step 1e-20, all codes 0
    return x


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("g,shape", [(256, (1061, 3072)), (2, (5, 6)), (4, (33, 12)), (16, (7, 112)),
                                     (128, (3, 4096)), (1024, (9, 16384)), (256, (1, 256)), (512, (17, 1536)),
                                     (8, (5, 512)), (16, (9, 2048)), (64, (2, 12288)), (32, (3, 16384))])
def test_rot_quant_rows_bit_exact(cuda, dtype, g, shape):
    from rdna2_ops.quantize import rotate_quantize_int8_rowwise
    case(f"rot quant {dtype} g{g} {shape}")
    x = _rows(shape, g * 31 + shape[1]).to(dtype)
    q, step = rotate_quantize_int8_rowwise(x.to(cuda), g)
    qo, so = cr.rot_quant_rows(x.float().numpy(), g)
    assert np.array_equal(step.cpu().numpy().reshape(-1), so)
    assert np.array_equal(q.cpu().numpy(), qo)


def test_rot_quant_rows_half_away_and_row_stride(cuda):
    from rdna2_ops.quantize import rotate_quantize_int8_rowwise
    case("rot quant half_away, row stride 4160")
    wide = _rows((64, 4160), 5).to(cuda)
    x = wide[:, :4096]
    assert x.stride(0) == 4160
    q, step = rotate_quantize_int8_rowwise(x, 256, rounding="half_away")
    qo, so = cr.rot_quant_rows(x.cpu().numpy(), 256, "half_away")
    assert np.array_equal(step.cpu().numpy().reshape(-1), so)
    assert np.array_equal(q.cpu().numpy(), qo)
    # exact ties: small integers rotate exactly; half_even and half_away then differ only at ties
    xi = torch.randint(-40, 40, (16, 1024), generator=torch.Generator().manual_seed(2)).float()
    for rounding in ("half_even", "half_away"):
        q, step = rotate_quantize_int8_rowwise(xi.to(cuda), 256, rounding=rounding)
        qo, so = cr.rot_quant_rows(xi.numpy(), 256, rounding)
        assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(step.cpu().numpy().reshape(-1), so)


def test_rot_quant_rows_against_kitchen_dense_rotation(cuda):
    """Kitchen's rotation is a dense fp32 product (comfy_int8.py:117-118)."""
    from rdna2_ops.quantize import quantize_int8_rowwise, rotate_quantize_int8_rowwise
    case("rot quant vs dense fp32 rotation on the GPU")
    x = _rows((1061, 3072), 77).to(cuda)
    h = torch.from_numpy(cr.hadamard(256) / 16.0).float().to(cuda)
    dense = (x.reshape(1061, 12, 256) @ h).reshape(1061, 3072)
    qd, sd = quantize_int8_rowwise(dense)
    qf, sf = rotate_quantize_int8_rowwise(x, 256)
    assert torch.all((sd - sf).abs() <= 2.0 ** -18 * sd)
    diff = (qd.int() - qf.int()).abs()
    assert int(diff.max()) <= 1
    assert int(diff.count_nonzero()) <= 1e-3 * diff.numel()


def _weights(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    ws = torch.rand(n, generator=g) * 1e-3 + 1e-4
    bias = torch.randn(n, generator=g)
    return w, ws, bias


@pytest.mark.parametrize("out", FLOATS)
@pytest.mark.parametrize("xdt", FLOATS)
def test_w8a8_linear_convrot_bit_exact(cuda, out, xdt):
    from rdna2_ops.int8_gemm import w8a8_linear
    case(f"w8a8 convrot x={xdt} out={out}")
    m, n, k = 37, 200, 1024
    x = _rows((m, k), 3).to(xdt)
    w, ws, bias = _weights(n, k, 4)
    y = w8a8_linear(x.to(cuda), w.to(cuda), ws.to(cuda), bias.to(cuda), out_dtype=out, convrot_groupsize=256)
    yo, _, _, _ = cr.moss_linear(x.float().numpy(), w.numpy(), ws.numpy(), bias.numpy(), g=256,
                                 out=OUT_NAME[out])
    assert np.array_equal(bits(y), bits(torch.from_numpy(yo).to(out)))


@pytest.mark.parametrize("out", FLOATS)
@pytest.mark.parametrize("rdt", FLOATS)
@pytest.mark.parametrize("scale_kind", ["none", "scalar", "channel"])
def test_w8a8_linear_residual_bit_exact_small(cuda, out, rdt, scale_kind):
    from rdna2_ops.int8_gemm import w8a8_linear
    case(f"w8a8 residual out={out} residual={rdt} scale={scale_kind}")
    m, n, k = 45, 136, 512
    x = _rows((m, k), 8)
    w, ws, bias = _weights(n, k, 9)
    gen = torch.Generator().manual_seed(10)
    res = (torch.randn(m, n, generator=gen) * 3).to(rdt)
    rs = {"none": None, "scalar": torch.tensor([0.75]), "channel": torch.rand(n, generator=gen)}[scale_kind]
    for with_bias, g in ((True, None), (False, 128)):
        y = w8a8_linear(x.to(cuda), w.to(cuda), ws.to(cuda), bias.to(cuda) if with_bias else None, out_dtype=out,
                        convrot_groupsize=g, residual=res.to(cuda),
                        residual_scale=None if rs is None else rs.to(cuda))
        yo, _, _, _ = cr.moss_linear(x.numpy(), w.numpy(), ws.numpy(), bias.numpy() if with_bias else None, g=g,
                                     residual=res.float().numpy(), residual_scale=None if rs is None else rs.numpy(),
                                     out=OUT_NAME[out])
        assert np.array_equal(bits(y), bits(torch.from_numpy(yo).to(out))), (with_bias, g)


@pytest.mark.parametrize("out", FLOATS)
def test_w8a8_linear_residual_moss_shape(cuda, out):
    """MOSS shape [1, 1061, 3072] x [3072, 3072] with ConvRot g256 and a per-channel
    residual scale: the fused output is the plain linear's fp32 value plus the
    residual term, rounded once."""
    from rdna2_ops.int8_gemm import w8a8_linear
    case(f"w8a8 residual MOSS shape out={out}")
    m, n, k = 1061, 3072, 3072
    x = _rows((m, k), 12).reshape(1, m, k).to(cuda)
    w, ws, bias = (t.to(cuda) for t in _weights(n, k, 13))
    gen = torch.Generator().manual_seed(14)
    res = torch.randn(1, m, n, generator=gen).to(cuda)
    rs = torch.rand(n, generator=gen).to(cuda)
    plain = w8a8_linear(x, w, ws, bias, out_dtype=torch.float32, convrot_groupsize=256)
    fused = w8a8_linear(x, w, ws, bias, out_dtype=out, convrot_groupsize=256, residual=res, residual_scale=rs)
    want = (plain + res * rs).to(out)
    assert fused.shape == (1, m, n)
    assert torch.equal(fused.view(torch.int16) if out != torch.float32 else fused.view(torch.int32),
                       want.view(torch.int16) if out != torch.float32 else want.view(torch.int32))
    # GELU epilogue then the residual
    plain_g = w8a8_linear(x, w, ws, bias, out_dtype=torch.float32, activation="gelu_tanh")
    fused_g = w8a8_linear(x, w, ws, bias, out_dtype=torch.float32, activation="gelu_tanh", residual=res)
    assert torch.equal(fused_g, plain_g + res)


@pytest.mark.parametrize("m,n,k,pad", [(1061, 9216, 3072, 0), (1100, 9002, 256, 3)])
def test_w8a8_linear_residual_pingpong_grid(cuda, m, n, k, pad):
    """Grids of >= 192 tiles of 256 x 192 run the residual epilogue on the
    persistent ping-pong kernel: for every output / residual dtype and scale
    kind the fused output equals the plain linear's fp32 value plus
    f32(residual) (x scale), rounded once — including a ragged N (edge tiles)
    and a residual row stride that is not a multiple of 4 (unaligned rows:
    element-wise residual loads)."""
    from rdna2_ops.int8_gemm import w8a8_linear
    x = _rows((m, k), 15).to(cuda)
    w, ws, bias = (t.to(cuda) for t in _weights(n, k, 16))
    gen = torch.Generator().manual_seed(17)
    plain = w8a8_linear(x, w, ws, bias, out_dtype=torch.float32)
    for rdt in FLOATS:
        base = (torch.randn(m, n + pad, generator=gen) * 2).to(rdt).to(cuda)
        res = base[:, :n]
        for scale_kind in ("none", "scalar", "channel"):
            rs = {"none": None, "scalar": torch.tensor([0.75], device=cuda),
                  "channel": (torch.rand(n, generator=gen) + 0.25).to(cuda)}[scale_kind]
            term = res.float() if rs is None else res.float() * rs
            for out in FLOATS:
                case(f"w8a8 residual ping-pong {m}x{n}x{k} res={rdt} scale={scale_kind} out={out}")
                fused = w8a8_linear(x, w, ws, bias, out_dtype=out, residual=res, residual_scale=rs)
                want = (plain + term).to(out)
                assert np.array_equal(bits(fused), bits(want)), (rdt, scale_kind, out)


def test_w8a8_linear_convrot_end_to_end_against_dense(cuda):
    """End to end at the MOSS shape: a rotated weight, then the fused linear
    against the exact fp64 product of the unrotated operands (ConvRot is exact
    in real arithmetic), and against Kitchen's dense-rotation pipeline."""
    from rdna2_ops.int8_gemm import w8a8_linear
    from rdna2_ops.quantize import quantize_int8_rowwise
    case("w8a8 convrot end to end")
    m, n, k = 1061, 3072, 3072
    gen = torch.Generator().manual_seed(15)
    x = torch.randn(m, k, generator=gen)
    w = torch.randn(n, k, generator=gen) * 0.02
    h = torch.from_numpy(cr.hadamard(256) / 16.0).float()
    w_rot = (w.reshape(n, -1, 256) @ h).reshape(n, k)
    wq, wstep = quantize_int8_rowwise(w_rot.to(cuda))
    y = w8a8_linear(x.to(cuda), wq, wstep.reshape(-1), out_dtype=torch.float32, convrot_groupsize=256)
    exact = (x.double() @ w.double().T).to(cuda)
    assert float((y.double() - exact).norm() / exact.norm()) < 0.02
    # Kitchen's order with the dense rotation: rotation -> quantizer -> product -> scale
    xr = (x.to(cuda).reshape(m, -1, 256) @ h.to(cuda)).reshape(m, k)
    y_dense = w8a8_linear(xr, wq, wstep.reshape(-1), out_dtype=torch.float32)
    assert float((y - y_dense).norm() / y_dense.norm()) < 1e-3


def test_w8a8_linear_ex_argument_errors(cuda):
    from rdna2_ops.int8_gemm import w8a8_linear
    case("w8a8 ex argument errors")
    x = torch.randn(4, 512, device=cuda)
    w = torch.zeros(64, 512, dtype=torch.int8, device=cuda)
    s = torch.ones(64, device=cuda)
    res = torch.zeros(4, 64, device=cuda)
    for g in (3, 96, 2048, 384):
        with pytest.raises(ValueError):
            w8a8_linear(x, w, s, convrot_groupsize=g)
    with pytest.raises(ValueError):
        w8a8_linear(x, w, s, residual=res, epilogue_order="eager")
    with pytest.raises(ValueError):
        w8a8_linear(x, w, s, residual=res[:, :32])
    with pytest.raises(ValueError):
        w8a8_linear(x, w, s, residual_scale=torch.ones(1, device=cuda))
    with pytest.raises(ValueError):
        w8a8_linear(x, w, s, residual=res, residual_scale=torch.ones(7, device=cuda))
