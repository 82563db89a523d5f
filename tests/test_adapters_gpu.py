"""The research adapters and Triton knobs of rdna2-ops/rdna2_ops/int8_gemm.py on
the GPU:

* ``wrapped=True`` and ``partial_dot=True`` (the wrapped-load variant and its
  acc += dot form, int8_gemm.py:70-123) give bits identical to the default and
  to the oracle, on the 4-wave 128x128 grid and on the persistent 256x192
  ping-pong grid, with ragged M and N, for the int32 and fp32 epilogues;
* ``moss_int8_gemm_candidate`` (int8_gemm.py:217-271), run through the Kitchen
  test double, is bit-identical to the double's eager int8_linear for fp32 in
  and out — per-channel and scalar weight scales, ConvRot, bias, residual —
  and counts hits, shapes and precision fallbacks;
* ``qwen_int8_gemm_candidate`` (int8_gemm.py:274-330), run on a patientx bridge
  test double found by its source path, is bit-identical to the oracle's
  rounding="fused" epilogue (one FMA of f32(acc), sa * sw and bias) for the
  per-row, tensor-scale and number-scale wrappers, and restores both wrappers.
"""
import importlib
import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import case
from oracle import int8 as o

pytestmark = pytest.mark.gpu
HERE = Path(__file__).resolve().parent
KITCHEN = str(HERE / "kitchen_stub")
BRIDGE = HERE / "patientx_stub" / "RDNA2-Qwen21-INT8" / "rocm_int8_kitchen_patch.py"


def _operands(m, n, k, seed, dev):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sa = torch.rand(m, generator=g) * 1e-2 + 1e-4
    sb = torch.rand(n, generator=g) * 1e-2 + 1e-4
    bias = torch.randn(n, generator=g)
    return a, w, sa, sb, bias, [t.to(dev) for t in (a, w, sa, sb, bias)]


# 4-wave grid (fewer than 192 tiles of 256x192) and the persistent ping-pong
# grid (8 x 25 = 200 tiles), both with ragged M and N
@pytest.mark.parametrize("m,n,k", [(333, 517, 384), (2000, 4700, 512)])
def test_wrapped_and_partial_dot_same_bits(cuda, m, n, k):
    from rdna2_ops.int8_gemm import int8_gemm_dequant, int8_matmul
    a, w, sa, sb, bias, (da, dw, dsa, dsb, dbias) = _operands(m, n, k, 11, cuda)
    acc = o.int8_matmul(a.numpy(), np.ascontiguousarray(w.numpy().T))
    exp_f = o.epilogue_f(acc, sa.numpy(), sb.numpy(), bias.numpy())
    for wrapped, partial in ((False, False), (True, False), (True, True)):
        case(f"int8 knobs wrapped={wrapped} partial_dot={partial} {m}x{n}x{k}")
        got_i, meta = int8_matmul(da, dw.T, wrapped=wrapped, partial_dot=partial, return_kernel=True)
        assert meta["requested_wrapped"] == wrapped and meta["requested_partial_dot"] == partial
        assert np.array_equal(got_i.cpu().numpy(), acc)
        got_f = int8_gemm_dequant(da, dw.T, dsa, dsb, dbias, wrapped=wrapped, partial_dot=partial)
        assert np.array_equal(got_f.cpu().numpy().view(np.uint32), exp_f.view(np.uint32))
    with pytest.raises(ValueError):
        int8_matmul(da, dw.T, partial_dot=True)  # the reference's rule: only with wrapped


@pytest.fixture()
def kitchen(monkeypatch, cuda):
    monkeypatch.syspath_prepend(KITCHEN)
    for name in [m for m in sys.modules if m.startswith("comfy_kitchen")]:
        monkeypatch.delitem(sys.modules, name)
    import comfy_kitchen.backends.eager as backend
    import comfy_kitchen.backends.eager.quantization as q
    return backend, q


@pytest.mark.parametrize("scalar_scale", [False, True])
@pytest.mark.parametrize("convrot,residual", [(False, False), (True, True)])
def test_moss_candidate_bit_exact(kitchen, cuda, scalar_scale, convrot, residual):
    from rdna2_ops.int8_gemm import moss_int8_gemm_candidate
    backend, q = kitchen
    case(f"moss candidate scalar={scalar_scale} convrot={convrot} residual={residual}")
    g = torch.Generator().manual_seed(21)
    x = torch.randn(2, 187, 768, generator=g).to(cuda)
    w = torch.randint(-127, 128, (640, 768), generator=g, dtype=torch.int8).to(cuda)
    ws = (torch.rand(1 if scalar_scale else 640, 1, generator=g) * 1e-3).to(cuda)
    b = torch.randn(640, generator=g).to(cuda)
    r = torch.randn(2, 187, 640, generator=g).to(cuda) if residual else None
    kw = dict(bias=b, out_dtype=torch.float32, convrot=convrot, convrot_groupsize=256, residual=r)
    expected = q.int8_linear(x, w, ws, **kw)  # the double's exact int64 accumulator
    saved = backend.int8_linear
    with moss_int8_gemm_candidate(tile=(64, 64, 64), num_warps=8, wrapped=True) as stats:
        assert backend.int8_linear is not saved
        got = backend.int8_linear(x, w, ws, **kw)
        fb = backend.int8_linear(x.bfloat16(), w, ws, bias=b.bfloat16(), out_dtype=torch.bfloat16)
    assert backend.int8_linear is saved
    assert got.dtype == torch.float32 and got.shape == (2, 187, 640)
    assert torch.equal(got, expected)
    assert torch.equal(fb, q.int8_linear(x.bfloat16(), w, ws, bias=b.bfloat16(), out_dtype=torch.bfloat16))
    assert stats == {"hits": 1, "fallbacks": 1, "shapes": {str((374, 640, 768)): 1}}


def test_moss_candidate_without_bias(kitchen, cuda):
    from rdna2_ops.int8_gemm import moss_int8_gemm_candidate
    backend, q = kitchen
    case("moss candidate no bias, 2-D input")
    g = torch.Generator().manual_seed(22)
    x = torch.randn(61, 512, generator=g).to(cuda)
    w = torch.randint(-127, 128, (96, 512), generator=g, dtype=torch.int8).to(cuda)
    ws = (torch.rand(96, generator=g) * 1e-3).to(cuda)
    with moss_int8_gemm_candidate() as stats:
        got = backend.int8_linear(x, w, ws, out_dtype=torch.float32)
    assert torch.equal(got, q.int8_linear(x, w, ws, out_dtype=torch.float32))
    assert stats["hits"] == 1 and stats["fallbacks"] == 0


@pytest.fixture()
def bridge(monkeypatch, cuda):
    spec = importlib.util.spec_from_file_location("patientx_rocm_int8_kitchen_patch", BRIDGE)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    monkeypatch.setitem(sys.modules, spec.name, mod)
    return mod


def _fused_expected(bridge, x, w, ws_vec, bias):
    a, sa = bridge.triton_quantize_rowwise(x.reshape(-1, x.shape[-1]).float())
    acc = o.int8_matmul(a.cpu().numpy(), np.ascontiguousarray(w.cpu().numpy().T))
    b = None if bias is None else bias.float().cpu().numpy()
    v = o.epilogue_f(acc, sa.cpu().numpy(), ws_vec, b, fused=True)
    return v.reshape(*x.shape[:-1], w.shape[0])


@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.float16, None])
def test_qwen_candidate_fused_epilogue(bridge, cuda, bias_dtype):
    from rdna2_ops.int8_gemm import qwen_int8_gemm_candidate
    case(f"qwen candidate bias={bias_dtype}")
    g = torch.Generator().manual_seed(23)
    x = torch.randn(3, 71, 1024, generator=g).to(cuda)
    w = torch.randint(-127, 128, (448, 1024), generator=g, dtype=torch.int8).to(cuda)
    ws_row = (torch.rand(448, 1, generator=g) * 1e-3 + 1e-5).to(cuda)
    ws_one = (torch.rand(1, generator=g) * 1e-3 + 1e-5).to(cuda)
    b = None if bias_dtype is None else torch.randn(448, generator=g).to(device=cuda, dtype=bias_dtype)
    saved = (bridge.triton_int8_linear, bridge.triton_int8_linear_per_row)
    number = 3.0517578125e-05  # an fp32-exact Python float
    with qwen_int8_gemm_candidate() as stats:  # found among the loaded modules by path
        y_row = bridge.triton_int8_linear_per_row(x, w, ws_row, bias=b, compute_dtype=torch.float32)
        y_ten = bridge.triton_int8_linear(x, w, ws_one, bias=b, compute_dtype=torch.float32)
        y_num = bridge.triton_int8_linear(x, w, number, bias=b, compute_dtype=torch.float32)
        y_fb = bridge.triton_int8_linear(x, w, ws_one, bias=b)  # compute_dtype fp16: not served
    assert (bridge.triton_int8_linear, bridge.triton_int8_linear_per_row) == saved
    assert stats["hits"] == 3 and stats["fallbacks"] == 1
    assert stats["shapes"] == {str((213, 448, 1024)): 3}
    assert y_fb.dtype == torch.float16
    for got, scale in ((y_row, ws_row.cpu().numpy().reshape(-1)), (y_ten, ws_one.cpu().numpy()),
                       (y_num, np.array([number], np.float32))):
        exp = _fused_expected(bridge, x, w, scale, b)
        assert got.shape == exp.shape
        assert np.array_equal(got.cpu().numpy().view(np.uint32), exp.view(np.uint32))


def test_qwen_candidate_refuses_foreign_patch(bridge, cuda):
    from rdna2_ops.int8_gemm import qwen_int8_gemm_candidate
    case("qwen candidate foreign patch")
    saved = bridge.triton_int8_linear_per_row
    with pytest.raises(RuntimeError):
        with qwen_int8_gemm_candidate(bridge):
            bridge.triton_int8_linear_per_row = lambda *a, **k: None
    bridge.triton_int8_linear_per_row = saved
