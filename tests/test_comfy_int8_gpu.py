"""MOSS / Kitchen INT8 boundary on the GPU: with this library's int8_matmul
installed as Kitchen's accumulator, the weight.T-view export (one fused
GEMM + eager-order epilogue launch) is bit-identical to Kitchen's eager
int8_linear (the test double in tests/kitchen_stub) on the same inputs —
fp32 activations / output, per-channel and scalar weight scales, ConvRot,
bias and residual — and the legacy layout (Kitchen's own linear over the
installed GEMM) is too."""
import importlib
import sys
from pathlib import Path

import pytest
import torch

from conftest import case

pytestmark = pytest.mark.gpu
STUB = str(Path(__file__).resolve().parent / "kitchen_stub")


@pytest.fixture()
def kitchen(monkeypatch, cuda):
    monkeypatch.syspath_prepend(STUB)
    for name in [m for m in sys.modules if m.startswith("comfy_kitchen") or m == "rdna2_ops.comfy_int8"]:
        monkeypatch.delitem(sys.modules, name)
    import comfy_kitchen.backends.eager.quantization as q
    ci = importlib.import_module("rdna2_ops.comfy_int8")
    from rdna2_ops.int8_gemm import int8_matmul
    yield ci, q, int8_matmul
    ci.disable_backend()


@pytest.mark.parametrize("scalar_scale", [False, True])
def test_view_export_matches_eager_bitwise(kitchen, cuda, scalar_scale):
    ci, q, int8_matmul = kitchen
    case(f"moss int8_linear view export scalar_scale={scalar_scale}")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 300, 1024, generator=g).to(cuda)
    w = torch.randint(-127, 128, (768, 1024), generator=g, dtype=torch.int8).to(cuda)
    ws = (torch.rand(1 if scalar_scale else 768, generator=g) * 1e-3).to(cuda)
    b = torch.randn(768, generator=g).to(cuda)
    r = torch.randn(2, 300, 768, generator=g).to(cuda)
    kw = dict(bias=b, out_dtype=torch.float32, convrot=True, convrot_groupsize=256, residual=r)
    expected = q.int8_linear(x, w, ws, **kw)  # stub's exact int64 accumulator
    q._int8_matmul_accumulate = int8_matmul
    legacy = q.int8_linear(x, w, ws, **kw)  # MOSS_RDNA2_INT8_LAYOUT=legacy
    assert torch.equal(legacy, expected)
    ci.install_backend(int8_matmul)
    got = ci.int8_linear(x, w, ws, **kw)
    assert got.dtype == torch.float32 and got.shape == (2, 300, 768)
    assert torch.equal(got, expected)
    # bf16 is not intercepted: Kitchen's original export runs unchanged
    got16 = ci.int8_linear(x.bfloat16(), w, ws, bias=b.bfloat16(), out_dtype=torch.bfloat16)
    assert torch.equal(got16, q.int8_linear(x.bfloat16(), w, ws, bias=b.bfloat16(), out_dtype=torch.bfloat16))
