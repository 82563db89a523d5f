"""Host logic of the research adapters (CPU only): the scoped swap and its
restore, precision fallbacks and their counters, the refusal to undo a
foreign patch, and the patientx bridge lookup (rdna2-ops/rdna2_ops/
int8_gemm.py:217-330). The fp32 GEMM path of both adapters is covered on
the GPU (tests/test_adapters_gpu.py)."""
import importlib.util
import sys
from pathlib import Path

import pytest
import torch

from rdna2_ops import _kitchen
from rdna2_ops.int8_gemm import moss_int8_gemm_candidate, qwen_int8_gemm_candidate

HERE = Path(__file__).resolve().parent
KITCHEN = str(HERE / "kitchen_stub")
BRIDGE = HERE / "patientx_stub" / "RDNA2-Qwen21-INT8" / "rocm_int8_kitchen_patch.py"


@pytest.fixture()
def kitchen(monkeypatch):
    monkeypatch.syspath_prepend(KITCHEN)
    for name in [m for m in sys.modules if m.startswith("comfy_kitchen")]:
        monkeypatch.delitem(sys.modules, name)
    import comfy_kitchen.backends.eager as backend
    import comfy_kitchen.backends.eager.quantization as q
    return backend, q


@pytest.fixture()
def bridge(monkeypatch):
    spec = importlib.util.spec_from_file_location("patientx_rocm_int8_kitchen_patch", BRIDGE)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    monkeypatch.setitem(sys.modules, spec.name, mod)
    return mod


def test_moss_candidate_fallback_and_restore(kitchen):
    backend, q = kitchen
    saved = backend.int8_linear
    x = torch.randn(4, 64).bfloat16()
    w = torch.randint(-127, 128, (8, 64), dtype=torch.int8)
    ws = torch.rand(8) * 1e-3
    with moss_int8_gemm_candidate() as stats:
        got = backend.int8_linear(x, w, ws, out_dtype=torch.bfloat16)
        got32in = backend.int8_linear(x.float(), w, ws, out_dtype=torch.bfloat16)
    assert backend.int8_linear is saved
    assert torch.equal(got, q.int8_linear(x, w, ws, out_dtype=torch.bfloat16))
    assert torch.equal(got32in, q.int8_linear(x.float(), w, ws, out_dtype=torch.bfloat16))
    assert stats == {"hits": 0, "fallbacks": 2, "shapes": {}}


def test_moss_candidate_refuses_foreign_patch(kitchen):
    backend, _ = kitchen
    foreign = lambda *a, **k: None  # noqa: E731
    with pytest.raises(RuntimeError):
        with moss_int8_gemm_candidate():
            backend.int8_linear = foreign
    assert backend.int8_linear is foreign  # left alone


def test_moss_candidate_argument_checks_before_the_gemm(kitchen):
    backend, _ = kitchen
    x = torch.randn(3, 512)
    w = torch.zeros(16, 512, dtype=torch.int8)
    with moss_int8_gemm_candidate() as stats:
        with pytest.raises(ValueError):  # inner dimensions
            backend.int8_linear(x, w[:, :256], torch.ones(16), out_dtype=torch.float32)
        with pytest.raises(ValueError):  # scale neither scalar nor per channel
            backend.int8_linear(x, w, torch.ones(7), out_dtype=torch.float32)
        with pytest.raises(ValueError):  # ConvRot group does not divide K
            backend.int8_linear(x, w, torch.ones(16), out_dtype=torch.float32, convrot=True,
                                convrot_groupsize=384)
    assert stats["hits"] == 0


def test_qwen_candidate_lookup_and_fallbacks(bridge, monkeypatch):
    saved = (bridge.triton_int8_linear, bridge.triton_int8_linear_per_row)
    x = torch.randn(2, 5, 32)
    w = torch.randint(-127, 128, (12, 32), dtype=torch.int8)
    ws = torch.rand(12, 1) * 1e-3
    with qwen_int8_gemm_candidate() as stats:  # found by its source path
        y16 = bridge.triton_int8_linear_per_row(x, w, ws)  # compute_dtype fp16: not served
        yh = bridge.triton_int8_linear(x.half(), w, 0.001, compute_dtype=torch.float32)
    assert (bridge.triton_int8_linear, bridge.triton_int8_linear_per_row) == saved
    assert stats == {"hits": 0, "fallbacks": 2, "shapes": {}}
    assert torch.equal(y16, saved[1](x, w, ws))
    assert torch.equal(yh, saved[0](x.half(), w, 0.001, compute_dtype=torch.float32))
    # a second loaded bridge makes the lookup ambiguous, none makes it fail
    monkeypatch.setitem(sys.modules, "second_bridge", bridge)
    with pytest.raises(RuntimeError):
        with qwen_int8_gemm_candidate():
            pass
    monkeypatch.delitem(sys.modules, "second_bridge")
    monkeypatch.delitem(sys.modules, "patientx_rocm_int8_kitchen_patch")
    with pytest.raises(RuntimeError):
        with qwen_int8_gemm_candidate():
            pass


def test_swapped_restores_on_error():
    class Owner:
        f = staticmethod(len)
    with pytest.raises(KeyError):
        with _kitchen.swapped(Owner, {"f": abs}, "changed"):
            assert Owner.f is abs
            raise KeyError("body failed")
    assert Owner.f is len


def test_call_stats():
    s = _kitchen.CallStats()
    s.hit(4, 8, 16)
    s.hit(4, 8, 16)
    s.fallback()
    assert s.data == {"hits": 2, "fallbacks": 1, "shapes": {"(4, 8, 16)": 2}}
