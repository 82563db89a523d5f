"""Host logic of the MOSS / Kitchen INT8 boundary (CPU only), against the
Kitchen test double in tests/kitchen_stub: install / rollback checks, the
precision fallback, statistics, the scoped context and the node switches."""
import importlib
import os
import sys
import threading
from pathlib import Path

import pytest
import torch

STUB = str(Path(__file__).resolve().parent / "kitchen_stub")


@pytest.fixture()
def kitchen(monkeypatch):
    monkeypatch.syspath_prepend(STUB)
    for name in [m for m in sys.modules if m.startswith("comfy_kitchen") or m == "rdna2_ops.comfy_int8"]:
        monkeypatch.delitem(sys.modules, name)
    import comfy_kitchen.backends.eager as eager_backend
    import comfy_kitchen.backends.eager.quantization as q
    # import_module, not "from rdna2_ops import comfy_int8": the package
    # attribute of an earlier test would be bound to that test's Kitchen
    ci = importlib.import_module("rdna2_ops.comfy_int8")
    yield ci, eager_backend, q
    ci.disable_backend()


def test_uninstalled_call_and_bad_arguments(kitchen):
    ci, eb, q = kitchen
    with pytest.raises(RuntimeError):
        ci.int8_linear(torch.zeros(2, 4), torch.zeros(3, 4, dtype=torch.int8), torch.ones(3))
    with pytest.raises(TypeError):
        ci.install_backend(None)
    with pytest.raises(RuntimeError):  # accumulator hook not installed first
        ci.install_backend(q._int8_matmul_accumulate.__call__)


def test_install_rollback_and_conflicts(kitchen):
    ci, eb, q = kitchen
    original = eb.int8_linear
    f = q._int8_matmul_accumulate
    ci.install_backend(f)
    from comfy_kitchen.registry import registry
    assert eb.int8_linear is ci.int8_linear
    assert registry.get_implementation("int8_linear", backend="eager") is ci.int8_linear
    ci.install_backend(f)  # idempotent
    with pytest.raises(RuntimeError):
        ci.install_backend(lambda a, b: None)
    ci.disable_backend()
    assert eb.int8_linear is original
    ci.disable_backend()  # no-op
    # refuse to overwrite a foreign patch
    ci.install_backend(f)
    foreign = lambda *a, **k: None  # noqa: E731
    eb.int8_linear = foreign
    with pytest.raises(RuntimeError):
        ci.disable_backend()
    eb.int8_linear = ci.int8_linear


def test_fallback_and_fp32_path_match_eager(kitchen):
    ci, eb, q = kitchen
    torch.manual_seed(0)
    x = torch.randn(3, 5, 512)
    w = torch.randint(-127, 128, (96, 512), dtype=torch.int8)
    ws = torch.rand(96, 1) * 1e-3
    b = torch.randn(96)
    r = torch.randn(3, 5, 96)
    ref32 = q.int8_linear(x, w, ws, bias=b, out_dtype=torch.float32, convrot=True, residual=r)
    ref16 = q.int8_linear(x.bfloat16(), w, ws, bias=b.bfloat16(), out_dtype=torch.bfloat16)
    ci.install_backend(q._int8_matmul_accumulate)
    got32 = ci.int8_linear(x, w, ws, bias=b, out_dtype=torch.float32, convrot=True, residual=r)
    assert torch.equal(got32, ref32)
    got16 = ci.int8_linear(x.bfloat16(), w, ws, bias=b.bfloat16(), out_dtype=torch.bfloat16)
    assert torch.equal(got16, ref16)  # not intercepted: Kitchen's original export
    with pytest.raises(ValueError):
        ci.int8_linear(x, w[:, :256], ws, out_dtype=torch.float32)
    with pytest.raises(ValueError):
        ci.int8_linear(x, w, torch.ones(7), out_dtype=torch.float32)
    with pytest.raises(ValueError):
        ci.int8_linear(x, w, ws, out_dtype=torch.float32, convrot=True, convrot_groupsize=384)


def test_scoped_context(kitchen):
    ci, eb, q = kitchen
    original = eb.int8_linear
    with ci.kitchen_int8_without_transpose_copy(q._int8_matmul_accumulate):
        assert eb.int8_linear is ci.int8_linear
        with pytest.raises(RuntimeError):
            with ci.kitchen_int8_without_transpose_copy(q._int8_matmul_accumulate):
                pass
    assert eb.int8_linear is original


def test_stats_switch(kitchen, monkeypatch):
    ci, eb, q = kitchen
    assert ci.get_stats()["enabled"] is False
    monkeypatch.setenv("MOSS_RDNA2_INT8_STATS", "1")
    ci = importlib.reload(ci)
    ci.install_backend(q._int8_matmul_accumulate)
    try:
        ci.int8_linear(torch.randn(4, 64), torch.ones(8, 64, dtype=torch.int8), torch.ones(8),
                       out_dtype=torch.float32)
        st = ci.get_stats()
        assert st["enabled"] and st["calls"] == 1
        assert st["weight_layouts"][0]["shape"] == (8, 64) and st["weight_layouts"][0]["rhs_stride"] == (1, 64)
        ci.reset_stats()
        assert ci.get_stats()["calls"] == 0
    finally:
        ci.disable_backend()


def test_concurrent_installs_are_serialised(kitchen):
    ci, eb, q = kitchen
    errors = []

    def run():
        try:
            ci.install_backend(q._int8_matmul_accumulate)
        except Exception as e:  # pragma: no cover - would be a bug
            errors.append(e)
    threads = [threading.Thread(target=run) for _ in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors and eb.int8_linear is ci.int8_linear


def test_node_switches(kitchen, monkeypatch):
    node_dir = Path(__file__).resolve().parents[1] / "rdna2-gfx1030-ai-handbook_amd"
    monkeypatch.syspath_prepend(str(node_dir))
    monkeypatch.delenv("MOSS_RDNA2_INT8_PATCH", raising=False)
    sys.modules.pop("MOSS_RDNA2_INT8", None)
    node = importlib.import_module("MOSS_RDNA2_INT8")
    assert node.NODE_CLASS_MAPPINGS == {}
    monkeypatch.setenv("MOSS_RDNA2_INT8_LAYOUT", "other")
    with pytest.raises(ValueError):
        node._install()
    monkeypatch.setenv("MOSS_RDNA2_INT8_LAYOUT", "view")
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError):
            node._install()
