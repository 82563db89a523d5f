"""Checkpoint loaders and the resident-copy validity contract (CPU): safetensors
files written here, read back through rdna2_ops.checkpoint."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from rdna2_ops import checkpoint as ck


@pytest.fixture()
def int8_file(tmp_path):
    g = torch.Generator().manual_seed(0)
    t = {
        "blocks.0.attn.qkv.weight": torch.randint(-127, 128, (96, 64), generator=g, dtype=torch.int8),
        "blocks.0.attn.qkv.weight_scale": torch.rand(96, 1, generator=g) * 0.01,
        "blocks.0.attn.qkv.bias": torch.randn(96, generator=g).to(torch.float16),
        "blocks.0.mlp.fc.weight": torch.randint(-127, 128, (32, 64), generator=g, dtype=torch.int8),
        "blocks.0.mlp.fc.weight_scale": torch.tensor([0.02]),
        "blocks.0.norm.weight": torch.ones(64),                      # not int8: skipped
        "blocks.0.raw.weight": torch.zeros(8, 64, dtype=torch.int8),  # no scale: skipped
    }
    path = tmp_path / "int8.safetensors"
    save_file(t, str(path))
    return path, t


def test_read_weight_like_the_reference(int8_file):
    path, t = int8_file
    w, s, info = ck.read_weight(path, "blocks.0.attn.qkv.weight")
    assert torch.equal(w, t["blocks.0.attn.qkv.weight"]) and s.shape == (96,)
    assert torch.equal(s, t["blocks.0.attn.qkv.weight_scale"].reshape(-1))
    assert info["shape"] == [96, 64] and info["dtype"] == "torch.int8" and len(info["tensor_sha256"]) == 64
    w2, s2, info2 = ck.read_weight(path, "blocks.0.raw.weight")
    assert s2 is None and info2["scale_sha256"] is None
    with pytest.raises(KeyError):
        ck.read_weight(path, "missing.weight")


def test_load_int8_linears(int8_file):
    path, t = int8_file
    layers = ck.load_int8_linears(path, device="cpu")
    assert sorted(layers) == ["blocks.0.attn.qkv", "blocks.0.mlp.fc"]
    q = layers["blocks.0.attn.qkv"]
    assert q.weight.dtype == torch.int8 and q.weight.is_contiguous() and q.scale.dtype == torch.float32
    assert torch.equal(q.scale, t["blocks.0.attn.qkv.weight_scale"].reshape(-1))
    assert q.bias.dtype == torch.float16 and torch.equal(q.bias, t["blocks.0.attn.qkv.bias"])
    assert layers["blocks.0.mlp.fc"].scale.shape == (1,) and layers["blocks.0.mlp.fc"].bias is None
    assert sorted(ck.load_int8_linears(path, device="cpu", prefix="blocks.0.mlp")) == ["blocks.0.mlp.fc"]


def test_load_int8_rejects_bad_tensors(tmp_path):
    bad = {"a.weight": torch.zeros(4, 8, dtype=torch.int8), "a.weight_scale": torch.ones(3)}
    save_file(bad, str(tmp_path / "bad.safetensors"))
    with pytest.raises(ValueError, match="1 or N"):
        ck.load_int8_linears(tmp_path / "bad.safetensors", device="cpu")
    nan = {"a.weight": torch.zeros(4, 8, dtype=torch.int8), "a.weight_scale": torch.tensor([float("nan")] * 4)}
    save_file(nan, str(tmp_path / "nan.safetensors"))
    with pytest.raises(ValueError, match="non-finite"):
        ck.load_int8_linears(tmp_path / "nan.safetensors", device="cpu")


def test_load_fp8_weight(tmp_path):
    w = (torch.randn(16, 32) * 0.1).to(torch.float8_e4m3fn)
    save_file({"l.weight": w, "l.weight_scale": torch.tensor([0.5])}, str(tmp_path / "f.safetensors"))
    got, s = ck.load_fp8_weight(tmp_path / "f.safetensors", "l.weight", device="cpu")
    assert got.dtype == torch.float8_e4m3fn and torch.equal(got.view(torch.uint8), w.view(torch.uint8))
    assert s.shape == (16,) and (s == 0.5).all()
    save_file({"m.weight": torch.ones(2, 2)}, str(tmp_path / "g.safetensors"))
    with pytest.raises(ValueError, match="fp8"):
        ck.load_fp8_weight(tmp_path / "g.safetensors", "m.weight", device="cpu")


def test_resident_copy_contract():
    """A copy is reused while its source is unchanged; an in-place update
    (version bump), a new tensor at another address, or an explicit
    invalidate() each force a new preparation."""
    cache = ck.ResidentWeights(lambda t: t.clone() * 2)
    w = torch.arange(12.0).reshape(3, 4)
    a = cache.get("w", w)
    assert cache.get("w", w) is a and cache.prepared == 1
    w.add_(1)  # in-place update: the version counter moves
    b = cache.get("w", w)
    assert cache.prepared == 2 and torch.equal(b, (torch.arange(12.0).reshape(3, 4) + 1) * 2)
    w2 = w.clone()  # same values, another tensor
    cache.get("w", w2)
    assert cache.prepared == 3
    cache.invalidate("w")
    assert "w" not in cache
    cache.get("w", w2)
    assert cache.prepared == 4 and len(cache) == 1
    cache.get("v", w2.t())  # another key and another view (strides differ)
    assert cache.prepared == 5
    cache.clear()
    assert len(cache) == 0


def test_dequantize_int8():
    w = torch.tensor([[1, -2], [127, -128]], dtype=torch.int8)
    s = torch.tensor([0.5, 0.25])
    assert torch.equal(ck.dequantize_int8(w, s), torch.tensor([[0.5, -1.0], [31.75, -32.0]]))
    assert ck.dequantize_int8(w, s, torch.bfloat16).dtype == torch.bfloat16
    with pytest.raises(ValueError):
        ck.dequantize_int8(w.float(), s)
