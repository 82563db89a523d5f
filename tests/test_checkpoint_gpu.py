"""Checkpoint loaders on the GPU: an INT8 checkpoint's layers run through the
INT8 GEMM in place, bit-identical to the direct call and to the oracle; the
W4 converter's resident copy equals a direct packing and is re-packed after
an in-place update."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from conftest import case
from oracle import int8 as o8

pytestmark = pytest.mark.gpu


def test_int8_checkpoint_linear_bit_exact(cuda, tmp_path):
    from rdna2_ops import checkpoint as ck
    from rdna2_ops.int8_gemm import w8a8_linear
    case("checkpoint int8 linear")
    g = torch.Generator().manual_seed(3)
    w = torch.randint(-127, 128, (384, 512), generator=g, dtype=torch.int8)
    s = torch.rand(384, 1, generator=g) * 0.01
    b = torch.randn(384, generator=g).to(torch.float16)
    save_file({"l.weight": w, "l.weight_scale": s, "l.bias": b}, str(tmp_path / "c.safetensors"))
    layer = ck.load_int8_linears(tmp_path / "c.safetensors", device=cuda)["l"]
    x = torch.randn(200, 512, generator=g).to(torch.float16)
    y = layer(x.to(cuda))
    assert torch.equal(y, w8a8_linear(x.to(cuda), w.to(cuda), s.reshape(-1).to(cuda), b.to(cuda)))
    ref, _, _, _ = o8.w8a8_linear(x.float().numpy(), w.numpy(), s.reshape(-1).numpy(), b.float().numpy(), out="f16")
    assert np.array_equal(y.cpu().view(torch.int16).numpy(), o8.encode(ref, "f16").view(np.int16))


def test_w4_converter_resident_copy(cuda):
    from rdna2_ops import checkpoint as ck
    from rdna2_ops import int4_weight_gemm_v07 as w4
    case("checkpoint w4 converter")
    g = torch.Generator().manual_seed(4)
    wq = torch.randint(-127, 128, (256, 512), generator=g, dtype=torch.int8).to(cuda)
    sc = (torch.rand(256, generator=g) * 0.01).to(cuda)
    wf = ck.dequantize_int8(wq, sc, torch.float32)
    conv = ck.w4_converter(group_size=128, uint4=True)
    p = conv.get("layer", wf)
    direct = w4.pack_uint4(wf, group_size=128)
    for name in ("data", "scales", "zeros"):
        assert torch.equal(getattr(p, name), getattr(direct, name)), name
    assert conv.get("layer", wf) is p and conv.prepared == 1
    wf.mul_(2)  # an in-place update (a LoRA merge, say): re-packed on next use
    p2 = conv.get("layer", wf)
    assert conv.prepared == 2 and torch.equal(p2.data, w4.pack_uint4(wf, group_size=128).data)


def test_resident_copy_misses_a_reloaded_weight_at_the_same_address(cuda):
    """A weight freed and re-allocated with other values (an offload round trip,
    a LoRA merged on the CPU) may land at the same address with version 0; the
    storage reference makes that a miss instead of a stale packed copy."""
    from rdna2_ops import checkpoint as ck
    from rdna2_ops import int4_weight_gemm_v07 as w4
    case("checkpoint w4 converter reload at the same address")
    conv = ck.w4_converter(group_size=128, uint4=True)
    g = torch.Generator().manual_seed(6)
    host_a = torch.randn(256, 512, generator=g) * 0.02
    host_b = torch.randn(256, 512, generator=g) * 0.02
    torch.cuda.synchronize()
    w = host_a.to(cuda)
    ptr = w.data_ptr()
    p = conv.get("layer", w)
    del w
    reused = None
    for _ in range(8):  # the caching allocator hands the freed block back
        w = host_b.to(cuda)
        if w.data_ptr() == ptr and w._version == 0:
            reused = w
            break
        del w
    if reused is None:
        pytest.skip("the allocator did not reuse the freed block")
    p2 = conv.get("layer", reused)
    assert conv.prepared == 2 and p2 is not p
    assert torch.equal(p2.data, w4.pack_uint4(reused, group_size=128).data)
