"""Host-side W4 code of the product package (CPU only): the torch CPU packer
that the reference exposes (pack_int4_cpu / unpack_int4_cpu) against the
numpy oracle, and the PackedInt4 container."""
import numpy as np
import pytest
import torch

from oracle import int4 as o4
from rdna2_ops import int4_weight_gemm_v07 as w4
from test_oracle_int4 import smoke_weight


@pytest.mark.parametrize("g", o4.GROUPS)
@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("order", ["low", "high"])
def test_pack_int4_cpu_equals_oracle(g, sym, layout, order):
    w = smoke_weight()
    rng = np.random.default_rng(g)
    w = np.concatenate([w, (rng.standard_normal((13, w.shape[1])) * 0.02).astype(np.float32)])
    p = w4.pack_int4_cpu(torch.from_numpy(w), group_size=g, symmetric=sym, layout=layout, order=order)
    r = o4.pack_int4_ref(w, group_size=g, symmetric=sym, layout=layout, order=order)
    for name in ("data", "scales", "zeros", "sums"):
        assert np.array_equal(getattr(p, name).numpy(), r[name]), name
    assert np.array_equal(w4.unpack_int4_cpu(p).numpy(), o4.unpack_int4_ref(r))
    assert np.array_equal(w4.unpack_int4_cpu(p, floating=False).numpy(), o4.unpack_int4_ref(r, floating=False))


def test_packed_container_properties():
    p = w4.pack_int4_cpu(torch.randn(16, 256), group_size=64, layout="kn", order="high")
    assert p.flags == w4._lib.W4_SIGNED_NIBBLES | w4._lib.W4_LAYOUT_KN | w4._lib.W4_ORDER_HIGH
    assert p.logical_stride == (1, 16)
    assert p.bytes == 16 * 32 * 4 + 3 * 16 * 4 * 4
    q = p.to("cpu")
    assert q.layout == "kn" and q.order == "high" and q.signed and not q.zeros_packed


def test_unpack_cpu_reads_baseline_storage():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    r = o4.pack_uint4_baseline(w, group_size=128)
    p = w4.PackedInt4(torch.from_numpy(r["data"]), torch.from_numpy(r["scales"].view(np.int16)).view(torch.bfloat16),
                      torch.from_numpy(r["zeros"]), torch.zeros(8, 4, dtype=torch.int32), 8, 512, 128, False,
                      signed=False, zeros_packed=True)
    assert np.array_equal(w4.unpack_int4_cpu(p, floating=False).numpy(), o4.dequant_baseline(r, floating=False))
    assert np.array_equal(w4.unpack_int4_cpu(p).numpy(), o4.dequant_baseline(r))


def test_cpu_pack_rejects_like_the_reference():
    with pytest.raises(ValueError):
        w4.pack_int4_cpu(torch.zeros(4, 100))
    with pytest.raises(ValueError):
        w4.pack_int4_cpu(torch.zeros(4, 128), layout="xy")
    with pytest.raises(ValueError):
        w4.pack_int4_cpu(torch.full((4, 128), float("nan")))
