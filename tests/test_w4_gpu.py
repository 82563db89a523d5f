"""W4 GPU parity: packing and unpacking bit-exact against the CPU oracle,
W4A16 GEMM against the float64 oracle.

Bar for the GEMM (the benchmark's): |y - y64| <= 1e-2 * rms(y64) for the arithmetic,
plus the rounding of the output format itself (half an ulp of bf16 / fp16 at
|y64|): one bf16 ulp at |y| in [2, 4) is 0.0156, more than 1e-2 * rms of these
outputs, so no implementation that writes bf16 meets the bare bar for every
element. With fp32 output the bare bar is checked as written. The kernel is
also held to a tighter bound that shows it computes the exact group sums: the
error stays within the output format's rounding (0.5 ulp of the output dtype
at |y64|) plus a few fp32 ulps of the biased group partial sums the kernel
accumulates (weights enter the MFMA as 128 + u, so 2^-20 * 144 *
sum_g s_g sum_k |a_k|)."""
import numpy as np
import pytest
import torch

from conftest import case
from oracle import int4 as o4
from oracle.int8 import bf16_bits_to_f32
from test_oracle_int4 import smoke_weight

pytestmark = pytest.mark.gpu


def w4():
    from rdna2_ops import int4_weight_gemm_v07 as mod
    return mod


def _np(t):
    return t.detach().cpu().numpy()


def act_values(a):
    return a.detach().cpu().float().numpy().astype(np.float64)


def check_product(y, y64, absmag, out_dtype, label):
    got = y.detach().cpu().float().numpy().astype(np.float64)
    err = np.abs(got - y64)
    rms = float(np.sqrt(np.mean(y64 ** 2))) if y64.size else 0.0
    half_ulp = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 0.0}[out_dtype]
    assert (err <= 1e-2 * rms + half_ulp * np.abs(y64) * 1.0001 + 1e-30).all(), f"{label}: 1e-2 x RMS bar"
    half_ulp = max(half_ulp, 2.0 ** -24)
    bound = half_ulp * np.abs(y64) * 1.0001 + 2.0 ** -20 * 144 * absmag + 1e-30
    if out_dtype == torch.float16:
        bound = bound + 2.0 ** -25  # fp16 subnormal spacing
    bad = err > bound
    assert not bad.any(), f"{label}: {bad.sum()} elements beyond one output rounding, worst {err[bad].max()}"


@pytest.mark.parametrize("g", o4.GROUPS)
@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("order", ["low", "high"])
def test_pack_unpack_reference_format(cuda, g, sym, layout, order):
    case(f"w4 pack g{g} sym={sym} {layout} {order}")
    w = smoke_weight()
    rng = np.random.default_rng(g)
    w = np.concatenate([w, (rng.standard_normal((45, w.shape[1])) * 0.02).astype(np.float32)])
    p = w4().pack_int4(torch.from_numpy(w).to(cuda), group_size=g, symmetric=sym, layout=layout, order=order)
    r = o4.pack_int4_ref(w, group_size=g, symmetric=sym, layout=layout, order=order)
    for name in ("data", "scales", "zeros", "sums"):
        assert np.array_equal(_np(getattr(p, name)), r[name]), name
    assert np.array_equal(_np(w4().unpack_int4(p, dtype=torch.int8)).astype(np.int32), o4.unpack_int4_ref(r, floating=False))
    f32 = o4.unpack_int4_ref(r)
    assert np.array_equal(_np(w4().unpack_int4(p, dtype=torch.float32)), f32)
    assert np.array_equal(_np(w4().unpack_int4(p, dtype=torch.float16)), f32.astype(np.float16))
    # bf16: torch's CPU round-to-nearest-even of the exact fp32 values, bit for bit
    bf = torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16)
    assert torch.equal(w4().unpack_int4(p, dtype=torch.bfloat16).cpu().view(torch.int16), bf)


@pytest.mark.parametrize("wdtype", [torch.float32, torch.float16, torch.bfloat16])
def test_pack_strided_and_half_inputs(cuda, wdtype):
    case(f"w4 pack strided {wdtype}")
    rng = np.random.default_rng(1)
    base = torch.from_numpy((rng.standard_normal((256, 96)) * 0.02).astype(np.float32)).to(wdtype)
    w = base.to(cuda).T  # [96, 256] with strides (1, 96)
    p = w4().pack_int4(w, group_size=64, symmetric=False)
    r = o4.pack_int4_ref(base.T.float().numpy(), group_size=64, symmetric=False)
    for name in ("data", "scales", "zeros", "sums"):
        assert np.array_equal(_np(getattr(p, name)), r[name]), name


def test_pack_uint4_baseline(cuda):
    case("w4 pack_uint4 baseline 300x1024")
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((300, 1024)) * 0.02).astype(np.float32)
    w[7] = 0
    p = w4().pack_uint4(torch.from_numpy(w).to(cuda), group_size=128)
    r = o4.pack_uint4_baseline(w, group_size=128)
    assert np.array_equal(_np(p.data), r["data"])
    assert np.array_equal(_np(p.scales.view(torch.int16)).view(np.uint16), r["scales"])
    assert np.array_equal(_np(p.zeros), r["zeros"])
    assert np.array_equal(_np(w4().unpack_int4(p, dtype=torch.int8)).astype(np.int32), o4.dequant_baseline(r, floating=False))
    assert np.array_equal(_np(w4().unpack_int4(p, dtype=torch.float32)), o4.dequant_baseline(r))


def _gemm_case(cuda, m, n, k, g, sym, layout, order, adtype, bias, out_dtype=None, a_pad=0, seed=0):
    from rdna2_ops import _lib
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p = w4().pack_int4(torch.from_numpy(w).to(cuda), group_size=g, symmetric=sym, layout=layout, order=order)
    r = o4.pack_int4_ref(w, group_size=g, symmetric=sym, layout=layout, order=order)
    a_full = torch.from_numpy(rng.standard_normal((m, k + a_pad)).astype(np.float32)).to(adtype)
    a = a_full.to(cuda)[:, :k]
    b = torch.from_numpy((rng.standard_normal(n) * 0.1).astype(np.float32)).to(adtype).to(cuda) if bias else None
    y = w4().w4a16_gemm(a, p, b, out_dtype=out_dtype)
    cen = o4.unpack_int4_ref(r, floating=False)
    av = act_values(a)
    y64 = o4.w4a16_linear(av, cen, r["scales"], g, act_values(b) if bias else None)
    absmag = o4.w4a16_linear(np.abs(av), np.ones_like(cen), np.abs(r["scales"]), g)
    label = f"m{m} n{n} k{k} g{g} {layout} {order}"
    if _lib.library().qg_w4a16_gemm_workspace_bytes(m, n, k, g, p.flags) > 0:
        # the dequant formulation: the weights are rounded to the activation
        # dtype first (the reference's dequant method), so the result is the
        # rounded-weight product within fp32 accumulation slack and the exact
        # product within the 1e-2 x RMS bar
        wq = w4().unpack_int4(p, dtype=adtype).float().cpu().numpy().astype(np.float64)
        bias64 = act_values(b) if bias else 0.0
        yq = av @ wq.T + bias64
        y32 = w4().w4a16_gemm(a, p, b, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
        slack = 2.0 ** -17 * (np.abs(av) @ np.abs(wq).T + np.abs(bias64))
        assert (np.abs(y32 - yq) <= slack).all(), f"{label}: fp32 output vs rounded-weight product"
        got = y.float().cpu().numpy().astype(np.float64)
        rms = float(np.sqrt(np.mean(y64 ** 2)))
        half = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 0.0}[out_dtype or adtype]
        assert (np.abs(got - y64) <= 1e-2 * rms + half * np.abs(y64) * 1.0001 + 1e-30).all(), f"{label}: 1e-2 x RMS bar"
    else:
        check_product(y, y64, absmag, out_dtype or adtype, label)


@pytest.mark.parametrize("g", o4.GROUPS)
@pytest.mark.parametrize("layout,order", [("nk", "low"), ("nk", "high"), ("kn", "low"), ("kn", "high")])
@pytest.mark.parametrize("adtype", [torch.float16, torch.bfloat16])
def test_w4a16_small_all_formats(cuda, g, layout, order, adtype):
    for m, sym, bias in ((1, False, True), (3, True, True), (7, True, False), (16, False, False), (37, False, True)):
        case(f"w4a16 m{m} n53 k384 g{g} {layout} {order} {adtype} sym={sym}")
        _gemm_case(cuda, m, 53, 384, g, sym, layout, order, adtype, bias, seed=m + g)


@pytest.mark.parametrize("m", [1, 3, 16, 17, 32, 33, 64, 65, 130])
def test_w4a16_row_tiles(cuda, m):
    case(f"w4a16 rows m{m} n200 k512")
    _gemm_case(cuda, m, 200, 512, 128, False, "nk", "low", torch.bfloat16, True, seed=m)


@pytest.mark.parametrize("k,g", [(96, 32), (160, 32), (192, 64), (320, 64)])
def test_w4a16_k_tails(cuda, k, g):
    case(f"w4a16 k-tail k{k} g{g}")
    for layout in ("nk", "kn"):
        _gemm_case(cuda, 5, 40, k, g, False, layout, "low", torch.float16, True, seed=k)


def test_w4a16_strided_activation_and_f32_out(cuda):
    case("w4a16 strided A, fp32 out")
    _gemm_case(cuda, 9, 64, 256, 64, False, "nk", "low", torch.bfloat16, True, out_dtype=torch.float32, a_pad=24)


def test_int4_linear_a16_methods(cuda):
    case("int4_linear_a16 dequant / prepared / dot2")
    mod = w4()
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((96, 256)) * 0.02).astype(np.float32)
    p = mod.pack_int4(torch.from_numpy(w).to(cuda), group_size=32, symmetric=False, layout="kn")
    a = torch.from_numpy(rng.standard_normal((5, 256)).astype(np.float32)).half().to(cuda)
    b = torch.from_numpy(rng.standard_normal(96).astype(np.float32) * 0.1).half().to(cuda)
    r = o4.pack_int4_ref(w, group_size=32, symmetric=False, layout="kn")
    y64 = o4.w4a16_linear(act_values(a), o4.unpack_int4_ref(r, floating=False), r["scales"], 32, act_values(b))
    rms = np.sqrt(np.mean(y64 ** 2))
    ref_out = y64.astype(np.float16).astype(np.float64)  # the fp16 output of the exact product
    for method in ("dequant", "dot2", "fused"):
        y = mod.int4_linear_a16(a, p, bias=b, method=method)
        assert y.dtype == torch.float16 and y.shape == (5, 96)
        assert np.abs(y.float().cpu().numpy() - ref_out).max() <= 1e-2 * rms, method
    wp = mod.unpack_int4(p)
    y = mod.int4_linear_a16(a, p, bias=b, method="prepared", prepared=wp)
    assert np.abs(y.float().cpu().numpy() - ref_out).max() <= 1e-2 * rms
    y, md = mod.int4_linear_a16(a, p, bias=b, method="dot2", return_kernel=True)
    assert md["variant"] == "w4a16_decode" and md["vgpr"] is not None  # 5 rows, K 256
    y, md = mod.int4_linear_a16(torch.cat([a] * 8), p, bias=b, method="dot2", return_kernel=True)
    assert md["variant"] == "w4a16_skinny" and md["vgpr"] is not None  # 40 rows
    y, md = mod.int4_linear_a16(torch.cat([a] * 20), p, bias=b, method="dot2", return_kernel=True)
    # 100 rows at group 32: the dequant formulation (every group-32 prefill grid)
    assert md["variant"] == "w4a16_dequant_pingpong" and md["vgpr"] is not None
    with pytest.raises(ValueError):
        mod.int4_linear_a16(a.float(), p)
    with pytest.raises(ValueError):
        mod.int4_linear_a16(a, p, method="prepared")
    with pytest.raises(ValueError):
        mod.int4_linear_a16(a, p, method="dot2", tile=(64, 64, 48))


@pytest.mark.parametrize("m", [1, 16])
def test_cfg2_decode_full_size(cuda, m):
    """Benchmark configuration 2 at its real shape (K 4096, N 14336, g128,
    uint4 storage with bf16 scales, bf16 activations and output)."""
    case(f"cfg2 w4a16 m{m} k4096 n14336")
    g = torch.Generator().manual_seed(2)
    w = (torch.randn(14336, 4096, generator=g) * 0.02)
    a = torch.randn(m, 4096, generator=g).to(torch.bfloat16)
    p = w4().pack_uint4(w.to(cuda), group_size=128)
    r = o4.pack_uint4_baseline(w.numpy(), group_size=128)
    assert np.array_equal(_np(p.data), r["data"]) and np.array_equal(_np(p.zeros), r["zeros"])
    av = act_values(a)
    cen = o4.dequant_baseline(r, floating=False)
    s = bf16_bits_to_f32(r["scales"])
    y64 = o4.w4a16_linear(av, cen, s, 128)
    absmag = o4.w4a16_linear(np.abs(av), np.ones_like(cen), s, 128)
    for out_dtype in (torch.bfloat16, torch.float32):
        y = w4().w4a16_gemm(a.to(cuda), p, out_dtype=out_dtype)
        check_product(y, y64, absmag, out_dtype, f"cfg2 m{m} {out_dtype}")


@pytest.mark.parametrize("n,k", [(1000, 512), (4100, 1536), (64, 4096), (14336, 4096)])
def test_uint4_single_row_kernel(cuda, n, k):
    """The single-row kernel (one bf16 row, uint4 storage, g128, K a multiple
    of 512 up to 4096): ragged N, short K (waves past K idle), bias and every
    output dtype, against the float64 oracle; and the kernel metadata names it."""
    case(f"uint4 single-row kernel n{n} k{k}")
    g = torch.Generator().manual_seed(n + k)
    w = torch.randn(n, k, generator=g) * 0.02
    a = torch.randn(1, k, generator=g).to(torch.bfloat16)
    b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    p = w4().pack_uint4(w.to(cuda), group_size=128)
    r = o4.pack_uint4_baseline(w.numpy(), group_size=128)
    av = act_values(a)
    cen = o4.dequant_baseline(r, floating=False)
    s = bf16_bits_to_f32(r["scales"])
    absmag = o4.w4a16_linear(np.abs(av), np.ones_like(cen), s, 128)
    for bias in (None, b):
        y64 = o4.w4a16_linear(av, cen, s, 128, None if bias is None else act_values(bias))
        for out_dtype in (torch.bfloat16, torch.float16, torch.float32):
            y = w4().w4a16_gemm(a.to(cuda), p, None if bias is None else bias.to(cuda), out_dtype=out_dtype)
            check_product(y, y64, absmag, out_dtype, f"single-row n{n} k{k} bias={bias is not None} {out_dtype}")
    _, md = w4().int4_linear_a16(a.to(cuda), p, method="dot2", return_kernel=True)
    assert md["variant"] == "w4a16_gemv1" and md["vgpr"] is not None


@pytest.mark.parametrize("m", [2, 5, 16])
@pytest.mark.parametrize("n,k", [(1000, 256), (4100, 1536), (64, 4096), (14336, 4096)])
def test_uint4_multi_row_decode(cuda, m, n, k):
    """The 2-16-row decode on the benchmark's uint4 storage (bf16 rows, g128):
    ragged N, short K (waves past K idle), bias and every output dtype,
    strided activation rows, against the float64 oracle; the kernel metadata
    names the decode kernel."""
    case(f"uint4 multi-row kernel m{m} n{n} k{k}")
    g = torch.Generator().manual_seed(m * 7 + n + k)
    w = torch.randn(n, k, generator=g) * 0.02
    a_full = torch.randn(m, k + 24, generator=g).to(torch.bfloat16)
    b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    p = w4().pack_uint4(w.to(cuda), group_size=128)
    r = o4.pack_uint4_baseline(w.numpy(), group_size=128)
    cen = o4.dequant_baseline(r, floating=False)
    s = bf16_bits_to_f32(r["scales"])
    for strided in (False, True):
        a = a_full[:, 8:8 + k] if strided else a_full[:, :k].contiguous()
        av = act_values(a)
        absmag = o4.w4a16_linear(np.abs(av), np.ones_like(cen), s, 128)
        ag = a_full.to(cuda)[:, 8:8 + k] if strided else a.to(cuda)
        for bias in (None, b):
            y64 = o4.w4a16_linear(av, cen, s, 128, None if bias is None else act_values(bias))
            for out_dtype in (torch.bfloat16, torch.float16, torch.float32):
                y = w4().w4a16_gemm(ag, p, None if bias is None else bias.to(cuda), out_dtype=out_dtype)
                check_product(y, y64, absmag, out_dtype,
                              f"multi-row m{m} n{n} k{k} strided={strided} bias={bias is not None} {out_dtype}")
    _, md = w4().int4_linear_a16(a.to(cuda), p, method="dot2", return_kernel=True)
    assert md["variant"] == "w4a16_decode" and md["vgpr"] is not None


def test_decode_metadata_column_tiles(cuda):
    """The decode kernel's reported column tile follows the launcher's choice
    per group size and row count (16 * CT columns)."""
    case("decode metadata column tiles")
    g = torch.Generator().manual_seed(9)
    for group, m, cols in ((32, 1, 32), (32, 5, 16), (64, 5, 32), (128, 5, 64), (128, 3, 32)):
        w = torch.randn(96, 512, generator=g) * 0.02
        p = w4().pack_int4(w.to(cuda), group_size=group, symmetric=False)
        a = torch.randn(m, 512, generator=g).to(torch.float16).to(cuda)
        _, md = w4().int4_linear_a16(a, p, method="dot2", return_kernel=True)
        assert md["variant"] == "w4a16_decode" and md["tile"][1] == cols, (group, m, md)
        assert md["vgpr"] is not None, (group, m)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 16])
@pytest.mark.parametrize("adtype", [torch.bfloat16, torch.float16])
def test_uint4_decode_row_counts_and_activation_types(cuda, m, adtype):
    """The uint4 decode path (K 3073-4096, g128, bf16 scales, nk storage) at
    every row-count instantiation the launcher picks for M <= 16 (1, 2-4, 5-16)
    and with fp16 as well as bf16 activations; N 2048 keeps it short."""
    case(f"uint4 decode m{m} {adtype} k4096 n2048")
    g = torch.Generator().manual_seed(40 + m)
    w = (torch.randn(2048, 4096, generator=g) * 0.02)
    a = torch.randn(m, 4096, generator=g).to(adtype)
    p = w4().pack_uint4(w.to(cuda), group_size=128)
    r = o4.pack_uint4_baseline(w.numpy(), group_size=128)
    av = act_values(a)
    cen = o4.dequant_baseline(r, floating=False)
    s = bf16_bits_to_f32(r["scales"])
    y64 = o4.w4a16_linear(av, cen, s, 128)
    absmag = o4.w4a16_linear(np.abs(av), np.ones_like(cen), s, 128)
    for out_dtype in (adtype, torch.float32):
        y = w4().w4a16_gemm(a.to(cuda), p, out_dtype=out_dtype)
        check_product(y, y64, absmag, out_dtype, f"uint4 decode m{m} {adtype} -> {out_dtype}")


@pytest.mark.parametrize("g", o4.GROUPS)
@pytest.mark.parametrize("layout,order", [("nk", "low"), ("nk", "high"), ("kn", "low")])
@pytest.mark.parametrize("adtype", [torch.float16, torch.bfloat16])
def test_w4a16_tiled_all_formats(cuda, g, layout, order, adtype):
    """M > 64 and K % 128 == 0: the tiled kernel (activation stages in LDS)."""
    for m, n, sym, bias in ((200, 200, False, True), (129, 64, True, False)):
        case(f"w4a16 tiled m{m} n{n} k384 g{g} {layout} {order} {adtype} sym={sym}")
        _gemm_case(cuda, m, n, 384, g, sym, layout, order, adtype, bias, seed=m + g)


@pytest.mark.parametrize("g,layout,m,n,variant,tile", [
    (64, "nk", 130, 200, "w4a16_tiled_mfma", [128, 64, 128]),         # 2 tiles of 256 x 192
    (128, "kn", 130, 200, "w4a16_tiled_mfma", [128, 64, 128]),        # 4 tiles of 128 x 128
    (128, "nk", 1024, 4096, "w4a16_tiled_mfma", [128, 128, 128]),     # 256 of 128 x 128, 88 of 256 x 192
    (64, "kn", 1024, 4096, "w4a16_dequant_pingpong", [256, 192, 64]),  # 88 >= 64 tiles of 256 x 192
    (32, "nk", 130, 200, "w4a16_dequant_pingpong", [256, 192, 64]),    # group 32: every prefill grid
    (32, "kn", 1024, 4096, "w4a16_dequant_pingpong", [256, 192, 64])])
def test_w4a16_prefill_kernel_choice(cuda, g, layout, m, n, variant, tile):
    """Prefill grids (M > 64, K 512): the tiled kernel's two tile widths (128 x 64
    where 128 x 128 tiles would leave CUs idle, else 128 x 128), and the dequant
    formulation from the group's tile threshold (192 tiles of 256 x 192 at group
    128, 64 at group 64, every grid at group 32). Each against the float64
    oracle (the dequant formulation against the rounded-weight product); the
    metadata names the launched kernel and tile, which spill nothing to scratch."""
    case(f"w4a16 prefill choice g{g} {layout} m{m} n{n}")
    _gemm_case(cuda, m, n, 512, g, False, layout, "low", torch.float16, True, seed=m + n + g)
    rng = np.random.default_rng(g)
    w = (rng.standard_normal((n, 512)) * 0.02).astype(np.float32)
    p = w4().pack_int4(torch.from_numpy(w).to(cuda), group_size=g, symmetric=False, layout=layout)
    a = torch.ones(m, 512, dtype=torch.float16, device=cuda)
    _, md = w4().int4_linear_a16(a, p, method="dot2", return_kernel=True)
    assert md["variant"] == variant and md["tile"] == tile, md
    assert md["vgpr"] is not None and md["vgpr_spills"] == 0 and md["scratch_bytes"] == 0, md


def test_w4a16_tiled_uint4_and_f32_out(cuda):
    case("w4a16 tiled uint4 storage, fp32 out")
    rng = np.random.default_rng(12)
    m, n, k = 300, 160, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p = w4().pack_uint4(torch.from_numpy(w).to(cuda), group_size=128)
    r = o4.pack_uint4_baseline(w, group_size=128)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    b = torch.from_numpy((rng.standard_normal(n) * 0.1).astype(np.float32)).to(torch.bfloat16)
    av = act_values(a)
    cen = o4.dequant_baseline(r, floating=False)
    s = bf16_bits_to_f32(r["scales"])
    y64 = o4.w4a16_linear(av, cen, s, 128, act_values(b))
    absmag = o4.w4a16_linear(np.abs(av), np.ones_like(cen), s, 128)
    for out_dtype in (torch.bfloat16, torch.float32):
        y = w4().w4a16_gemm(a.to(cuda), p, b.to(cuda), out_dtype=out_dtype)
        check_product(y, y64, absmag, out_dtype, f"tiled uint4 {out_dtype}")


def test_cfg2_prefill_full_size(cuda):
    """Benchmark configuration 2, prefill M = 2048 at its real shape. This grid
    takes the dequant path (W dequantised once to bf16 in the workspace, the
    reference's dequant formulation, then the 2-byte ping-pong GEMM). Every
    output is finite, meets the 1e-2 x RMS bar against the exact float64
    product of the oracle on the CPU, and matches the float64 product of the
    bf16-rounded weights the GEMM multiplies within one output rounding plus
    fp32 accumulation slack (all 2048 x 14336 outputs)."""
    from oracle.int8 import round_to
    case("cfg2 w4a16 m2048 k4096 n14336")
    g = torch.Generator().manual_seed(2)
    w = (torch.randn(14336, 4096, generator=g) * 0.02)
    a = torch.randn(2048, 4096, generator=g).to(torch.bfloat16)
    p = w4().pack_uint4(w.to(cuda), group_size=128)
    r = o4.pack_uint4_baseline(w.numpy(), group_size=128)
    y, md = w4().int4_linear_a16(a.to(cuda), p, method="dot2", return_kernel=True)
    assert md["variant"] == "w4a16_dequant_pingpong"
    assert torch.isfinite(y).all()
    av = act_values(a)
    got = y.float().cpu().numpy().astype(np.float64)
    cen = o4.dequant_baseline(r, floating=False)
    s = bf16_bits_to_f32(r["scales"])
    y64 = o4.w4a16_linear(av, cen, s, 128)
    rms = float(np.sqrt(np.mean(y64 ** 2)))
    assert (np.abs(got - y64) <= 1e-2 * rms + 2.0 ** -8 * np.abs(y64) * 1.0001).all(), "1e-2 x RMS bar"
    del y64
    wq = round_to(o4.dequant_baseline(r), "bf16").astype(np.float64)
    yq = av @ wq.T
    slack = 2.0 ** -17 * (np.abs(av) @ np.abs(wq).T)
    bad = np.abs(got - yq) > 2.0 ** -8 * np.abs(yq) * 1.0001 + slack
    assert not bad.any(), f"{bad.sum()} outputs beyond one rounding of the bf16-weight product"


@pytest.mark.parametrize("adtype,layout,group,m,n", [
    (torch.float16, "kn", 64, 1100, 7500), (torch.bfloat16, "nk", 32, 1100, 7500),
    (torch.bfloat16, "nk", 128, 2000, 6344), (torch.float16, "kn", 32, 2000, 6344)])
def test_w4a16_dequant_path_ragged(cuda, adtype, layout, group, m, n):
    """The dequant path on ragged grids with the reference's signed storage,
    bias and fp32 output. M 1100, N 7500: 200 tiles of 256 x 192 with partial
    edge tiles, one launch. M 2000, N 6344: 272 tiles, so the GEMM splits into
    columns [0, 6144) in one whole round of 256 x 192 tiles and a tail of
    128 x 128 tiles over columns [6144, 6344) (a partial column tile, ragged
    rows) that writes at the output's full row stride. The weights are
    dequantised to the activation dtype, so the result matches the float64
    product of those rounded weights within fp32 accumulation slack, and the
    exact product within the 1e-2 x RMS bar (every output, both parts)."""
    from oracle.int8 import round_to
    case(f"w4a16 dequant path m{m} n{n} k512 {adtype} {layout} g{group}")
    k = 512
    rng = np.random.default_rng(group)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    p = w4().pack_int4(torch.from_numpy(w).to(cuda), group_size=group, symmetric=False, layout=layout)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(adtype)
    b = torch.from_numpy((rng.standard_normal(n) * 0.1).astype(np.float32)).to(adtype)
    y, md = w4().int4_linear_a16(a.to(cuda), p, bias=b.to(cuda), method="dot2", return_kernel=True)
    assert md["variant"] == "w4a16_dequant_pingpong"
    y32 = w4().w4a16_gemm(a.to(cuda), p, b.to(cuda), out_dtype=torch.float32)
    av = act_values(a)
    # the weights the GEMM multiplies: the library's own dequantisation (checked
    # bit-exact against the oracle by the unpack tests), in the activation dtype
    wq = w4().unpack_int4(p, dtype=adtype).float().cpu().numpy().astype(np.float64)
    wexact = w4().unpack_int4(p, dtype=torch.float32).cpu().numpy().astype(np.float64)
    bias64 = act_values(b)
    yq = av @ wq.T + bias64
    yx = av @ wexact.T + bias64
    got32 = y32.cpu().numpy().astype(np.float64)
    slack = 2.0 ** -17 * (np.abs(av) @ np.abs(wq).T + np.abs(bias64))
    assert (np.abs(got32 - yq) <= slack).all(), "fp32 output vs rounded-weight product"
    rms = float(np.sqrt(np.mean(yx ** 2)))
    half = 2.0 ** -11 if adtype == torch.float16 else 2.0 ** -8
    got = y.float().cpu().numpy().astype(np.float64)
    assert (np.abs(got - yx) <= 1e-2 * rms + half * np.abs(yx) * 1.0001).all(), "1e-2 x RMS bar"


def test_read_floor_reads_without_writing(cuda):
    """qg_read_floor (the plain-read floor the decode is measured against)
    reads a ragged byte count and leaves its sink alone unless the folded word
    hits its constant."""
    from rdna2_ops import _lib
    case("read floor 30.5 MB")
    buf = torch.ones(30543872 + 48, dtype=torch.uint8, device=cuda)
    sink = torch.full((1,), 7, dtype=torch.int32, device=cuda)
    _lib.check(_lib.library().qg_read_floor(_lib.ptr(buf), buf.numel(), _lib.ptr(sink),
                                            _lib.stream_of(buf)), "qg_read_floor")
    torch.cuda.synchronize()
    assert int(sink.item()) == 7
