"""The allocation-free W8A8 linear (qg_w8a8_linear_noalloc) through the C ABI:
bit-identical to qg_w8a8_linear with caller workspace on two calls in a row,
the second with a smaller input (the persistent 256x192 grid, then the 4-wave
grid with a weight that needs packing into the scratch), and a size beyond
the scratch refused before any HIP call."""
import ctypes

import pytest
import torch

from conftest import case

pytestmark = pytest.mark.gpu
INVALID = 1  # hipErrorInvalidValue
SCRATCH = 64 << 20


def _inputs(m, n, k, seed, dev, w_pad=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.float16)
    x[torch.rand(m, k, generator=g) < 1e-3] *= 20
    w_store = torch.randint(-127, 128, (n, k + w_pad), generator=g, dtype=torch.int8)
    ws = torch.rand(n, generator=g) * 1e-3 + 1e-5
    b = (torch.randn(n, generator=g) * 0.01).to(torch.float16)
    return x.to(dev), w_store.to(dev)[:, :k], ws.to(dev), b.to(dev)


def _run(lib, L, noalloc, x, w, ws, b, epi):
    m, k = x.shape
    n = w.shape[0]
    out = torch.full((m, n), float("nan"), dtype=torch.float16, device=x.device)
    s = torch.cuda.current_stream(x.device).cuda_stream
    args = [L.ptr(x), L.F16, x.stride(0), m, k, L.ptr(w), w.stride(0), n, L.ptr(ws), ws.numel(), L.ptr(b), L.F16,
            L.ptr(out), L.F16, L.ROUND_HALF_EVEN, epi]
    if noalloc:
        status = lib.qg_w8a8_linear_noalloc(*args, s)
        work = None
    else:
        need = lib.qg_w8a8_linear_workspace_bytes(L.ptr(w), w.stride(0), m, n, k)
        work = torch.empty(max(int(need), 16), dtype=torch.uint8, device=x.device)
        status = lib.qg_w8a8_linear(*args, L.ptr(work), work.numel(), s)
    L.check(status, "qg_w8a8_linear_noalloc" if noalloc else "qg_w8a8_linear")
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_workspace_entry_two_calls(cuda):
    from rdna2_ops import _lib as L
    lib = L.library()
    cases = (
        # persistent ping-pong grid (256 tiles of 256x192), GELU epilogue
        ("first", 4096, 3072, 3072, 0, L.EPI_GELU_TANH),
        # smaller: 4-wave grid, K not a multiple of 128 and a padded weight row
        # stride, so the weight is packed into the scratch as well
        ("second, smaller", 300, 640, 1000, 24, 0),
    )
    for label, m, n, k, pad, epi in cases:
        case(f"w8a8 noalloc {label}: m{m} n{n} k{k} w_pad{pad} epi{epi}")
        x, w, ws, b = _inputs(m, n, k, 31 + m, cuda, pad)
        need = lib.qg_w8a8_linear_workspace_bytes(L.ptr(w), w.stride(0), m, n, k)
        assert 0 < need <= SCRATCH
        ref = _run(lib, L, False, x, w, ws, b, epi)
        got = _run(lib, L, True, x, w, ws, b, epi)
        assert torch.isfinite(ref).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), label


def test_noalloc_refuses_sizes_beyond_the_scratch(cuda):
    from rdna2_ops import _lib as L
    lib = L.library()
    case("w8a8 noalloc oversize")
    p = ctypes.c_void_p(16)  # never dereferenced: the size check fails first
    m, n, k = 8192, 3072, 12288  # 100 MB of int8 activations
    assert lib.qg_w8a8_linear_workspace_bytes(p, k, m, n, k) > SCRATCH
    s = torch.cuda.current_stream(cuda).cuda_stream
    status = lib.qg_w8a8_linear_noalloc(p, L.F16, k, m, k, p, k, n, p, n, None, 0, p, L.F16,
                                        L.ROUND_HALF_EVEN, 0, s)
    assert status == INVALID
