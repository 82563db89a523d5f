"""HIP graph capture of the library's launches (the benchmark-shape wrappers on torch's
capture stream): the library issues no memset, allocation or
synchronisation, so a captured W8A8 linear (quantizer + INT8 GEMM + fused
epilogue), W4A16 decode, W4A16 prefill (unpack + split 2-byte GEMM) and MoE
forward replay to the bits of the eager calls. Every replay
is checked, with eager work and synchronisations between the replays. The
reference-mirroring entry points refuse capture, as the reference does
(eager inference only)."""
import pytest
import torch

from conftest import case

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(cuda):
    from rdna2_ops import int4_weight_gemm_v07 as w4
    from rdna2_ops.int8_gemm import w8a8_linear
    from rdna2_ops.quantize import quantize_int8_rowwise
    case("graph capture: w8a8 linear + w4a16 decode")
    g = torch.Generator().manual_seed(11)
    x = torch.randn(512, 768, generator=g).half().to(cuda)
    w = (torch.randn(1024, 768, generator=g) * 0.02).half().to(cuda)
    wq, ws = quantize_int8_rowwise(w)
    bias = (torch.randn(1024, generator=g) * 0.01).half().to(cuda)
    a1 = torch.randn(1, 4096, generator=g).to(torch.bfloat16).to(cuda)
    p = w4.pack_int4((torch.randn(2048, 4096, generator=g) * 0.02).to(cuda), group_size=128)

    def work():
        return w8a8_linear(x, wq, ws, bias), w4.w4a16_gemm(a1, p)

    eager = [t.clone() for t in work()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = work()
    for i in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(outs, eager):
            assert torch.equal(got, ref), f"replay {i}"
        other = work()  # eager work between replays
        torch.cuda.synchronize()
        for got, ref in zip(other, eager):
            assert torch.equal(got, ref)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_reference_entry_points_refuse_capture(cuda):
    """int4_linear_a16 keeps the reference's eager-only contract
    (int4_weight_gemm_v07.py _eager): a ValueError under stream capture."""
    from rdna2_ops import int4_weight_gemm_v07 as w4
    case("graph capture refused by int4_linear_a16")
    p = w4.pack_int4((torch.randn(64, 256) * 0.02).to(cuda), group_size=128)
    a = torch.randn(1, 256).to(torch.bfloat16).to(cuda)
    w4.int4_linear_a16(a, p, method="dot2")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(ValueError, match="eager"):
        with torch.cuda.graph(graph):
            w4.int4_linear_a16(a, p, method="dot2")


def test_graph_replays_w4a16_prefill_split_and_moe(cuda):
    """The multi-launch paths under capture: the W4A16 dequant formulation
    (unpack into the workspace, then the 2-byte GEMM split into whole rounds
    of 256 x 192 tiles and a round of 128 x 128 tiles: M 2000, N 6344) and a
    MoE forward (dispatch, quantizers, the persistent grouped GEMMs, combine).
    Every replay matches the eager call's bits, with eager work and
    synchronisations between the replays."""
    from rdna2_ops import int4_weight_gemm_v07 as w4
    from rdna2_ops import moe_int8
    case("graph capture: w4a16 prefill split + moe forward")
    g = torch.Generator().manual_seed(12)
    p = w4.pack_uint4((torch.randn(6344, 512, generator=g) * 0.02).to(cuda), group_size=128)
    a = torch.randn(2000, 512, generator=g).to(torch.bfloat16).to(cuda)
    b = (torch.randn(6344, generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    t, e, h, f, k = 300, 16, 512, 256, 4
    x = torch.randn(t, h, generator=g).to(torch.bfloat16).to(cuda)
    logits = torch.randn(t, e, generator=g).to(cuda)
    prep = moe_int8.prepare_moe_weights((torch.randn(e, f, h, generator=g) * 0.05).to(cuda),
                                        (torch.randn(e, f, h, generator=g) * 0.05).to(cuda),
                                        (torch.randn(e, h, f, generator=g) * 0.05).to(cuda))

    def work():
        return w4.w4a16_gemm(a, p, b), moe_int8.moe_int8_forward(x, logits, prep, top_k=k)

    eager = [o.clone() for o in work()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = work()
    for i in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(outs, eager):
            assert torch.equal(got, ref), f"replay {i}"
        other = work()  # eager work between replays
        torch.cuda.synchronize()
        for got, ref in zip(other, eager):
            assert torch.equal(got, ref)
