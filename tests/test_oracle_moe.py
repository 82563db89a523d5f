"""Pins of oracle/moe.py (CPU): routing against torch's softmax / topk,
dispatch invariants, the grouped organisation against a token-by-token
restatement, SiLU against its closed form, and a planted mistake that the
checks must catch."""
import numpy as np
import pytest
import torch

from oracle import int8 as o8
from oracle import moe


def small_case(seed=0, t=48, e=8, h=64, f=32, top_k=3):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16).float().numpy()
    logits = torch.randn(t, e, generator=g).numpy()
    wg = (torch.randn(e, f, h, generator=g) * 0.02).numpy()
    wu = (torch.randn(e, f, h, generator=g) * 0.02).numpy()
    wd = (torch.randn(e, h, f, generator=g) * 0.02).numpy()
    qg, sg = moe.quantize_experts(wg)
    qu, su = moe.quantize_experts(wu)
    qd, sd = moe.quantize_experts(wd)
    return x, logits, qg, sg, qu, su, qd, sd, top_k


def test_route_matches_torch():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(200, 64, generator=g)
    ex, w = moe.route_topk(logits.numpy(), 8)
    p = torch.softmax(logits, dim=1)
    tw, ti = torch.topk(logits, 8, dim=1)
    assert np.array_equal(ex, ti.numpy())
    np.testing.assert_allclose(w, torch.gather(p, 1, ti).numpy(), rtol=1e-6, atol=0)  # a few ulps: summation order
    assert (np.diff(np.take_along_axis(logits.numpy(), ex, 1), axis=1) <= 0).all()


def test_route_ties_lower_index_first():
    logits = np.zeros((2, 8), np.float32)
    logits[0, [5, 2, 7]] = 1.0
    ex, w = moe.route_topk(logits, 4)
    assert ex[0].tolist() == [2, 5, 7, 0]
    assert ex[1].tolist() == [0, 1, 2, 3]
    np.testing.assert_allclose(w[1], np.full(4, 1 / 8, np.float32))


def test_dispatch_invariants():
    g = torch.Generator().manual_seed(2)
    ex, _ = moe.route_topk(torch.randn(300, 16, generator=g).numpy(), 4)
    counts, offsets, rows, row_token, row_slot = moe.dispatch(ex, 16, pad=64)
    assert counts.sum() == 300 * 4
    assert (offsets % 64 == 0).all() and rows % 64 == 0
    for e in range(16):
        seg = slice(offsets[e], offsets[e] + counts[e])
        assert (ex.reshape(-1)[row_slot[seg]] == e).all()
        assert (row_token[offsets[e] + counts[e]: offsets[e] + (counts[e] + 63) // 64 * 64] == -1).all()
    assert np.array_equal(np.sort(row_slot[row_slot >= 0]), np.arange(1200))
    assert (row_token[row_slot >= 0] == row_slot[row_slot >= 0] // 4).all()


def test_silu_closed_form():
    g = np.linspace(-30, 30, 10001).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    np.testing.assert_allclose(moe.silu(g), ref, rtol=2e-6, atol=1e-30)
    assert moe.silu(np.float32([0.0]))[0] == 0.0


def test_grouped_equals_token_by_token():
    case = small_case()
    out, inter = moe.moe_forward(*case)
    ref = moe.moe_forward_bruteforce(*case)
    assert np.array_equal(out, ref)
    # a subset of tokens gives the same rows
    out2, _ = moe.moe_forward(*case, tokens=[3, 17, 40])
    assert np.array_equal(out2, out[[3, 17, 40]])


def test_int_parts_are_exact():
    x, logits, qg, sg, qu, su, qd, sd, k = small_case(seed=3)
    xq, xs = o8.quant_rows(x)
    acc = o8.int8_matmul(xq, qg[0].T)
    ref = xq.astype(np.int64) @ qg[0].T.astype(np.int64)
    assert np.array_equal(acc.astype(np.int64), ref)


def test_planted_mistake_is_caught():
    """Swapping gate and up (a plausible wiring slip) must change the result."""
    x, logits, qg, sg, qu, su, qd, sd, k = small_case(seed=4)
    good, _ = moe.moe_forward(x, logits, qg, sg, qu, su, qd, sd, k)
    bad, _ = moe.moe_forward(x, logits, qu, su, qg, sg, qd, sd, k)
    assert not np.array_equal(good, bad)


@pytest.mark.parametrize("seed", [5, 6])
def test_linearity_in_routing_weight(seed):
    """With one expert selected, halving every logit gap changes only the
    routing weight; the combined output of a single-slot token is its y row."""
    x, logits, qg, sg, qu, su, qd, sd, _ = small_case(seed=seed, top_k=1)
    out, inter = moe.moe_forward(x, logits, qg, sg, qu, su, qd, sd, 1)
    assert np.array_equal(out, inter["y"][:, 0])
