"""Pins of oracle/fp8.py (CPU only): every byte pattern against torch's own
float8 -> float32 casts, the encoder against torch's round-to-nearest-even
cast, and the product against brute-force loops."""
import numpy as np
import pytest
import torch

from oracle import fp8 as o8


@pytest.mark.parametrize("dtype,e5", [(torch.float8_e4m3fn, False), (torch.float8_e5m2, True)])
def test_all_256_patterns_match_torch(dtype, e5):
    raw = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = raw.view(dtype).float().numpy()
    got = o8.decode_bits(raw.numpy(), e5)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # signed zeros too
    if not e5:
        assert nan.sum() == 2 and np.isnan(got[0x7F]) and np.isnan(got[0xFF])
        assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_encoder_matches_torch_rne_and_saturates():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000) * 100, rng.standard_normal(2000) * 1e-3,
                        [0.0, -0.0, 448.0, -448.0, 449.0, 1e6, -1e6]]).astype(np.float32)
    got = o8.encode_e4m3(x)
    ref = torch.from_numpy(np.clip(x, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_encoder_ties_go_to_even_codes():
    vals = o8.decode_bits(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    assert np.array_equal(mids.astype(np.float64), (vals[:-1] + vals[1:]) / 2)  # exact midpoints
    got = o8.encode_e4m3(np.concatenate([mids, -mids]))
    ref = torch.from_numpy(np.concatenate([mids, -mids])).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)
    assert (got[: len(mids)] % 2 == 0).all()


def test_per_channel_quantiser():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((6, 64)) * 0.02).astype(np.float32)
    w[2] = 0
    codes, s = o8.quantize_weight_per_channel(w)
    dec = o8.decode_bits(codes)
    assert s[2] == 1 and (dec[2] == 0).all()
    # the channel maximum maps to exactly +-448
    assert np.array_equal(np.abs(dec).max(1)[[0, 1, 3, 4, 5]], np.full(5, 448.0, np.float32))
    rel = np.abs(dec * s[:, None] - w) / np.maximum(np.abs(w), 2.0 ** -6 * s[:, None])
    assert rel.max() <= 2.0 ** -4 + 1e-6  # 3 mantissa bits: half an ulp is 2^-4 relative


@pytest.mark.parametrize("e5", [False, True])
def test_product_bruteforce(e5):
    rng = np.random.default_rng(4)
    a = rng.standard_normal((3, 40)).astype(np.float32)
    codes = rng.integers(0, 256, (5, 40)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # finite weights only
    if e5:
        codes[((codes >> 2) & 31) == 31] = 1
    s = rng.random(5).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    np.testing.assert_allclose(o8.fp8_linear(a, codes, s, b, e5), o8.fp8_linear_bruteforce(a, codes, s, b, e5),
                               rtol=1e-12, atol=1e-9)
