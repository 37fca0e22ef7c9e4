"""Pins for the oracle's b16 codec (oracle/dtypes.py)."""

import numpy as np
import torch

from oracle.dtypes import decode, encode, rounded


def test_bf16_rounding_uses_ties_to_even():
    # Known answers of the reference (tests/operators/test_attention_math.py:14-19).
    ties = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8)], dtype=np.float32)
    assert np.array_equal(rounded(ties, "bf16"), np.array([1, 1 + 2**-6, -1], dtype=np.float32))


def test_bf16_matches_torch_round_to_nearest_even():
    rng = np.random.default_rng(7)
    values = np.concatenate(
        [
            rng.standard_normal(200_000).astype(np.float32) * 10,
            rng.uniform(-1e30, 1e30, 10_000).astype(np.float32),
            np.array([0.0, -0.0, 1e-40, -1e-40, 3.4e38, np.inf, -np.inf], np.float32),
        ]
    )
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(encode(values, "bf16"), expected)


def test_f16_roundtrip_and_decode_of_every_bf16_word():
    words = np.arange(65536, dtype=np.uint16)
    finite = decode(words, "bf16")
    ok = np.isfinite(finite)
    # Every finite bf16 value is a fixed point of the codec.
    assert np.array_equal(encode(finite[ok], "bf16"), words[ok])
    halves = np.array([0.5, 1.0, 65504.0, 6.1e-5, -2.0], np.float32)
    assert np.array_equal(rounded(halves, "f16"), halves.astype(np.float16).astype(np.float32))
