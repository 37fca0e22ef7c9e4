"""Pins for the flash/teaching attention oracles (oracle/attention.py).

Known answers restated from the reference (tests/operators/test_attention_math.py:22-94).
"""

import numpy as np
import pytest

from oracle.attention import dense_reference, inputs, online_attention, simple_reference
from oracle.dtypes import rounded


def test_uniform_keys_give_the_mean_of_each_heads_own_values():
    data = inputs(1, 4, 2, 128, 1024, "bf16", case="uniform", scale=0.5)
    for head in range(4):
        actual = online_attention(data["q"][0, head], data["k"][0, head // 2], data["v"][0, head // 2], block_kv=1024, dtype="bf16", scale=128**-0.5)
        mean = rounded(data["v"][0, head // 2].mean(axis=0), "bf16")
        assert np.array_equal(actual, np.broadcast_to(mean, (128, 128)))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_causal_offset_uses_absolute_query_positions(dtype):
    positions = np.array([0, 15, 16, 31, 32, 63, 64, 127])
    q = np.zeros((len(positions), 64), np.float32)
    k = np.zeros((192, 64), np.float32)
    v = rounded(np.arange(192, dtype=np.float32)[:, None] / 16 + np.arange(64, dtype=np.float32)[None, :] / 256, dtype)
    actual = online_attention(q, k, v, block_kv=64, dtype=dtype, scale=0.125, causal=True, query_start=17, query_positions=positions)
    for index, row in enumerate(positions):
        mean = rounded(v[: 18 + row].mean(axis=0), dtype)
        assert np.allclose(actual[index], mean, rtol=0.002 if dtype == "f16" else 0.01, atol=0.001)


def test_head_rows_share_one_decode_query_position():
    q = np.zeros((4, 64), np.float32)
    k = np.zeros((128, 64), np.float32)
    v = np.broadcast_to(np.arange(128, dtype=np.float32)[:, None] / 16, (128, 64)).copy()
    actual = online_attention(q, k, v, block_kv=64, dtype="f16", scale=0.125, causal=True, query_start=17, query_positions=np.zeros(4, np.int64))
    assert np.array_equal(actual, np.broadcast_to(rounded(v[:18].mean(axis=0), "f16"), (4, 64)))


def test_online_oracle_rounds_probability_operands_before_pv():
    q = np.full((1, 64), 0.8, np.float32)
    k = np.arange(128 * 64, dtype=np.float32).reshape(128, 64) % 13 / 16
    v = np.arange(128 * 64, dtype=np.float32).reshape(128, 64) % 17 / 32
    scores = np.float32((q @ k.T) * np.float32(0.125))
    probabilities = np.exp(np.float32(scores - scores.max(axis=1, keepdims=True)))
    expected = rounded(np.float32((rounded(probabilities, "bf16") @ v) / probabilities.sum(axis=1, keepdims=True, dtype=np.float32)), "bf16")
    assert np.array_equal(online_attention(q, k, v, block_kv=128, dtype="bf16", scale=0.125), expected)


@pytest.mark.parametrize("causal", [False, True])
def test_online_recurrence_matches_dense_softmax(causal):
    data = inputs(1, 2, 1, 96, 300, "f16", scale=1.0)
    dense = dense_reference(data["q"], data["k"], data["v"], scale=128**-0.5, causal=causal)
    for head in range(2):
        online = online_attention(data["q"][0, head], data["k"][0, 0], data["v"][0, 0], block_kv=64, dtype="f16", scale=128**-0.5,
                                  causal=causal, query_positions=np.arange(96))
        np.testing.assert_allclose(online, dense[0, head], rtol=0.01, atol=0.002)


def test_dense_reference_gqa_and_causal_closed_forms():
    q = np.zeros((1, 4, 5, 8), np.float32)
    k = np.zeros((1, 2, 5, 8), np.float32)
    v = np.random.default_rng(0).standard_normal((1, 2, 5, 8)).astype(np.float32)
    out = dense_reference(q, k, v, scale=1.0, causal=True)
    for head in range(4):
        for row in range(5):
            np.testing.assert_allclose(out[0, head, row], v[0, head // 2, : row + 1].mean(axis=0), rtol=1e-6, atol=1e-6)


def test_simple_reference_is_row_stochastic_mix_of_values():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2, 64, 128)).astype(np.float32)
    k = rng.standard_normal((2, 128, 128)).astype(np.float32)
    v = np.ones((2, 128, 128), np.float32) * 3
    np.testing.assert_allclose(simple_reference(q, k, v), 3.0, rtol=1e-5)
    k[:] = 0
    v = rng.standard_normal((2, 128, 128)).astype(np.float32)
    np.testing.assert_allclose(simple_reference(q, k, v), np.broadcast_to(v.mean(axis=1, keepdims=True), (2, 64, 128)), rtol=1e-5, atol=1e-6)


def test_simple_reference_equals_dense_softmax_on_random_inputs():
    """Random q, k, v: a transposed K, a missing or wrong 128^-0.5 scale or a
    softmax over the wrong axis changes the output. dense_reference (einsum,
    GQA broadcast) is itself pinned by the closed forms above."""
    rng = np.random.default_rng(7)
    q = rng.standard_normal((3, 96, 128)).astype(np.float32)
    k = rng.standard_normal((3, 128, 128)).astype(np.float32)
    v = rng.standard_normal((3, 128, 128)).astype(np.float32)
    dense = dense_reference(q[None], k[None], v[None], scale=128**-0.5, causal=False)[0]
    np.testing.assert_allclose(simple_reference(q, k, v), dense, rtol=1e-5, atol=1e-6)
    for wrong in (1.0, 0.125, 128**-0.5 * 1.01):
        assert not np.allclose(dense_reference(q[None], k[None], v[None], scale=wrong)[0], dense, rtol=1e-4, atol=1e-5)
    assert not np.allclose(simple_reference(q, k.transpose(0, 2, 1).copy(), v), dense, rtol=1e-4, atol=1e-5)


def test_simple_reference_matches_textbook_softmax_brute_force():
    """Scalar float64 loops of O[i] = sum_j softmax_j(q_i . k_j / sqrt(128)) v_j on a tiny input."""
    import math

    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 3, 128)).astype(np.float32)
    k = rng.standard_normal((1, 128, 128)).astype(np.float32)
    v = rng.standard_normal((1, 128, 128)).astype(np.float32)
    expected = np.zeros((1, 3, 128))
    for i in range(3):
        scores = [sum(float(q[0, i, d]) * float(k[0, j, d]) for d in range(128)) / math.sqrt(128) for j in range(128)]
        top = max(scores)
        weights = [math.exp(s - top) for s in scores]
        total = sum(weights)
        for j in range(128):
            expected[0, i] += weights[j] / total * v[0, j].astype(np.float64)
    np.testing.assert_allclose(simple_reference(q, k, v), expected, rtol=1e-5, atol=1e-6)
