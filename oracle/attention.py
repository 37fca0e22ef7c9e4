"""Flash-attention and teaching-attention oracles (test infrastructure only).

- ``online_attention`` restates the reference's FP32 online recurrence
  (``benchmarks/validation/attention.py:19-57``): per KV block
  ``m' = max(m, rowmax(s))``, ``alpha = e^(m - m')``, ``p = e^(s - m')``,
  ``l = l*alpha + sum(p)`` (unrounded FP32, 64-wide partial sums),
  ``O = O*alpha + b16(p) @ V``, final ``b16(O * (1/l))``. Causal masking is
  ``key > query_start + query_position`` -> -inf (``attention.py:35-41``).
- ``inputs`` draws FA inputs as the reference's ``inputs_and_oracle`` does
  (``attention.py:60-84``): standard normal * ``scale``, optional ``uniform``
  (K = 0) and ``sharp`` (Q, K * 3) cases, rounded to the storage dtype.
- ``simple_reference`` is the dense FP32 teaching reference
  (``benchmarks/attention/run_simple.py:115-118``): stable softmax, P @ V.
- ``dense_reference`` is plain FP32 softmax attention (with GQA and causal
  options) used as the reference for the fused FA kernel at full sizes.

Pinned by ``tests/test_oracle_attention.py`` with the reference's known
answers (``tests/operators/test_attention_math.py:14-94``): ties-to-even,
uniform K gives the per-head mean of V with the GQA head mapping, causal
absolute positions give prefix means, and P is rounded before PV.
"""

from __future__ import annotations

import numpy as np

from .dtypes import rounded


def online_attention(q, k, v, *, block_kv, dtype, scale, query_positions=None, causal=False, query_start=0):
    rows, dim = q.shape
    q = np.asarray(q, np.float32)
    maximum = np.full(rows, -np.inf, np.float32)
    denominator = np.zeros(rows, np.float32)
    output = np.zeros((rows, dim), np.float32)
    for first in range(0, k.shape[0], block_kv):
        keys = np.asarray(k[first : first + block_kv], np.float32)
        scores = ((q @ keys.T) * np.float32(scale)).astype(np.float32)
        if causal:
            if query_positions is None:
                raise ValueError("causal oracle needs absolute query positions")
            columns = np.arange(first, first + scores.shape[1])
            visible = columns[None, :] <= (query_start + np.asarray(query_positions))[:, None]
            scores = np.where(visible, scores, np.float32(-np.inf))
        new_max = np.maximum(maximum, scores.max(axis=1))
        # A block masked for a row keeps that row's state (exp(-inf) = 0).
        safe = np.where(np.isneginf(new_max), np.float32(0), new_max)
        alpha = np.exp((maximum - safe).astype(np.float32))
        probabilities = np.exp((scores - safe[:, None]).astype(np.float32))
        width = -(-probabilities.shape[1] // 64) * 64
        padded = np.zeros((rows, width), np.float32)
        padded[:, : probabilities.shape[1]] = probabilities
        row_sum = padded.reshape(rows, -1, 64).sum(axis=2, dtype=np.float32).sum(axis=1, dtype=np.float32)
        denominator = (denominator * alpha + row_sum).astype(np.float32)
        pv = rounded(probabilities, dtype) @ np.asarray(v[first : first + block_kv], np.float32)
        output = (output * alpha[:, None] + pv).astype(np.float32)
        maximum = new_max
    return rounded((output * (np.float32(1) / denominator[:, None])).astype(np.float32), dtype)


def inputs(batch, heads, kv_heads, sq, sk, dtype, *, seed=9102201, scale=1.0, case="standard", d=128):
    """Seeded FA inputs (b16-exact FP32 arrays): q [B,HQ,Sq,D], k/v [B,HKV,Sk,D]."""
    if case not in ("standard", "uniform", "sharp"):
        raise ValueError(f"unknown FA data case {case!r}")
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in (("q", (batch, heads, sq, d)), ("k", (batch, kv_heads, sk, d)), ("v", (batch, kv_heads, sk, d))):
        values = rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)
        if case == "uniform" and name == "k":
            values[:] = 0
        if case == "sharp" and name in ("q", "k"):
            values *= np.float32(3)
        out[name] = rounded(values, dtype)
    return out


def dense_reference(q, k, v, *, scale, causal=False):
    """FP32 softmax attention over [.., S, D] arrays with GQA broadcast on axis 1."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    group = q.shape[1] // k.shape[1]
    k = np.repeat(k, group, axis=1)
    v = np.repeat(v, group, axis=1)
    scores = np.einsum("bhqd,bhkd->bhqk", q, k, dtype=np.float32) * np.float32(scale)
    if causal:
        sq, sk = scores.shape[-2:]
        mask = np.arange(sk)[None, :] > np.arange(sq)[:, None]
        scores = np.where(mask, np.float32(-np.inf), scores)
    scores = scores - scores.max(axis=-1, keepdims=True)
    weights = np.exp(scores)
    weights /= weights.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", weights, v, dtype=np.float32)


def simple_reference(q, k, v, scale=128 ** -0.5):
    """Dense FP32 teaching-attention reference: q [H,S,D], k/v [H,128,D]."""
    q = np.asarray(q, np.float32)
    scores = (q @ np.asarray(k, np.float32).transpose(0, 2, 1)) * np.float32(scale)
    probability = np.exp(scores - scores.max(axis=-1, keepdims=True))
    probability /= probability.sum(axis=-1, keepdims=True)
    return probability @ np.asarray(v, np.float32)
