"""Top-k index selection oracle (test infrastructure only).

The reference has no indexer: ``cmp_sparse_indices`` is an input of its sparse
operator, produced by the caller (``docs/operators/sparse-mla.md:8,266``). This
module states the contract that tensor must meet and the selection rule of
this repository's producer, ``launch_sparse_topk_indices``:

- ``cutoff``   <- ``query_geometry`` (``sparse_reference.py``, restating
  ``benchmarks/attention/sparse_reference.py:29-42``): for token ``t`` of request
  ``b`` with ``n`` queries and offset ``j``,
  ``cutoff = max(0, C_b R + r_b - n + j + 1) // R``.
- ``count``    ``min(TOPK, C_b, cutoff)``, the ranks the operator reads
  (``sparse_reference.py:117-124`` in the reference; ``docs/operators/sparse-mla.md:41-51``).
- ``topk_indices``  per token, the ``min(count, C)`` positions ``p < min(cutoff, C)``
  of largest score (ties to the lower position; -0 equals +0; NaN above +inf),
  ascending, then -1 (``docs/operators/sparse-mla.md:79``). Brute force: one
  stable ``lexsort`` per token.

Pinned by ``tests/test_oracle_topk.py``: the defining order property on random
tied scores, ``torch.topk`` on distinct scores, closed forms (monotone and
constant scores), and the reference's own index distribution
(``benchmarks/attention/sparse_performance.py:44-47``: sorted, without
replacement, ``min(512, right // R)`` of ``[0, right // R)``) recovered exactly
from indicator scores. Parity with any particular upstream indexer (the
scores themselves) is unpinned: the reference holds none.
"""

from __future__ import annotations

import numpy as np


def score_keys(scores):
    """Order-preserving uint32 keys of f32 scores (larger score, larger key;
    -0 and +0 share a key; every NaN takes the largest key)."""
    bits = np.ascontiguousarray(scores, dtype=np.float32).view(np.uint32)
    mag = bits & np.uint32(0x7FFFFFFF)
    keys = np.where(bits >> np.uint32(31), ~bits, bits | np.uint32(0x80000000))
    keys = np.where(mag == 0, np.uint32(0x80000000), keys)
    return np.where(mag > np.uint32(0x7F800000), np.uint32(0xFFFFFFFF), keys).astype(np.uint32)


def token_bounds(cu_seqlens_q, seqused_cmp_kv, cmp_residual_kv, ratio):
    """Per token: (cutoff, count) of the sparse contract, as ``query_geometry``."""
    cu = np.asarray(cu_seqlens_q, np.int64)
    t = int(cu[-1])
    tokens = np.arange(t)
    batch = np.searchsorted(cu, tokens, side="right") - 1
    n = cu[batch + 1] - cu[batch]
    offset = tokens - cu[batch]
    available = np.asarray(seqused_cmp_kv, np.int64)[batch]
    end = available * ratio + np.asarray(cmp_residual_kv, np.int64)[batch]
    cutoff = np.maximum(0, end - n + offset + 1) // ratio
    return cutoff, np.minimum(available, cutoff)


def topk_indices(scores, cu_seqlens_q, seqused_cmp_kv, cmp_residual_kv, topk, ratio):
    """``cmp_sparse_indices`` [T, 1, TOPK] int32 selected from ``scores`` [T, C]."""
    scores = np.asarray(scores, np.float32)
    t, c = scores.shape
    cutoff, bound = token_bounds(cu_seqlens_q, seqused_cmp_kv, cmp_residual_kv, ratio)
    out = np.full((t, 1, topk), -1, np.int32)
    keys = score_keys(scores)
    for token in range(t):
        cand = int(min(cutoff[token], c))
        take = int(min(topk, bound[token], cand))
        if take <= 0:
            continue
        # lexsort: last key is primary; descending key, then ascending position.
        order = np.lexsort((np.arange(cand), -keys[token, :cand].astype(np.int64)))
        out[token, 0, :take] = np.sort(order[:take])
    return out
