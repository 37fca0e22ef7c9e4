"""Pins for the top-k index selection oracle (oracle/topk_reference.py).

The reference has no indexer (docs/operators/sparse-mla.md:8,266), so there is
no golden vector for the selection itself. The pins are: the float order
(``score_keys`` against NumPy's comparisons), the defining property of a top-k
set checked by brute force on tied scores, ``torch.topk`` on distinct scores,
closed forms, and the reference's own index distribution
(benchmarks/attention/sparse_performance.py:44-47) recovered from indicator
scores, which ties the cutoff and count to the sparse contract.
"""

import numpy as np
import pytest
import torch

from ascendflow_amd.sparse_attention.inputs import make_metadata, measurement_policy
from oracle import topk_reference as tr


def special_floats(rng, n):
    pool = np.array([0.0, -0.0, 1.0, -1.0, 0.5, np.inf, -np.inf, 3.0e38, -3.0e38, 1e-45, -1e-45, 2.0], np.float32)
    return np.concatenate([pool, rng.normal(0, 10, n).astype(np.float32)])


def test_score_keys_follow_the_float_order():
    values = np.sort(special_floats(np.random.default_rng(1), 4000))
    keys = tr.score_keys(values)
    assert np.all(np.diff(keys.astype(np.int64)) >= 0)
    # Equal keys exactly where the floats compare equal (-0 == +0).
    same_key = keys[1:] == keys[:-1]
    same_float = values[1:] == values[:-1]
    assert np.array_equal(same_key, same_float)
    nans = np.array([np.nan, -np.nan, np.float32(np.nan) * -1], np.float32)
    nans = np.concatenate([nans, np.array([0x7F800001, 0xFFC00000], np.uint32).view(np.float32)])
    assert np.all(tr.score_keys(nans) == 0xFFFFFFFF)
    assert tr.score_keys(np.array([np.inf], np.float32))[0] < 0xFFFFFFFF


def ragged_metadata(rng, b, ratio, max_cmp):
    counts = rng.integers(0, 6, b).astype(np.int32)
    counts[0] = 0  # an empty request
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    seq_cmp = rng.integers(0, max_cmp + 1, b).astype(np.int32)
    residual = (rng.integers(0, ratio, b) if ratio > 1 else np.zeros(b)).astype(np.int32)
    return cu, seq_cmp, residual


def check_topk_property(scores, out, cu, seq_cmp, residual, topk, ratio):
    """The defining property of the selection, checked on each token by brute force."""
    t, c = scores.shape
    keys = tr.score_keys(scores).astype(np.int64)
    cutoff, bound = tr.token_bounds(cu, seq_cmp, residual, ratio)
    for token in range(t):
        cand = int(min(cutoff[token], c))
        take = int(min(topk, bound[token], cand))
        row = out[token, 0]
        assert np.all(row[take:] == -1)
        sel = row[:take]
        assert np.all(np.diff(sel) > 0) and (take == 0 or (sel[0] >= 0 and sel[-1] < cand))
        if take == 0 or take == cand:
            assert take == 0 or np.array_equal(sel, np.arange(cand))
            continue
        rest = np.setdiff1d(np.arange(cand), sel)
        lowest = keys[token, sel].min()
        assert lowest >= keys[token, rest].max()
        # Ties at the threshold go to the lowest positions.
        tied_rest = rest[keys[token, rest] == lowest]
        tied_sel = sel[keys[token, sel] == lowest]
        assert tied_rest.size == 0 or tied_sel.max() < tied_rest.min()


@pytest.mark.parametrize("ratio", [1, 2])
def test_selection_meets_the_top_k_property_on_tied_and_special_scores(ratio):
    rng = np.random.default_rng(20 + ratio)
    b, topk, max_cmp = 7, 6, 14
    cu, seq_cmp, residual = ragged_metadata(rng, b, ratio, max_cmp)
    t = int(cu[-1])
    for c in (max_cmp, 9):  # full rows, and rows shorter than the cutoff
        scores = rng.integers(-2, 3, (t, c)).astype(np.float32)  # heavy ties
        special = special_floats(rng, 0)
        mask = rng.random((t, c)) < 0.2
        scores[mask] = rng.choice(special, int(mask.sum()))
        out = tr.topk_indices(scores, cu, seq_cmp, residual, topk, ratio)
        check_topk_property(scores, out, cu, seq_cmp, residual, topk, ratio)


def test_distinct_scores_match_torch_topk():
    rng = np.random.default_rng(5)
    b, topk, ratio = 5, 17, 2
    cu, seq_cmp, residual = ragged_metadata(rng, b, ratio, 60)
    t, c = int(cu[-1]), 60
    scores = np.stack([rng.permutation(c) for _ in range(t)]).astype(np.float32) - 20.5
    out = tr.topk_indices(scores, cu, seq_cmp, residual, topk, ratio)
    cutoff, bound = tr.token_bounds(cu, seq_cmp, residual, ratio)
    for token in range(t):
        cand = int(min(cutoff[token], c))
        take = int(min(topk, bound[token], cand))
        expect = np.full(topk, -1, np.int32)
        if take:
            expect[:take] = np.sort(torch.topk(torch.from_numpy(scores[token, :cand]), take).indices.numpy())
        assert np.array_equal(out[token, 0], expect), token


def test_closed_forms():
    cu = np.array([0, 3], np.int32)
    seq_cmp, residual = np.array([40], np.int32), np.array([1], np.int32)
    cutoff, bound = tr.token_bounds(cu, seq_cmp, residual, 2)
    # cutoff = (40 * 2 + 1 - 3 + j + 1) // 2 for j = 0, 1, 2.
    assert list(cutoff) == [39, 40, 40] and list(bound) == [39, 40, 40]
    positions = np.tile(np.arange(40, dtype=np.float32), (3, 1))
    for scores, expect in (
        (-positions, lambda cand, take: np.arange(take)),  # falling scores: the first positions
        (positions, lambda cand, take: np.arange(cand - take, cand)),  # rising: the last ones
        (np.zeros_like(positions), lambda cand, take: np.arange(take)),  # constant: ties to the lowest
    ):
        out = tr.topk_indices(scores, cu, seq_cmp, residual, 8, 2)
        for token in range(3):
            assert np.array_equal(out[token, 0], expect(int(cutoff[token]), 8)), token
    # TOPK beyond the candidates: every candidate, then -1.
    out = tr.topk_indices(positions, cu, seq_cmp, residual, 48, 2)
    assert np.array_equal(out[0, 0], np.r_[np.arange(39), np.full(9, -1)])


@pytest.mark.parametrize("context,query_tokens,ratio", [(300, 3, 2), (257, 5, 1), (1100, 2, 2)])
def test_indicator_scores_recover_the_reference_index_distribution(context, query_tokens, ratio):
    policy = measurement_policy(3, query_tokens, context, topk=128, ratio=ratio, page=64)
    meta = make_metadata(policy, context, seed=11)
    indices = meta["cmp_sparse_indices"]
    t, c = policy["T"], context // ratio
    rng = np.random.default_rng(3)
    scores = rng.uniform(-1.0, 0.99, (t, c)).astype(np.float32)
    chosen = np.zeros((t, c), bool)
    for token in range(t):
        row = indices[token, 0]
        chosen[token, row[row >= 0]] = True
    scores[chosen] = rng.uniform(1.0, 2.0, int(chosen.sum())).astype(np.float32)
    # Positions past the generator's own bound right // R score highest of all:
    # a selection that let one in would differ.
    cu = meta["cu_seqlens_q"]
    for r in range(policy["B"]):
        n = int(cu[r + 1] - cu[r])
        for j in range(n):
            right = context - n + j + 1
            scores[cu[r] + j, right // ratio :] = 5.0
    out = tr.topk_indices(scores, meta["cu_seqlens_q"], meta["seqused_cmp_kv"], meta["cmp_residual_kv"],
                          policy["TOPK"], ratio)
    assert np.array_equal(out, indices)
