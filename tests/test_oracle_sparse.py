"""Pins for the sparse-MLA oracle (oracle/sparse_reference.py, oracle/cpu_reference.py).

The tiny fixture and its expected answers are the reference's own known-answer
tests (tests/operators/test_sparse_attention.py:14-129); the rest are closed
forms and brute-force restatements chosen so that a dropped term, a wrong
index or a transposed operand fails one of them.
"""

import numpy as np
import pytest

from oracle import sparse_reference as sr
from oracle.cpu_reference import CpuSparseMla
from oracle.dtypes import rounded


@pytest.fixture
def problem():
    policy = {
        "B": 1, "T": 1, "H": 2, "D": 4, "PAGE": 4, "RATIO": 2, "WINDOW": 3, "TOPK": 4, "S": 8,
        "DTYPE": "bf16", "SCALE": 0.5,
    }
    data = {
        "q": np.zeros((1, 2, 4), np.float32),
        "ori_kv": np.arange(32, dtype=np.float32).reshape(2, 4, 1, 4) / 16,
        "cmp_kv": np.arange(16, dtype=np.float32).reshape(2, 2, 1, 4) / 4,
        "ori_block_table": np.array([[1, 0]], np.int32),
        "cmp_block_table": np.array([[1, 0]], np.int32),
        "seqused_ori_kv": np.array([5], np.int32),
        "ori_topk_length": np.array([[2]], np.int32),
        "cu_seqlens_q": np.array([0, 1], np.int32),
        "seqused_cmp_kv": np.array([2], np.int32),
        "cmp_residual_kv": np.array([1], np.int32),
        "cmp_sparse_indices": np.array([[[1, 1, 2, -1]]], np.int32),
        "sinks": np.zeros(2, np.float32),
    }
    return data, policy


def test_pages_repeated_indices_and_compression_causality(problem):
    data, policy = problem
    rows, slots = sr.selected_rows(data, policy, 0)
    # Positions 3,4 cross a page; index 1 twice; index 2 not complete at L=5, R=2.
    assert slots == [0, 1, 3, 4]
    expected = np.stack([data["ori_kv"][1, 3, 0], data["ori_kv"][0, 0, 0], data["cmp_kv"][1, 1, 0], data["cmp_kv"][1, 1, 0]])
    assert np.array_equal(rows, expected)
    kv, bias = sr.gather_oracle(data, policy)
    assert np.array_equal(kv[0, slots], rows)
    assert np.all(kv[0, [2, 5, 6, 7]] == 0)
    assert np.array_equal(np.isfinite(bias[0]), [True, True, False, True, True, False, False, False])


def test_both_cache_planes_and_one_sink_share_a_single_denominator(problem):
    data, policy = problem
    rows, _ = sr.selected_rows(data, policy, 0)
    actual = sr.oracle(data, policy)
    expected = rounded((rows.sum(axis=0) / 5)[None, None, :].repeat(2, axis=1), "bf16")
    assert np.array_equal(actual, expected)
    data["cmp_sparse_indices"][0, 0, :2] = [0, 1]
    assert not np.array_equal(sr.oracle(data, policy), actual)


def test_empty_selection_and_extreme_finite_sinks_are_zero(problem):
    data, policy = problem
    for key in ("seqused_ori_kv", "seqused_cmp_kv", "cmp_residual_kv"):
        data[key][:] = 0
    data["cmp_sparse_indices"][:] = -1
    data["sinks"][:] = [-80, 80]
    assert np.array_equal(sr.oracle(data, policy), np.zeros_like(data["q"]))


def test_padding_is_not_read_and_replay_window_is_respected(problem):
    data, policy = problem
    data["ori_topk_length"][:] = 1
    data["cmp_sparse_indices"][0, 0] = [0, -1, -1, -1]
    rows, slots = sr.selected_rows(data, policy, 0)
    assert slots == [0, 3]
    assert np.array_equal(rows[0], data["ori_kv"][0, 0, 0])


def test_four_verification_tokens_have_individual_windows_indices_and_compression_edges(problem):
    data, policy = problem
    policy["T"] = 4
    data["q"] = np.zeros((4, 2, 4), np.float32)
    data["cu_seqlens_q"] = np.array([0, 4], np.int32)
    data["seqused_ori_kv"][:] = 6
    data["seqused_cmp_kv"][:] = 3
    data["cmp_residual_kv"][:] = 0
    data["ori_topk_length"] = np.zeros((4, 1), np.int32)
    data["cmp_sparse_indices"] = np.array(
        [[[2, 0, 1, -1]], [[0, 2, 1, -1]], [[1, 0, 2, -1]], [[2, 0, 1, -1]]], np.int32
    )
    for token, compressed in enumerate(([], [0], [1, 0], [2, 0, 1])):
        expected = [data["ori_kv"][data["ori_block_table"][0, p // 4], p % 4, 0] for p in range(token, token + 3)]
        expected += [data["cmp_kv"][data["cmp_block_table"][0, p // 2], p % 2, 0] for p in compressed]
        rows, _ = sr.selected_rows(data, policy, token)
        np.testing.assert_array_equal(rows, expected)
    before = sr.oracle(data, policy)
    data["ori_kv"][0, 1, 0] += 10  # raw position 5
    data["cmp_kv"][0, 0, 0] += 10  # compressed index 2
    after = sr.oracle(data, policy)
    np.testing.assert_array_equal(before[:3], after[:3])
    assert not np.array_equal(before[3], after[3])


def brute_force_selection(data, policy, token):
    """Selection from first principles for complete caches (C = L // R, r = L % R).

    A token at absolute position P = L - n + j sees raw positions
    (P - visible, P] and compressed entry i iff its last raw position
    (i + 1) * R - 1 is <= P (docs/operators/sparse-mla.md:47-52).
    """
    cu = data["cu_seqlens_q"]
    batch = max(b for b in range(policy["B"]) if cu[b] <= token and cu[b + 1] > token)
    n = cu[batch + 1] - cu[batch]
    position = int(data["seqused_ori_kv"][batch]) - n + (token - cu[batch])
    visible = min(policy["WINDOW"], max(0, position + 1))
    if data["ori_topk_length"][token, 0] > 0:
        visible = min(visible, int(data["ori_topk_length"][token, 0]))
    out = []
    for slot, p in enumerate(range(position - visible + 1, position + 1)):
        blk = data["ori_block_table"][batch, p // policy["PAGE"]]
        out.append((slot, 0, int(blk) * policy["PAGE"] + p % policy["PAGE"]))
    cpage = policy["PAGE"] // policy["RATIO"]
    for rank in range(policy["TOPK"]):
        i = int(data["cmp_sparse_indices"][token, 0, rank])
        if i >= 0 and (i + 1) * policy["RATIO"] - 1 <= position and i < data["seqused_cmp_kv"][batch]:
            blk = data["cmp_block_table"][batch, i // cpage]
            out.append((policy["WINDOW"] + rank, 1, int(blk) * cpage + i % cpage))
    return out


@pytest.mark.parametrize("ratio", [1, 2])
@pytest.mark.parametrize("case", ["mixed", "ragged", "padding", "duplicates", "replay"])
def test_selection_matches_first_principles(case, ratio):
    policy = sr.default_policy(B=4, T=16, H=2, D=8, MAX_SEQ=1024, ORI_BLOCKS=16, CMP_BLOCKS=16, TOPK=64, RATIO=ratio)
    data = sr.inputs(policy, case)
    for token in range(policy["T"]):
        if data["cu_seqlens_q"][-1] <= token:
            continue
        assert sr.selected_physical(data, policy, token) == brute_force_selection(data, policy, token)


def test_sink_as_zero_valued_extra_column_closed_form():
    """softmax over [scores, sink] applied to [rows; 0] equals the oracle (float64)."""
    policy = sr.default_policy(B=3, T=9, H=4, D=16, MAX_SEQ=512, ORI_BLOCKS=8, CMP_BLOCKS=8, TOPK=32)
    data = sr.inputs(policy, "mixed")
    data["sinks"] = np.array([-3.0, 0.0, 1.5, 6.0], np.float32)
    got = sr.oracle_fp32(data, policy)
    for token in range(policy["T"]):
        rows, _ = sr.selected_rows(data, policy, token)
        q = data["q"][token].astype(np.float64)
        scores = np.concatenate([q @ rows.T.astype(np.float64) * policy["SCALE"], data["sinks"][:, None]], axis=1)
        weights = np.exp(scores - scores.max(axis=1, keepdims=True))
        weights /= weights.sum(axis=1, keepdims=True)
        values = np.concatenate([rows.astype(np.float64), np.zeros((1, policy["D"]))])
        np.testing.assert_allclose(got[token], weights @ values, rtol=2e-5, atol=2e-6)


def test_zero_query_gives_rows_over_n_plus_exp_sink():
    policy = sr.default_policy(B=2, T=4, H=3, D=8, MAX_SEQ=512, ORI_BLOCKS=8, CMP_BLOCKS=8, TOPK=16)
    data = sr.inputs(policy, "mixed")
    data["q"][:] = 0
    data["sinks"] = np.array([-1.0, 0.0, 2.0], np.float32)
    got = sr.oracle_fp32(data, policy)
    for token in range(policy["T"]):
        rows, _ = sr.selected_rows(data, policy, token)
        for h, sink in enumerate(data["sinks"]):
            np.testing.assert_allclose(got[token, h], rows.sum(axis=0) / (len(rows) + np.exp(sink)), rtol=1e-5, atol=1e-6)


def test_every_validation_case_selects_real_rows():
    policy = sr.default_policy(B=1, T=1, H=32, D=128, MAX_SEQ=4096, ORI_BLOCKS=32, CMP_BLOCKS=32)
    for case in ("window", "mixed", "padding", "duplicates", "replay", "sink"):
        data = sr.inputs(policy, case)
        rows, _ = sr.selected_rows(data, policy, 0)
        assert len(rows) > 0 and np.any(rows != 0)


def test_patched_cache_reads_like_the_dense_cache():
    policy = sr.default_policy(B=2, T=6, H=2, D=8, MAX_SEQ=512, ORI_BLOCKS=8, CMP_BLOCKS=8, TOPK=16)
    data = sr.inputs(policy, "mixed")
    dense = sr.oracle_fp32(data, policy)
    flat = data["ori_kv"].reshape(-1, 8)
    keep = np.flatnonzero(np.any(flat != 0, axis=1))
    patched = dict(data, ori_kv=sr.PatchedRows(keep, flat[keep]))
    np.testing.assert_array_equal(sr.oracle_fp32(patched, policy), dense)


def test_cpu_reference_matches_oracle():
    policy = sr.default_policy(B=4, T=16, H=4, D=32, MAX_SEQ=1024, ORI_BLOCKS=32, CMP_BLOCKS=32, TOPK=128)
    for case in ("mixed", "ragged", "empty", "duplicates"):
        data = sr.inputs(policy, case)
        tokens = range(policy["T"])
        ref = CpuSparseMla(data, policy, data["q"], tokens).run(chunk=5).numpy()
        np.testing.assert_allclose(ref, sr.oracle_fp32(data, policy), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("ratio", [1, 2])
def test_measurement_inputs_validity_matches_oracle(ratio):
    """The generator's rows equal the oracle's (tests/tooling/test_sparse_performance.py:14-46)."""
    from ascendflow_amd.sparse_attention.inputs import make_metadata, measurement_policy

    policy = measurement_policy(batch=2, query_tokens=5, context=40, max_seq=256, heads=2, features=8, topk=16, ratio=ratio)
    host = make_metadata(policy, 40, seed=11)
    data = dict(host, q=np.zeros((policy["T"], 2, 8), np.float32), ori_kv=np.zeros((policy["ORI_BLOCKS"], 128, 1, 8)),
                cmp_kv=np.zeros((policy["CMP_BLOCKS"], 128 // ratio, 1, 8)), sinks=np.zeros(2, np.float32))
    for token in range(policy["T"]):
        right = 40 - 5 + token % 5 + 1
        chosen = sr.selected_physical(data, policy, token)
        assert len(chosen) == min(128, right) + min(16, right // ratio)
    first = measurement_policy(batch=1, query_tokens=8, context=8, max_seq=128, heads=2, features=8, topk=16, ratio=ratio)
    host = make_metadata(first, 8, seed=3)
    data = dict(host, ori_kv=np.zeros((1, 128, 1, 8)), cmp_kv=np.zeros((1, 128 // ratio, 1, 8)))
    assert len(sr.selected_physical(data, first, 0)) == 1 + (ratio == 1)


def test_lse_closed_forms_zero_query_and_empty_selection():
    """q = 0: every score is 0, so the normaliser is ln(n + e^sink); an empty
    selection leaves the sink alone."""
    rng = np.random.default_rng(3)
    rows = rng.standard_normal((7, 16)).astype(np.float32)
    sinks = np.array([-2.0, 0.0, 1.5], np.float32)
    q = np.zeros((3, 16), np.float32)
    np.testing.assert_allclose(sr.attend_lse(q, rows, sinks, 0.25), np.log(7 + np.exp(sinks.astype(np.float64))),
                               rtol=1e-15)
    np.testing.assert_array_equal(sr.attend_lse(q, np.zeros((0, 16), np.float32), sinks, 0.25), sinks)


def test_lse_is_logsumexp_with_the_sink_as_one_more_column():
    from scipy.special import logsumexp

    rng = np.random.default_rng(4)
    q = rng.standard_normal((4, 32))
    rows = rng.standard_normal((50, 32))
    sinks = rng.standard_normal(4) * 3
    scores = q @ rows.T * 0.3
    expected = logsumexp(np.concatenate([scores, sinks[:, None]], axis=1), axis=1)
    np.testing.assert_allclose(sr.attend_lse(q, rows, sinks, 0.3), expected, rtol=1e-12)


@pytest.mark.parametrize("case", ["mixed", "sink", "empty", "duplicates"])
def test_lse_rebuilds_the_oracle_output(case):
    """attention_out = sum_j exp(s_j - lse) k_j: the normaliser is the
    denominator the oracle divides by."""
    policy = sr.default_policy(B=4, T=16, MAX_SEQ=4096, ORI_BLOCKS=64, CMP_BLOCKS=64, D=128, H=32, BM=32)
    data = sr.inputs(policy, case)
    out = sr.oracle_fp32(data, policy)
    lse = sr.oracle_lse(data, policy)
    for token in range(policy["T"]):
        rows, _ = sr.selected_rows(data, policy, token)
        q = np.asarray(data["q"][token], np.float64)
        if len(rows) == 0:
            np.testing.assert_array_equal(out[token], 0.0)
            continue
        weights = np.exp(q @ rows.astype(np.float64).T * policy["SCALE"] - lse[token][:, None])
        np.testing.assert_allclose(out[token], weights @ rows, rtol=2e-4, atol=2e-6)


@pytest.mark.parametrize("ratio", [1, 2])
@pytest.mark.parametrize("case", sr.CASES)
def test_vectorised_selection_and_plan_images_match_the_oracle(case, ratio):
    """The GPU tests' fast selection images (tests/sparse_helpers.py) equal the
    oracle's per-slot selection: tagged rows in slot order, the debug image,
    and the padded plan lists (first row repeated, or CHUNK zeros when empty)."""
    from tests.sparse_helpers import CHUNK, CMP_BIT, expected_plan, expected_rows, selection_tagged

    policy = sr.default_policy(B=4, T=16, MAX_SEQ=4096, ORI_BLOCKS=64, CMP_BLOCKS=64, RATIO=ratio)
    data = sr.inputs(policy, case)
    tokens = list(range(policy["T"]))
    image = expected_rows(data, policy, tokens)
    counts, lists = expected_plan(data, policy, tokens)
    for token in tokens:
        chosen = sr.selected_physical(data, policy, token)
        tagged = [(CMP_BIT if cache else 0) | row for _, cache, row in chosen]
        assert selection_tagged(data, policy, token).tolist() == tagged
        assert counts[token] == len(chosen)
        assert image[token, : len(chosen)].tolist() == [[cache, row] for _, cache, row in chosen]
        assert (image[token, len(chosen):] == -1).all()
        want = tagged + [tagged[0]] * (-len(tagged) % CHUNK) if tagged else [0] * CHUNK
        assert lists[token].tolist() == want
