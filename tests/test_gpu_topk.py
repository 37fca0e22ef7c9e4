"""GPU parity of the top-k index selection (launch_sparse_topk_indices).

Bit-exact against the oracle (oracle/topk_reference.py) on ragged requests
with heavy ties and special values, and at the full measured shapes: the
reference's own index distribution (benchmarks/attention/sparse_performance.py:44-47)
recovered from indicator scores for every token, and random scores checked on
sampled tokens against the oracle plus, for every token, the size-independent
properties of the output (ascending, inside the cutoff, the contract's count,
-1 after).
"""

import numpy as np
import pytest
import torch

from ascendflow_amd.sparse_attention import sparse_topk_indices
from ascendflow_amd.sparse_attention.inputs import make_metadata, measurement_policy
from oracle import topk_reference as tr

pytestmark = pytest.mark.gpu

SPECIAL = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.0e38, -3.0e38, 1e-45], np.float32)


def run(device, scores, cu, seq_cmp, residual, topk, ratio, misalign=False):
    """One launch; also checks the 64 guard words after the output. With
    ``misalign`` the score rows start 4 bytes past a 16-byte boundary (the
    kernels' scalar-load path)."""
    to = lambda a, dt: torch.as_tensor(np.ascontiguousarray(a), dtype=dt, device=device)
    t = scores.shape[0]
    buffer = torch.full((t * topk + 64,), 7, dtype=torch.int32, device=device)
    out = buffer[: t * topk].view(t, 1, topk)
    flat = torch.empty(scores.size + 4, dtype=torch.float32, device=device)
    start = 1 if misalign else 0
    dev_scores = flat[start : start + scores.size].view(scores.shape)
    dev_scores.copy_(to(scores, torch.float32))
    assert (dev_scores.data_ptr() % 16 != 0) == misalign
    sparse_topk_indices(dev_scores, to(cu, torch.int32), to(seq_cmp, torch.int32),
                        to(residual, torch.int32), TOPK=topk, RATIO=ratio, out=out)
    torch.cuda.synchronize()
    assert torch.all(buffer[t * topk :] == 7), "write past the output"
    return out.cpu().numpy()


def ragged(rng, b, ratio, max_cmp, max_q=6):
    counts = rng.integers(0, max_q, b).astype(np.int32)
    counts[0] = 0  # an empty request
    counts[-1] = max(1, counts[-1])
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    seq_cmp = rng.integers(0, max_cmp + 1, b).astype(np.int32)
    seq_cmp[1 % b] = max_cmp
    residual = (rng.integers(0, ratio, b) if ratio > 1 else np.zeros(b)).astype(np.int32)
    return cu, seq_cmp, residual


@pytest.mark.parametrize("ratio", [1, 2])
@pytest.mark.parametrize("shape", ["short-rows", "odd-rows", "full-rows", "misaligned", "topk-beyond"])
def test_ragged_tied_and_special_scores_match_the_oracle(device, ratio, shape):
    rng = np.random.default_rng(100 * ratio + len(shape))
    max_cmp = 700
    topk = 1000 if shape == "topk-beyond" else 96
    cu, seq_cmp, residual = ragged(rng, 9, ratio, max_cmp)
    t = int(cu[-1])
    c = {"short-rows": 300, "odd-rows": 301}.get(shape, max_cmp)
    scores = rng.integers(-3, 4, (t, c)).astype(np.float32)
    mask = rng.random((t, c)) < 0.1
    scores[mask] = rng.choice(SPECIAL, int(mask.sum()))
    got = run(device, scores, cu, seq_cmp, residual, topk, ratio, misalign=shape == "misaligned")
    expect = tr.topk_indices(scores, cu, seq_cmp, residual, topk, ratio)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("c", [4096, 5001, 16387, 65536, 262144, 300001])
def test_ties_spanning_many_chunks_match_the_oracle(device, c):
    """Few distinct values: the threshold key is shared by thousands of
    positions, so the equal keys taken are spread over the whole row (and
    more than the filter kernel's buffer reach the estimate). The widths run
    up to the filter kernel's 256K-position limit and past it, where the
    streaming form takes over."""
    rng = np.random.default_rng(c)
    cu = np.array([0, 20, 40], np.int32)
    seq_cmp = np.array([c, c // 2], np.int32)
    residual = np.array([1, 0], np.int32)
    scores = rng.integers(0, 3, (40, c)).astype(np.float32)
    got = run(device, scores, cu, seq_cmp, residual, 512, 2)
    expect = tr.topk_indices(scores, cu, seq_cmp, residual, 512, 2)
    assert np.array_equal(got, expect)


def measured(name):
    shapes = {
        "decode-b64x6-128k": dict(batch=64, query_tokens=6, context=131072),
        "prefill-q8k-32k": dict(batch=1, query_tokens=8192, context=32768),
    }
    policy = measurement_policy(**shapes[name])
    meta = make_metadata(policy, shapes[name]["context"], seed=4102026)
    return policy, meta, shapes[name]["context"]


def generator_bounds(meta, context, ratio):
    """right // R per token, from the generator's own expression (sparse_performance.py:45-46)."""
    counts = meta["counts"]
    bounds = []
    for n in counts:
        bounds.extend(context - int(n) + j + 1 for j in range(int(n)))
    return np.asarray(bounds, np.int64) // ratio


@pytest.mark.parametrize("name", ["decode-b64x6-128k", "prefill-q8k-32k"])
def test_indicator_scores_recover_the_measured_indices(device, name):
    policy, meta, context = measured(name)
    t, ratio, topk = policy["T"], policy["RATIO"], policy["TOPK"]
    c = context // ratio
    gen = torch.Generator(device=device).manual_seed(7)
    scores = torch.rand((t, c), generator=gen, device=device) * 1.99 - 1.0
    indices = torch.as_tensor(meta["cmp_sparse_indices"], device=device).view(t, topk).long()
    valid = indices >= 0
    rows = torch.arange(t, device=device)[:, None].expand_as(indices)
    scores[rows[valid], indices[valid]] = 1.5 + torch.rand(int(valid.sum()), generator=gen, device=device)
    bound = torch.as_tensor(generator_bounds(meta, context, ratio), device=device)
    scores[torch.arange(c, device=device)[None, :] >= bound[:, None]] = 5.0
    args = [torch.as_tensor(meta[k], device=device) for k in ("cu_seqlens_q", "seqused_cmp_kv", "cmp_residual_kv")]
    got = sparse_topk_indices(scores, *args, TOPK=topk, RATIO=ratio)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.as_tensor(meta["cmp_sparse_indices"]))
    # The framework op runs the same kernel.
    via_op = torch.ops.ascendflow_amd.sparse_topk_indices(scores, *args, topk, ratio)
    assert torch.equal(via_op, got)


@pytest.mark.parametrize("name", ["decode-b64x6-128k", "prefill-q8k-32k"])
def test_random_scores_at_full_size(device, name):
    policy, meta, context = measured(name)
    t, ratio, topk = policy["T"], policy["RATIO"], policy["TOPK"]
    c = context // ratio
    gen = torch.Generator(device=device).manual_seed(11)
    # b16-rounded normals: ties occur, as with scores stored in b16.
    scores = torch.randn((t, c), generator=gen, device=device).to(torch.bfloat16).float()
    args = [torch.as_tensor(meta[k], device=device) for k in ("cu_seqlens_q", "seqused_cmp_kv", "cmp_residual_kv")]
    got = sparse_topk_indices(scores, *args, TOPK=topk, RATIO=ratio)
    torch.cuda.synchronize()
    # Every token: ascending inside the cutoff, the contract's count, then -1.
    cutoff, bound = tr.token_bounds(meta["cu_seqlens_q"], meta["seqused_cmp_kv"], meta["cmp_residual_kv"], ratio)
    take = torch.as_tensor(np.minimum(np.minimum(topk, bound), np.minimum(cutoff, c)), device=device)
    flat = got.view(t, topk).long()
    slots = torch.arange(topk, device=device)[None, :]
    used = slots < take[:, None]
    assert torch.all(flat[~used] == -1)
    assert torch.all((flat >= 0) == used)
    assert torch.all(flat < torch.as_tensor(cutoff, device=device)[:, None])
    steps = flat[:, 1:] - flat[:, :-1]
    assert torch.all((steps > 0) | ~used[:, 1:])
    # Sampled tokens, bit-exact against the oracle (first, last, and spread):
    # each as a one-query request whose cutoff is the token's own.
    sample = np.unique(np.r_[0, 1, 5, t - 1, np.linspace(0, t - 1, 40).astype(int)])
    for token in sample:
        row = scores[token : token + 1].cpu().numpy()
        alone = np.array([cutoff[token]], np.int32)
        expect = tr.topk_indices(row, np.array([0, 1], np.int32), alone, np.array([0], np.int32), topk, 1)
        assert np.array_equal(got[token].cpu().numpy(), expect[0]), f"token {token}"


@pytest.mark.parametrize("c", [1000, 16384, 65536])
@pytest.mark.parametrize("case", ["estimate-holds", "estimate-refiltered", "estimate-too-high", "buffer-overflow"])
def test_estimate_fallbacks(device, c, case):
    """The filter kernel (256 threads up to 32K positions, 1024 beyond)
    estimates the threshold from S sampled keys, 4 per thread of 256 (1024)
    or 2 per thread of 1024 (2048); the whole row when shorter: sample i in
    block i // 16 of 16 consecutive positions, block b starting at
    floor(b c / (S / 16)), and selects from the keys that reach it.
    When fewer than TOPK reach it, or more than its LDS buffer holds (2 TOPK
    entries within [1024, 8192] up to 32K positions, 4096 beyond), it filters again at another sample rank (binary search,
    up to four passes), then selects from the whole row. Large scores on a
    32nd of the sampled positions need further passes; on all of them the
    estimate stays too high once TOPK exceeds the sample; a TOPK of 9000
    overflows the buffer. Every outcome must select the same."""
    full = 4 * 256 if c <= 32768 else 2 * 1024
    samples = min(full, c)
    topk = {"estimate-holds": samples // 4 - 12, "estimate-refiltered": samples // 32 + 40,
            "estimate-too-high": samples + 88, "buffer-overflow": 9000}[case]
    i = np.arange(samples)
    sampled = i if samples < full else (i // 16) * c // (samples // 16) + i % 16
    scores = np.random.default_rng(c + topk).normal(size=(2, c)).astype(np.float32)
    scores[0, sampled[::32] if case == "estimate-refiltered" else sampled] = 10.0
    cu = np.array([0, 2], np.int32)
    seq_cmp, residual = np.array([c], np.int32), np.array([0], np.int32)
    got = run(device, scores, cu, seq_cmp, residual, topk, 1)
    expect = tr.topk_indices(scores, cu, seq_cmp, residual, topk, 1)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("topk", [2048, 4000])
def test_large_topk_matches_the_oracle(device, topk):
    """Rows up to 32K positions size the filter buffer to 2 TOPK entries (up to
    8192), so large selections stay on the buffered path."""
    rng = np.random.default_rng(topk)
    c = 16384
    cu = np.array([0, 24, 48], np.int32)
    seq_cmp, residual = np.array([c, c // 2 + 1000], np.int32), np.array([1, 0], np.int32)
    scores = rng.normal(size=(48, c)).astype(np.float32)
    got = run(device, scores, cu, seq_cmp, residual, topk, 2)
    expect = tr.topk_indices(scores, cu, seq_cmp, residual, topk, 2)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("topk", [4097, 8192])
def test_topk_beyond_the_wide_buffer_matches_the_oracle(device, topk):
    """Rows over 32K positions run the 1024-thread form, whose filter buffer
    holds 4096 entries: a selection of more than that goes straight to the
    whole-row selection (no filter pass can hold it). Ties and a request whose
    cutoff leaves fewer candidates than TOPK are included."""
    rng = np.random.default_rng(topk)
    c = 40000
    cu = np.array([0, 5, 9], np.int32)
    seq_cmp, residual = np.array([c, 6000], np.int32), np.array([1, 0], np.int32)
    scores = rng.normal(size=(9, c)).astype(np.float32)
    scores[1, ::7] = 1.5  # a block of equal keys around the threshold
    scores[2] = np.round(scores[2] * 4) / 4
    got = run(device, scores, cu, seq_cmp, residual, topk, 2)
    expect = tr.topk_indices(scores, cu, seq_cmp, residual, topk, 2)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("c,topk", [(1, 1), (3, 2), (4, 1), (7, 16), (33, 33)])
def test_tiny_rows_many_empty_requests(device, c, topk):
    """Rows of 1-33 positions (the scalar and the 16-byte load paths), TOPK 1
    and TOPK equal to the row, 40 requests of which most are empty, and a
    request holding a single token."""
    rng = np.random.default_rng(c * 100 + topk)
    counts = np.zeros(40, np.int32)
    counts[[3, 17, 18, 39]] = (2, 1, 3, 1)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    seq_cmp = rng.integers(0, c + 1, 40).astype(np.int32)
    residual = rng.integers(0, 2, 40).astype(np.int32)
    t = int(cu[-1])
    scores = rng.integers(-2, 3, (t, c)).astype(np.float32)
    for ratio in (1, 2):
        got = run(device, scores, cu, seq_cmp, residual if ratio == 2 else np.zeros_like(residual), topk, ratio)
        expect = tr.topk_indices(scores, cu, seq_cmp, residual if ratio == 2 else np.zeros_like(residual), topk, ratio)
        assert np.array_equal(got, expect), ratio


@pytest.mark.parametrize("c,b", [(700, 255), (700, 300), (40000, 1023), (40000, 1100)])
def test_requests_up_to_and_beyond_one_per_thread(device, c, b):
    """Request lookup with B just under and over the workgroup's thread count
    (256 threads up to 32K positions, 1024 beyond): one cu entry per thread,
    or every thread counting a strided share and one thread reading the
    request's values. Most requests are empty; tokens sit in the first, the
    last and a few requests between."""
    rng = np.random.default_rng(c + b)
    counts = np.zeros(b, np.int32)
    counts[[0, 1, b // 2, b // 2 + 1, b - 2, b - 1]] = (2, 0, 3, 1, 0, 2)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    seq_cmp = rng.integers(c // 2, c + 1, b).astype(np.int32)
    residual = rng.integers(0, 2, b).astype(np.int32)
    t = int(cu[-1])
    scores = rng.integers(-50, 50, (t, c)).astype(np.float32)
    got = run(device, scores, cu, seq_cmp, residual, 64, 2)
    assert np.array_equal(got, tr.topk_indices(scores, cu, seq_cmp, residual, 64, 2))


@pytest.mark.parametrize("ratio", [1, 2])
def test_selected_indices_drive_sparse_mla(device, ratio):
    """The chain the top-k step serves: index scores -> sparse_topk_indices ->
    sparse_mla. The indices the kernel selects meet the operator's input
    contract, so the attention over them matches the oracle run on the same
    indices (rows bit-exact through the operator's own selection image)."""
    from ascendflow_amd.sparse_attention import sparse_mla
    from oracle import sparse_reference as sr
    from tests.sparse_helpers import assert_close, call_args, call_kwargs, expected_rows, to_device

    policy = sr.default_policy(B=3, T=12, RATIO=ratio, MAX_SEQ=2048, ORI_BLOCKS=48, CMP_BLOCKS=48)
    data = sr.inputs(policy, "ragged")
    t, c = policy["T"], policy["MAX_SEQ"] // ratio
    scores = np.random.default_rng(ratio).normal(size=(t, c)).astype(np.float32)
    meta = {k: torch.as_tensor(data[k], device=device) for k in ("cu_seqlens_q", "seqused_cmp_kv", "cmp_residual_kv")}
    indices = sparse_topk_indices(torch.as_tensor(scores, device=device), meta["cu_seqlens_q"], meta["seqused_cmp_kv"],
                                  meta["cmp_residual_kv"], TOPK=policy["TOPK"], RATIO=ratio)
    torch.cuda.synchronize()
    data["cmp_sparse_indices"] = indices.cpu().numpy()
    assert np.array_equal(data["cmp_sparse_indices"],
                          tr.topk_indices(scores, data["cu_seqlens_q"], data["seqused_cmp_kv"], data["cmp_residual_kv"],
                                          policy["TOPK"], ratio))
    tensors = to_device(data, policy, device)
    debug = torch.empty((t, policy["S"], 2), dtype=torch.int32, device=device)
    sparse_mla(*call_args(tensors), **call_kwargs(policy), debug_rows=debug)
    torch.cuda.synchronize()
    assert np.array_equal(debug.cpu().numpy(), expected_rows(data, policy, list(range(t))))
    assert_close(tensors["attention_out"].float().cpu().numpy(), sr.oracle_fp32(data, policy), policy["DTYPE"])
