"""Sparse-MLA oracle: TND queries over PA_BBND paged caches (test infrastructure only).

Restates the reference's independent CPU semantics:

- ``query_geometry``  <- ``benchmarks/attention/sparse_reference.py:29-42`` and the
  device-side ``query_metadata`` (``examples/sparse_attention/gather.py:8-35``):
  ``batch = upper_bound(cu, t) - 1``, ``right = max(0, L - n + j + 1)``,
  ``visible = min(WINDOW, right)`` narrowed by a positive ``ori_topk_length``,
  ``cutoff = max(0, C*R + r - n + j + 1) // R``.
- ``selected_rows``   <- ``sparse_reference.py:107-124`` and ``gather_compressed``
  (``gather.py:86-131``): window positions ``[right-visible, right)`` then the
  compressed ranks ``< min(TOPK, C, cutoff)`` whose index is in ``[0, cutoff)``.
  The device kernel tests every rank on its own (``gather.py:116-127``); the
  reference oracle stops at the first negative index (``sparse_reference.py:117``).
  Under the input contract (non-negative prefix, then -1 padding;
  ``docs/operators/sparse-mla.md:79``) both agree; this restatement follows the
  per-rank device rule.
- ``gather_oracle``   <- ``sparse_reference.py:174-181`` (slot layout of the gather
  workspace: window slot ``i``, compressed slot ``WINDOW + rank``, bias 0 / -inf).
- ``oracle``          <- ``sparse_reference.py:127-138`` (FP32 softmax with one sink per
  head in the denominator, output rounded to the storage dtype).
- ``oracle_lse``      the natural-log softmax normaliser ln(sum_j e^(s_j) + e^sink) per
  (token, head): the ``softmax_lse`` output of the vendor operator the reference
  benchmarks against (``benchmarks/references/sparse_mla_aclnn.py:100-130``), i.e. the
  denominator ``oracle`` divides by. The reference's own kernel has no LSE output, so
  this is pinned by closed forms (q = 0 gives ln(n + e^sink), an empty selection gives
  the sink), by scipy's logsumexp over the scores with the sink as one more column, and
  by rebuilding ``oracle_fp32`` from it.
- ``inputs``          <- ``sparse_reference.py:45-104`` (the eight validation cases),
  written independently with this repository's own seed use.

Pinned by ``tests/test_oracle_sparse.py``: the reference's known-answer fixture
(``tests/operators/test_sparse_attention.py:14-129``), closed forms (q=0 and
sink=0 gives the mean over rows plus one sink; empty selection gives zeros;
uniform scores give the mean), brute force of the geometry against the
documented formulas, and the measurement-input validity mask
(``tests/tooling/test_sparse_performance.py:14-46``).
"""

from __future__ import annotations

import numpy as np

from .dtypes import rounded

CASES = ("empty", "window", "mixed", "ragged", "padding", "duplicates", "replay", "sink")

# Shapes of the thirteen external tensors, in the reference entry order
# (examples/sparse_attention/attention.py:211-224).
TENSOR_ORDER = (
    "q",
    "ori_kv",
    "cmp_kv",
    "cmp_sparse_indices",
    "ori_block_table",
    "cmp_block_table",
    "cu_seqlens_q",
    "seqused_ori_kv",
    "seqused_cmp_kv",
    "cmp_residual_kv",
    "ori_topk_length",
    "sinks",
    "attention_out",
)


def default_policy(**overrides):
    """Reference defaults (``examples/sparse_attention/attention.py:225-245``)."""
    policy = {
        "B": 4,
        "T": 16,
        "H": 64,
        "D": 512,
        "PAGE": 128,
        "RATIO": 2,
        "MAX_SEQ": 4096,
        "ORI_BLOCKS": 128,
        "CMP_BLOCKS": 128,
        "WINDOW": 128,
        "TOPK": 512,
        "S": 640,
        "BM": 64,
        "DTYPE": "bf16",
        "SCALE": 0.04419417382415922,
    }
    policy.update(overrides)
    if "S" not in overrides:
        policy["S"] = policy["WINDOW"] + -(-policy["TOPK"] // 512) * 512
    return policy


def query_geometry(data, policy, token):
    """(batch, right, visible, available, cutoff) of one query token."""
    cu = np.asarray(data["cu_seqlens_q"])
    batch = int(np.searchsorted(cu, token, side="right")) - 1
    count = int(cu[batch + 1]) - int(cu[batch])
    offset = token - int(cu[batch])
    right = max(0, int(data["seqused_ori_kv"][batch]) - count + offset + 1)
    visible = min(policy["WINDOW"], right)
    narrowed = int(data["ori_topk_length"][token, 0])
    if narrowed > 0:
        visible = min(visible, narrowed)
    available = int(data["seqused_cmp_kv"][batch])
    ratio = policy["RATIO"]
    end = available * ratio + int(data["cmp_residual_kv"][batch])
    cutoff = max(0, end - count + offset + 1) // ratio
    return batch, right, visible, available, cutoff


def selected_physical(data, policy, token):
    """Ordered selection of one token as (slot, cache, physical_row).

    ``cache`` is 0 for ``ori_kv`` and 1 for ``cmp_kv``; ``physical_row`` is the
    flattened ``block * page_rows + row`` index into that cache.
    """
    page = policy["PAGE"]
    cpage = page // policy["RATIO"]
    batch, right, visible, available, cutoff = query_geometry(data, policy, token)
    out = []
    for slot in range(visible):
        position = right - visible + slot
        block = int(data["ori_block_table"][batch, position // page])
        out.append((slot, 0, block * page + position % page))
    bound = min(policy["TOPK"], available, cutoff)
    for rank in range(bound):
        index = int(data["cmp_sparse_indices"][token, 0, rank])
        if 0 <= index < cutoff:
            block = int(data["cmp_block_table"][batch, index // cpage])
            out.append((policy["WINDOW"] + rank, 1, block * cpage + index % cpage))
    return out


CMP_BIT = 1 << 31  # tag of a cmp_kv row in a tagged row id


def selection_tagged(data, policy, token):
    """``selected_physical`` of one token as tagged uint32 row ids in slot order
    (bit 31 set for a cmp_kv row), vectorised with NumPy: the same geometry
    and the same per-rank rule. Pinned against ``selected_physical`` on every
    validation case."""
    page = policy["PAGE"]
    cpage = page // policy["RATIO"]
    batch, right, visible, available, cutoff = query_geometry(data, policy, token)
    positions = np.arange(right - visible, right, dtype=np.int64)
    window = np.asarray(data["ori_block_table"])[batch, positions // page].astype(np.int64) * page + positions % page
    bound = min(policy["TOPK"], available, cutoff)
    index = np.asarray(data["cmp_sparse_indices"])[token, 0, : max(bound, 0)].astype(np.int64)
    index = index[(index >= 0) & (index < cutoff)]
    compressed = np.asarray(data["cmp_block_table"])[batch, index // cpage].astype(np.int64) * cpage + index % cpage
    return np.concatenate([window, compressed | CMP_BIT]).astype(np.uint32)


class PatchedRows:
    """A cache that is zero except for listed rows (the measurement caches).

    ``rows`` are sorted flattened physical row ids, ``values`` their FP32 rows.
    Indexing with a physical row returns that row or zeros, like the dense
    cache the device reads.
    """

    def __init__(self, rows, values):
        self.rows = np.asarray(rows, np.int64)
        self.values = np.asarray(values, np.float32)
        if len(self.rows) != len(self.values) or np.any(np.diff(self.rows) <= 0):
            raise ValueError("PatchedRows needs sorted unique rows with one value row each")

    def __getitem__(self, row):
        at = int(np.searchsorted(self.rows, row))
        if at < len(self.rows) and self.rows[at] == row:
            return self.values[at]
        return np.zeros(self.values.shape[1], np.float32)


def _cache_rows(cache, d):
    return cache if isinstance(cache, PatchedRows) else np.asarray(cache).reshape(-1, d)


def selected_rows(data, policy, token):
    """FP32 rows [n, D] and their gather slots for one token."""
    d = policy["D"]
    caches = (_cache_rows(data["ori_kv"], d), _cache_rows(data["cmp_kv"], d))
    chosen = selected_physical(data, policy, token)
    if not chosen:
        return np.zeros((0, d), np.float32), []
    rows = np.stack([caches[cache][row] for _, cache, row in chosen]).astype(np.float32)
    return rows, [slot for slot, _, _ in chosen]


def attend(q_token, rows, sinks, scale):
    """FP32 softmax-with-sink attention of one token: [H, D] x [n, D] -> [H, D]."""
    q_token = np.asarray(q_token, np.float32)
    if len(rows) == 0:
        return np.zeros_like(q_token)
    scores = (q_token @ rows.T) * np.float32(scale)
    maximum = np.maximum(scores.max(axis=1), sinks)
    weights = np.exp(scores - maximum[:, None])
    denominator = weights.sum(axis=1) + np.exp(sinks - maximum)
    return (weights @ rows) / denominator[:, None]


def attend_lse(q_token, rows, sinks, scale):
    """Natural-log softmax normaliser of one token, float64 [H]:
    ln(sum_j exp(scale * q.k_j) + exp(sink)), the sink alone when nothing is selected."""
    sinks = np.asarray(sinks, np.float64)
    if len(rows) == 0:
        return sinks.copy()
    scores = (np.asarray(q_token, np.float64) @ np.asarray(rows, np.float64).T) * float(scale)
    maximum = np.maximum(scores.max(axis=1), sinks)
    return maximum + np.log(np.exp(scores - maximum[:, None]).sum(axis=1) + np.exp(sinks - maximum))


def oracle_lse(data, policy, tokens=None):
    """Softmax normaliser [len(tokens), H] in float64 (all tokens by default)."""
    tokens = range(policy["T"]) if tokens is None else tokens
    out = []
    for token in tokens:
        rows, _ = selected_rows(data, policy, token)
        out.append(attend_lse(data["q"][token], rows, data["sinks"], policy["SCALE"]))
    return np.stack(out)


def oracle_fp32(data, policy, tokens=None):
    """Unrounded FP32 outputs [len(tokens), H, D] (all tokens by default)."""
    tokens = range(policy["T"]) if tokens is None else tokens
    sinks = np.asarray(data["sinks"], np.float32)
    out = []
    for token in tokens:
        rows, _ = selected_rows(data, policy, token)
        out.append(attend(data["q"][token], rows, sinks, policy["SCALE"]))
    return np.stack(out).astype(np.float32)


def oracle(data, policy, tokens=None):
    """Output rounded to the storage dtype (``sparse_reference.py:127-138``)."""
    return rounded(oracle_fp32(data, policy, tokens), policy["DTYPE"])


def gather_oracle(data, policy, tokens=None):
    """Gather-workspace image: rows [n, S, D] (zero when unused) and bias [n, S]."""
    tokens = range(policy["T"]) if tokens is None else list(tokens)
    s, d = policy["S"], policy["D"]
    kv = np.zeros((len(tokens), s, d), np.float32)
    bias = np.full((len(tokens), s), -np.inf, np.float32)
    for i, token in enumerate(tokens):
        rows, slots = selected_rows(data, policy, token)
        if slots:
            kv[i, slots] = rows
            bias[i, slots] = 0.0
    return kv, bias


def query_counts(policy, ragged=False):
    """Per-request query counts: T spread over B, optionally ragged with an empty request."""
    b, t = policy["B"], policy["T"]
    counts = np.full(b, t // b, np.int32)
    counts[: t % b] += 1
    if ragged and b >= 3 and t >= 3:
        first = int(counts[:3].sum())
        counts[:3] = (0, first // 3, first - first // 3)
    return counts


def inputs(policy, case, query_lens=None, seed=4102026, scale=0.5):
    """Seeded validation inputs for one of ``CASES`` (values are b16-exact FP32)."""
    if case not in CASES:
        raise ValueError(f"unknown sparse attention case: {case}")
    b, t, h, d = policy["B"], policy["T"], policy["H"], policy["D"]
    page, ratio, max_seq, topk = policy["PAGE"], policy["RATIO"], policy["MAX_SEQ"], policy["TOPK"]
    dtype = policy["DTYPE"]
    rng = np.random.default_rng(seed)
    counts = (
        query_counts(policy, case == "ragged")
        if query_lens is None
        else np.asarray(query_lens, np.int32)
    )
    if len(counts) != b or int(counts.sum()) != t:
        raise ValueError("query lengths must have B entries summing to T")
    # Cache lengths cycle through page-edge cases and the full capacity.
    pattern = np.array([page - 1, page + 1, 2 * page + 1, max_seq - 1])
    lengths = np.resize(pattern, b)
    lengths = np.minimum(max_seq, np.maximum(counts, lengths)).astype(np.int32)
    if case == "empty":
        lengths[:] = 0

    def normal(shape):
        return rounded(rng.normal(0.0, scale, shape).astype(np.float32), dtype)

    data = {
        "q": normal((t, h, d)),
        "ori_kv": normal((policy["ORI_BLOCKS"], page, 1, d)),
        "cmp_kv": normal((policy["CMP_BLOCKS"], page // ratio, 1, d)),
        "cu_seqlens_q": np.concatenate([[0], np.cumsum(counts)]).astype(np.int32),
        "seqused_ori_kv": lengths,
        "seqused_cmp_kv": (lengths // ratio).astype(np.int32),
        "cmp_residual_kv": (lengths % ratio).astype(np.int32),
        "ori_topk_length": np.zeros((t, 1), np.int32),
        "cmp_sparse_indices": np.full((t, 1, topk), -1, np.int32),
        "sinks": np.linspace(-2.0, 2.0, h, dtype=np.float32),
    }
    # Page tables may share read-only physical pages across requests.
    data["ori_block_table"] = rng.integers(
        0, policy["ORI_BLOCKS"], (b, max_seq // page), dtype=np.int32
    )
    data["cmp_block_table"] = rng.integers(
        0, policy["CMP_BLOCKS"], (b, max_seq // page), dtype=np.int32
    )
    for token in range(t):
        _, _, _, available, cutoff = query_geometry(data, policy, token)
        count = min(topk, available, cutoff)
        if case not in ("empty", "window") and count > 0:
            if case == "padding":
                count = token % (count + 1)
            chosen = rng.permutation(available)[:count].astype(np.int32)
            if case == "duplicates":
                chosen[:] = 0
            elif case == "mixed" and count:
                # A future compressed entry: early tokens must filter it out.
                chosen[0] = available - 1
            data["cmp_sparse_indices"][token, 0, :count] = chosen
        if case == "replay" and token % 3 != 2:
            data["ori_topk_length"][token, 0] = 1 + token % 7
    if case == "sink":
        data["sinks"][:] = np.resize(np.array([-80.0, 80.0, 0.0, 5.0], np.float32), h)
    return data
