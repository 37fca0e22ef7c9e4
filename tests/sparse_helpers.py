"""Helpers shared by the sparse-MLA GPU tests: device copies of oracle inputs,
host views of device-built inputs, guard bytes and the tolerance contract."""

from __future__ import annotations

import numpy as np
import torch

from oracle import sparse_reference as sr
from oracle.cpu_reference import INT_KEYS, host_view  # noqa: F401  (re-exported for the tests)
from oracle.dtypes import rounded

TORCH_DTYPE = {"bf16": torch.bfloat16, "f16": torch.float16}
GUARD_WORDS = 256  # 512 guard bytes after the output (benchmarks/attention/run_sparse.py:31)


def to_device(data, policy, device):
    """Device tensors of an oracle input dict, plus a guarded output."""
    b16 = TORCH_DTYPE[policy["DTYPE"]]
    out = {name: torch.from_numpy(np.ascontiguousarray(data[name], np.float32)).to(device=device, dtype=b16)
           for name in ("q", "ori_kv", "cmp_kv")}
    for name in INT_KEYS:
        out[name] = torch.from_numpy(np.ascontiguousarray(data[name], np.int32)).to(device)
    out["sinks"] = torch.from_numpy(np.ascontiguousarray(data["sinks"], np.float32)).to(device)
    t, h, d = policy["T"], policy["H"], policy["D"]
    guarded = torch.full((t * h * d + GUARD_WORDS,), float("nan"), dtype=b16, device=device)
    out["_guarded"] = guarded
    out["attention_out"] = guarded[: t * h * d].view(t, h, d)
    return out


def call_args(tensors):
    return [tensors[name] for name in sr.TENSOR_ORDER]


def call_kwargs(policy):
    keys = ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS", "WINDOW", "TOPK", "S", "BM", "SCALE")
    return dict({k: policy[k] for k in keys}, DTYPE=policy["DTYPE"])


def guard_intact(tensors):
    tail = tensors["_guarded"][-GUARD_WORDS:]
    return bool(torch.isnan(tail.float()).all())


CMP_BIT = sr.CMP_BIT  # row-list tag of a cmp_kv row
CHUNK = 32            # rows per streamed chunk
selection_tagged = sr.selection_tagged


def expected_rows(data, policy, tokens):
    """Oracle selection as the kernel's debug image: int32 [n, S, 2], entry r
    the r-th selected row (cache, physical row) in slot order, then (-1, -1)."""
    img = np.full((len(tokens), policy["S"], 2), -1, np.int32)
    for i, token in enumerate(tokens):
        tagged = selection_tagged(data, policy, token)
        img[i, : len(tagged), 0] = (tagged >> 31).astype(np.int32)
        img[i, : len(tagged), 1] = (tagged & (CMP_BIT - 1)).astype(np.int32)
    return img


def expected_plan(data, policy, tokens):
    """Oracle selection as the plan workspace holds it: counts [n] and the
    tagged lists, padded with the first row to whole chunks ([CHUNK] zeros
    for an empty selection), as a list of uint32 arrays."""
    counts, lists = [], []
    for token in tokens:
        tagged = selection_tagged(data, policy, token)
        counts.append(len(tagged))
        if len(tagged):
            padded = -(-len(tagged) // CHUNK) * CHUNK
            lists.append(np.concatenate([tagged, np.full(padded - len(tagged), tagged[0], np.uint32)]))
        else:
            lists.append(np.zeros(CHUNK, np.uint32))
    return np.array(counts, np.int32), lists


def plan_from_workspace(workspace, policy):
    """Counts [T] and the full list table [T, entries] (uint32) read back from a workspace."""
    from ascendflow_amd.sparse_attention.attention import plan_layout

    t = policy["T"]
    count_at, rows_at, entries = plan_layout(t, policy["WINDOW"], policy["TOPK"])
    raw = workspace.cpu().numpy()
    counts = raw[count_at : count_at + 4 * t].view(np.int32)
    table = raw[rows_at : rows_at + 4 * t * entries].view(np.uint32).reshape(t, entries)
    return counts, table


def assert_plan_matches(workspace, data, policy, tokens):
    """Bit-exact: the plan the persistent kernel streamed equals the oracle's
    selection, compacted and padded, for every token in ``tokens``."""
    counts, table = plan_from_workspace(workspace, policy)
    want_counts, want_lists = expected_plan(data, policy, tokens)
    np.testing.assert_array_equal(counts[list(tokens)], want_counts)
    for token, want in zip(tokens, want_lists):
        got = table[token, : len(want)]
        if not np.array_equal(got, want):
            bad = int(np.flatnonzero(got != want)[0])
            raise AssertionError(f"plan list of token {token} differs at entry {bad}: {got[bad]:#x} != {want[bad]:#x}")


def assert_close(actual, ref_fp32, dtype):
    """Tolerance contract: max|err| <= 1e-2 * max|ref| (BASELINE) and the
    reference runner's allclose(rtol=0.02, atol=0.005) (run_sparse.py:32)."""
    actual = np.asarray(actual, np.float32)
    ref = np.asarray(ref_fp32, np.float32)
    assert np.isfinite(actual).all(), "non-finite output"
    err = float(np.max(np.abs(actual - ref))) if ref.size else 0.0
    bound = 1e-2 * float(np.max(np.abs(ref))) if ref.size else 0.0
    assert err <= max(bound, 1e-6), f"max|err| {err:.3g} > 1e-2 * max|ref| = {bound:.3g}"
    np.testing.assert_allclose(actual, rounded(ref, dtype), rtol=0.02, atol=0.005)
    return err, bound
