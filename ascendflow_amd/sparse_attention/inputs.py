"""Seeded long-context sparse-MLA inputs, built on the device.

Counterpart of the reference's measurement-input generator
(``benchmarks/attention/sparse_performance.py:27-82``), used by ``bench.py`` and
the parity tests:

- per-request block tables are a permutation of that request's own pages,
  shared by the raw and the compressed cache;
- ``seqused_ori_kv = context``, ``seqused_cmp_kv = context // R``,
  ``cmp_residual_kv = context % R``, ``ori_topk_length = 0``;
- every token gets ``min(TOPK, right // R)`` sorted compressed indices drawn
  without replacement from its causally valid range ``[0, right // R)``, with
  ``right = context - n + j + 1``;
- the caches are a zero background with values only in the rows some query
  touches (the union of the windows and of the top-k sets of each request), so
  the 12 GiB decode caches need no host copy;
- sinks are ``linspace(-2, 2, H)``.

Values are N(0, 1) * ``scale`` (0.1 for the measured configurations), drawn
with a seeded torch generator on the device and stored in the cache dtype;
index metadata comes from a seeded NumPy generator on the host.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .._tensors import DTYPES


@dataclass
class SparseInputs:
    policy: dict
    context: int
    tensors: dict                 # the 12 input tensors + attention_out, on the device
    host: dict                    # int32 metadata arrays (numpy), same values as the device copies
    touched: dict = field(default_factory=dict)  # cache name -> sorted physical rows holding values

    def call_args(self):
        order = (
            "q", "ori_kv", "cmp_kv", "cmp_sparse_indices", "ori_block_table", "cmp_block_table",
            "cu_seqlens_q", "seqused_ori_kv", "seqused_cmp_kv", "cmp_residual_kv",
            "ori_topk_length", "sinks", "attention_out",
        )
        return [self.tensors[name] for name in order]

    def call_kwargs(self):
        keys = ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS",
                "WINDOW", "TOPK", "S", "BM", "SCALE")
        out = {k: self.policy[k] for k in keys}
        out["DTYPE"] = self.policy["DTYPE"]
        return out


def measurement_policy(batch, query_tokens, context, max_seq=None, heads=64, features=512,
                       topk=512, window=128, ratio=2, page=128, dtype="bf16"):
    """Policy of one measured configuration (``run_sparse.py:50-96`` conventions)."""
    max_seq = context if max_seq is None else max_seq
    max_seq = -(-max_seq // page) * page
    blocks = batch * (max_seq // page)
    return {
        "B": batch,
        "T": batch * query_tokens,
        "H": heads,
        "D": features,
        "PAGE": page,
        "RATIO": ratio,
        "MAX_SEQ": max_seq,
        "ORI_BLOCKS": blocks,
        "CMP_BLOCKS": blocks,
        "WINDOW": window,
        "TOPK": topk,
        "S": window + -(-topk // 512) * 512,
        "BM": min(64, heads),
        "DTYPE": dtype,
        "SCALE": features ** -0.5,
    }


def make_metadata(policy, context, seed, query_lens=None):
    """Host int32 metadata: tables, cu_seqlens, lengths, sorted top-k indices."""
    b, t, topk, page, ratio, max_seq = (policy[k] for k in ("B", "T", "TOPK", "PAGE", "RATIO", "MAX_SEQ"))
    if query_lens is None:
        counts = np.full(b, t // b, np.int32)
        counts[: t % b] += 1
    else:
        counts = np.asarray(query_lens, np.int32)
    if len(counts) != b or int(counts.sum()) != t:
        raise ValueError("query lengths must have B entries summing to T")
    if not int(counts.max()) <= context <= max_seq:
        raise ValueError("context must contain the query tokens and fit MAX_SEQ")
    rng = np.random.default_rng(seed)
    width = max_seq // page
    tables = np.stack([rng.permutation(width) + r * width for r in range(b)]).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    indices = np.full((t, 1, topk), -1, np.int32)
    for r in range(b):
        for offset, token in enumerate(range(cu[r], cu[r + 1])):
            right = context - int(counts[r]) + offset + 1
            count = min(topk, right // ratio)
            if count > 0:
                indices[token, 0, :count] = np.sort(rng.choice(right // ratio, count, replace=False))
    return {
        "cu_seqlens_q": cu,
        "seqused_ori_kv": np.full(b, context, np.int32),
        "seqused_cmp_kv": np.full(b, context // ratio, np.int32),
        "cmp_residual_kv": np.full(b, context % ratio, np.int32),
        "ori_topk_length": np.zeros((t, 1), np.int32),
        "cmp_sparse_indices": indices,
        "ori_block_table": tables,
        "cmp_block_table": tables.copy(),
        "counts": counts,
    }


def touched_rows(policy, context, host):
    """Sorted unique physical rows of each cache that some query reads."""
    page, ratio, window = policy["PAGE"], policy["RATIO"], policy["WINDOW"]
    cpage = page // ratio
    cu, counts, tables = host["cu_seqlens_q"], host["counts"], host["ori_block_table"]
    ori, cmp = [], []
    for r in range(policy["B"]):
        n = int(counts[r])
        if not n:
            continue
        positions = np.arange(max(0, context - n + 1 - window), context, dtype=np.int64)
        ori.append(tables[r, positions // page].astype(np.int64) * page + positions % page)
        idx = np.unique(host["cmp_sparse_indices"][cu[r] : cu[r + 1]].reshape(-1))
        idx = idx[idx >= 0].astype(np.int64)
        cmp.append(host["cmp_block_table"][r, idx // cpage].astype(np.int64) * cpage + idx % cpage)
    cat = lambda parts: np.unique(np.concatenate(parts)) if parts else np.zeros(0, np.int64)
    return {"ori_kv": cat(ori), "cmp_kv": cat(cmp)}


def make_inputs(policy, context, seed=4102026, device="cuda", scale=0.1, query_lens=None):
    """Build one seeded configuration on ``device``; returns ``SparseInputs``."""
    device = torch.device(device)
    b16 = DTYPES[policy["DTYPE"]]
    t, h, d = policy["T"], policy["H"], policy["D"]
    page, ratio = policy["PAGE"], policy["RATIO"]
    host = make_metadata(policy, context, seed, query_lens)
    touched = touched_rows(policy, context, host)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def normal(shape):
        return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * scale).to(b16)

    tensors = {"q": normal((t, h, d))}
    for name, blocks, rows in (("ori_kv", policy["ORI_BLOCKS"], page), ("cmp_kv", policy["CMP_BLOCKS"], page // ratio)):
        cache = torch.zeros((blocks, rows, 1, d), dtype=b16, device=device)
        ids = torch.from_numpy(touched[name]).to(device)
        if ids.numel():
            cache.view(-1, d)[ids] = normal((ids.numel(), d))
        tensors[name] = cache
    for name in ("cmp_sparse_indices", "ori_block_table", "cmp_block_table", "cu_seqlens_q",
                 "seqused_ori_kv", "seqused_cmp_kv", "cmp_residual_kv", "ori_topk_length"):
        tensors[name] = torch.from_numpy(np.ascontiguousarray(host[name])).to(device)
    tensors["sinks"] = torch.linspace(-2.0, 2.0, h, dtype=torch.float32).to(device)
    tensors["attention_out"] = torch.empty((t, h, d), dtype=b16, device=device)
    return SparseInputs(policy=policy, context=context, tensors=tensors, host=host, touched=touched)


def effective_flops(policy, host, context):
    """QK+PV FLOPs with FMA = 2 over valid rows: 4*H*D*sum(valid window + compressed rows)
    (the reference README's convention, README.md:38)."""
    cu, counts = host["cu_seqlens_q"], host["counts"]
    window, ratio = policy["WINDOW"], policy["RATIO"]
    rows = 0
    for r in range(policy["B"]):
        n = int(counts[r])
        for j in range(n):
            right = context - n + j + 1
            rows += min(window, right) + min(policy["TOPK"], right // ratio)
    return 4 * policy["H"] * policy["D"] * rows


def compulsory_bytes(policy, touched):
    """Q + O + indices + unique KV rows touched (the roofline byte basis)."""
    t, h, d, topk = policy["T"], policy["H"], policy["D"], policy["TOPK"]
    qo = 2 * t * h * d * 2
    idx = t * topk * 4
    kv = (len(touched["ori_kv"]) + len(touched["cmp_kv"])) * d * 2
    return qo + idx + kv
