"""Vectorised FP32 PyTorch-CPU sparse MLA: the timed CPU baseline (test infrastructure only).

Restates the reference's batched FP32 reference (``benchmarks/attention/sparse_reference.py:141-171``)
on the host CPU instead of an NPU: per chunk of 128 tokens, gather the
selected rows into an FP32 [chunk, S, D] tensor (row selection from the
logical metadata, never from a kernel workspace), ``bmm`` for the scores,
-inf for unused slots, max with the per-head sink, ``exp``, denominator plus
``e^(sink - max)``, ``bmm`` with P kept in FP32, divide.

Its outputs are pinned against ``sparse_reference.oracle_fp32`` in
``tests/test_oracle_sparse.py``.
"""

from __future__ import annotations

import numpy as np
import torch

from .sparse_reference import CMP_BIT, PatchedRows, selection_tagged

# Integer metadata of a sparse call, in the reference entry order.
INT_KEYS = ("cmp_sparse_indices", "ori_block_table", "cmp_block_table", "cu_seqlens_q", "seqused_ori_kv",
            "seqused_cmp_kv", "cmp_residual_kv", "ori_topk_length")


def host_view(inputs, tokens):
    """Oracle data dict of device-built measurement inputs (an object with
    ``policy``, ``host`` int32 metadata, device ``tensors`` and the ``touched``
    rows of each cache): the metadata, the caches as ``PatchedRows`` of their
    touched rows, and the queries of ``tokens`` only (a dict keyed by token)."""
    d = inputs.policy["D"]
    data = {k: inputs.host[k] for k in INT_KEYS}
    data["sinks"] = inputs.tensors["sinks"].float().cpu().numpy()
    for name in ("ori_kv", "cmp_kv"):
        ids = inputs.touched[name]
        flat = inputs.tensors[name].view(-1, d)
        values = (flat[torch.from_numpy(ids).to(flat.device)].float().cpu().numpy() if len(ids)
                  else np.zeros((0, d), np.float32))
        data[name] = PatchedRows(ids, values)
    index = torch.as_tensor(list(tokens), device=inputs.tensors["q"].device, dtype=torch.long)
    rows = inputs.tensors["q"][index].float().cpu().numpy()
    data["q"] = {token: rows[i] for i, token in enumerate(tokens)}
    return data


class CpuSparseMla:
    """Precomputes the row tables; ``run(tokens)`` is the timed part."""

    def __init__(self, data, policy, q_rows, tokens):
        """``q_rows``: FP32 [len(tokens), H, D] queries of ``tokens``."""
        d, s = policy["D"], policy["S"]
        self.policy = policy
        self.tokens = list(tokens)
        tables, offsets = [], []
        for name in ("ori_kv", "cmp_kv"):
            cache = data[name]
            if isinstance(cache, PatchedRows):
                ids, values = cache.rows, cache.values
            else:
                values = np.asarray(cache, np.float32).reshape(-1, d)
                ids = np.arange(len(values), dtype=np.int64)
            offsets.append(sum(len(v) for _, v in tables))
            tables.append((ids, values))
        zero_row = sum(len(v) for _, v in tables)
        self.rows = torch.from_numpy(np.concatenate([v for _, v in tables] + [np.zeros((1, d), np.float32)]))
        # Selected rows are compacted in slot order (window positions, then the
        # valid compressed ranks): the softmax over a set of rows does not
        # depend on where in the gather workspace each one sits.
        index = np.full((len(self.tokens), s), zero_row, np.int64)
        valid = np.zeros((len(self.tokens), s), bool)
        for i, token in enumerate(self.tokens):
            tagged = selection_tagged(data, policy, token)
            for cache in (0, 1):
                which = np.flatnonzero((tagged >> 31) == cache)
                rows = (tagged[which] & (CMP_BIT - 1)).astype(np.int64)
                ids = tables[cache][0]
                at = np.minimum(np.searchsorted(ids, rows), max(len(ids) - 1, 0))
                hit = (ids[at] == rows) if len(ids) else np.zeros(len(rows), bool)
                index[i, which] = np.where(hit, offsets[cache] + at, zero_row)
            valid[i, : len(tagged)] = True
        self.index = torch.from_numpy(index)
        self.valid = torch.from_numpy(valid)
        self.q = torch.from_numpy(np.ascontiguousarray(q_rows, np.float32))
        self.sinks = torch.from_numpy(np.asarray(data["sinks"], np.float32))[None, :]

    @torch.inference_mode()
    def run(self, chunk=128):
        scale = self.policy["SCALE"]
        out = torch.empty_like(self.q)
        for first in range(0, len(self.tokens), chunk):
            last = min(first + chunk, len(self.tokens))
            cache = self.rows[self.index[first:last]]                   # [c, S, D]
            scores = torch.bmm(self.q[first:last], cache.transpose(1, 2)) * scale
            scores.masked_fill_(~self.valid[first:last, None, :], -torch.inf)
            maximum = torch.maximum(scores.amax(dim=-1), self.sinks)
            weight = torch.exp(scores - maximum[:, :, None])
            denominator = weight.sum(dim=-1) + torch.exp(self.sinks - maximum)
            out[first:last] = torch.bmm(weight, cache) / denominator[:, :, None]
        return out
