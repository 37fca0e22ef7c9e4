"""Row-list plan and gather probe (measurement helpers around the sparse path).

``sparse_mla_plan`` runs only the plan kernel of ``launch_sparse_mla`` and
returns its workspace (per-token selected-row counts and tagged row lists,
layout in ``include/ascendflow_amd.h``), which
``ascendflow_amd.sparse_attention.sparse_mla_planned`` then attends over. ``gather_probe`` streams those rows
through LDS the way the attention kernels do, with no compute, at a chosen
number of chunks in flight: the counterpart of the reference's standalone
gather micro-benchmark (``benchmarks/attention/gather_dma.py``), used to
measure what the sparse access pattern itself can reach.
"""

from __future__ import annotations

import ctypes as ct

import torch

from .. import _native
from .._tensors import require, storage_dtype, stream_handle
from .attention import make_params

PROBE_ROWS = 16  # rows per probe chunk


def _params(policy):
    keys = ("B", "T", "H", "D", "PAGE", "RATIO", "MAX_SEQ", "ORI_BLOCKS", "CMP_BLOCKS", "WINDOW", "TOPK", "S", "BM")
    return make_params(*(policy[k] for k in keys), storage_dtype(policy["DTYPE"]), policy["SCALE"], parts=1)


def sparse_mla_plan(tensors, policy, workspace=None):
    """The row-list plan of one call (a uint8 workspace tensor, allocated
    unless given) for the metadata in ``tensors``."""
    params = _params(policy)
    t = policy["T"]
    entries = -(-(policy["WINDOW"] + policy["TOPK"]) // 256) * 256
    nbytes = -(-4 * t // 256) * 256 + 4 * t * entries
    device = tensors["cmp_sparse_indices"].device
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
    require(workspace.dtype == torch.uint8 and workspace.is_contiguous() and workspace.numel() >= nbytes
            and workspace.device == device, "workspace must be a contiguous uint8 tensor holding the plan")
    names = ("cmp_sparse_indices", "ori_block_table", "cmp_block_table", "cu_seqlens_q", "seqused_ori_kv",
             "seqused_cmp_kv", "cmp_residual_kv", "ori_topk_length")
    status = _native.library().launch_sparse_mla_plan(stream_handle(device), *(tensors[n].data_ptr() for n in names),
                                                      workspace.data_ptr(), ct.byref(params))
    _native.check(status, "launch_sparse_mla_plan")
    return workspace


def gather_probe(tensors, policy, workspace, grid, depth, balanced=False, sums=None):
    """Launches the gather probe over the plan in ``workspace``; returns the
    int32 view of its per-thread sums [grid, 16] (uint32 values)."""
    require(depth in (1, 2, 4, 6, 8), "probe depth must be 1, 2, 4, 6 or 8 chunks")
    device = workspace.device
    if sums is None:
        sums = torch.empty((grid, PROBE_ROWS), dtype=torch.int32, device=device)
    params = _params(policy)
    status = _native.library().launch_gather_probe(stream_handle(device), tensors["ori_kv"].data_ptr(),
                                                   tensors["cmp_kv"].data_ptr(), workspace.data_ptr(), ct.byref(params),
                                                   grid, depth, int(bool(balanced)), sums.data_ptr())
    _native.check(status, "launch_gather_probe")
    return sums


def expected_probe_sum(tensors, policy, workspace):
    """Sum (mod 2^32) of the first dword of every row the probe streams: each
    token's first max(1, ceil(count / 16)) * 16 plan entries, computed with torch."""
    t, d = policy["T"], policy["D"]
    entries = -(-(policy["WINDOW"] + policy["TOPK"]) // 256) * 256
    rows_at = -(-4 * t // 256) * 256
    counts = workspace[: 4 * t].view(torch.int32).long()
    lists = workspace[rows_at : rows_at + 4 * t * entries].view(torch.int32).view(t, entries).long() & 0xFFFFFFFF
    chunks = torch.clamp((counts + PROBE_ROWS - 1) // PROBE_ROWS, min=1)
    used = torch.arange(entries, device=workspace.device)[None, :] < (chunks * PROBE_ROWS)[:, None]
    tags = lists[used]
    is_cmp = (tags >> 31) == 1
    row = tags & 0x7FFFFFFF
    first = {}
    for name in ("ori_kv", "cmp_kv"):
        flat = tensors[name].view(-1, d)
        first[name] = flat[:, :2].contiguous().view(torch.int32).view(-1).long() & 0xFFFFFFFF
    words = torch.where(is_cmp, first["cmp_kv"][torch.where(is_cmp, row, 0)], first["ori_kv"][torch.where(is_cmp, 0, row)])
    return int(words.sum().item()) & 0xFFFFFFFF
