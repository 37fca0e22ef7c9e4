"""Top-k index selection: the producer of ``cmp_sparse_indices``.

The reference takes ``cmp_sparse_indices`` as an input of the sparse operator
and leaves the indexer that produces it to the caller
(``docs/operators/sparse-mla.md:8,266``). What it fixes is the tensor's
contract: per token, at most ``min(TOPK, seqused_cmp_kv[b], cutoff)`` compressed
positions below the causal cutoff ``max(0, C_b R + r_b - n + j + 1) // R``,
ascending, then ``-1`` (``docs/operators/sparse-mla.md:41-51,79``;
``examples/sparse_attention/attention.py:339-341``).

``sparse_topk_indices`` fills that tensor on the GPU from one index score per
(token, compressed position): the positions of largest score below the
cutoff, ties to the lower position. How the scores are computed (the
indexer's own attention over compressed keys) is the caller's, as it is in the
reference.

The same call is registered as the torch custom op
``ascendflow_amd::sparse_topk_indices`` (with a shape-only fake), so a
framework can trace the indexer -> top-k -> ``sparse_flash_mla`` chain.
"""

from __future__ import annotations

import ctypes as ct

import torch

from .. import _native
from .._tensors import check_disjoint, check_tensor, require, stream_handle


class SparseTopkParams(ct.Structure):
    _fields_ = [
        ("B", ct.c_int32),
        ("T", ct.c_int32),
        ("TOPK", ct.c_int32),
        ("RATIO", ct.c_int32),
        ("C", ct.c_int64),
    ]


def sparse_topk_indices(scores, cu_seqlens_q, seqused_cmp_kv, cmp_residual_kv, TOPK=512, RATIO=2, out=None):
    """Writes (and returns) ``cmp_sparse_indices`` [T, 1, TOPK] int32 for f32 ``scores`` [T, C].

    Raises ``ValueError`` on a shape, dtype or device mismatch, as the sparse
    operator's own argument checks do; positions at or beyond ``C`` are never
    selected.
    """
    require(isinstance(scores, torch.Tensor) and scores.dim() == 2, "scores must be a [T, C] tensor")
    t, c = scores.shape
    require(t > 0 and c > 0, "scores must be non-empty")
    require(c < 2**31, "scores may hold at most 2^31 - 1 columns")
    require(TOPK > 0, "TOPK must be positive")
    require(RATIO in (1, 2), "RATIO must be 1 or 2")
    device = scores.device
    check_tensor("scores", scores, (t, c), torch.float32)
    b = cu_seqlens_q.numel() - 1
    require(b > 0, "cu_seqlens_q must hold B + 1 offsets")
    check_tensor("cu_seqlens_q", cu_seqlens_q, (b + 1,), torch.int32, device)
    check_tensor("seqused_cmp_kv", seqused_cmp_kv, (b,), torch.int32, device)
    check_tensor("cmp_residual_kv", cmp_residual_kv, (b,), torch.int32, device)
    if out is None:
        out = torch.empty((t, 1, TOPK), dtype=torch.int32, device=device)
    check_tensor("cmp_sparse_indices", out, (t, 1, TOPK), torch.int32, device)
    check_disjoint(
        [
            ("scores", scores, False),
            ("cu_seqlens_q", cu_seqlens_q, False),
            ("seqused_cmp_kv", seqused_cmp_kv, False),
            ("cmp_residual_kv", cmp_residual_kv, False),
            ("cmp_sparse_indices", out, True),
        ]
    )
    params = SparseTopkParams(b, t, TOPK, RATIO, c)
    status = _native.library().launch_sparse_topk_indices(
        stream_handle(device),
        scores.data_ptr(),
        cu_seqlens_q.data_ptr(),
        seqused_cmp_kv.data_ptr(),
        cmp_residual_kv.data_ptr(),
        out.data_ptr(),
        ct.byref(params),
    )
    _native.check(status, "launch_sparse_topk_indices")
    return out


@torch.library.custom_op("ascendflow_amd::sparse_topk_indices", mutates_args=())
def sparse_topk_indices_op(
    scores: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    seqused_cmp_kv: torch.Tensor,
    cmp_residual_kv: torch.Tensor,
    topk: int,
    cmp_ratio: int,
) -> torch.Tensor:
    """Framework-facing form of ``sparse_topk_indices``: returns a new
    ``cmp_sparse_indices`` [T, 1, topk] int32."""
    return sparse_topk_indices(scores, cu_seqlens_q, seqused_cmp_kv, cmp_residual_kv, TOPK=topk, RATIO=cmp_ratio)


@sparse_topk_indices_op.register_fake
def _(scores, cu_seqlens_q, seqused_cmp_kv, cmp_residual_kv, topk, cmp_ratio):
    return scores.new_empty((scores.shape[0], 1, topk), dtype=torch.int32)
