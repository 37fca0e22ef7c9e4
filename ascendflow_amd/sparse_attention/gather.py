"""Sparse-MLA row selection and gather on MI355X.

The reference's gather helpers (``examples/sparse_attention/gather.py:8-131``:
``query_metadata``, ``copy_window_pages``, ``copy_window_ring``,
``gather_compressed``) are in-kernel DSL functions with no external callers.
Their gfx950 counterparts are the device functions ``token_geometry``,
``resolve_slot`` and ``row_pointer`` of ``csrc/sparse_mla.hip``, shared by the
fused attention kernel and by the gather-image kernel exposed here.

``sparse_mla_gather`` writes the layout of the reference's gather workspace and
gather oracle (``benchmarks/attention/sparse_reference.py:174-181``): window
slot ``i`` for position ``right - visible + i``, compressed slot
``WINDOW + rank``, unused slots zero with bias ``-inf``. It is the device side
of the bit-exact gather check (``benchmarks/attention/run_sparse.py:111-130``).
"""

from __future__ import annotations

import ctypes as ct

import torch

from .. import _native
from .._tensors import DTYPES, check_tensor, storage_dtype, stream_handle
from .attention import check_inputs, make_params


def sparse_mla_gather(
    ori_kv,
    cmp_kv,
    cmp_sparse_indices,
    ori_block_table,
    cmp_block_table,
    cu_seqlens_q,
    seqused_ori_kv,
    seqused_cmp_kv,
    cmp_residual_kv,
    ori_topk_length,
    kv_out=None,
    bias_out=None,
    *,
    B,
    T,
    D=512,
    PAGE=128,
    RATIO=2,
    MAX_SEQ=4096,
    ORI_BLOCKS=128,
    CMP_BLOCKS=128,
    WINDOW=128,
    TOPK=512,
    S=640,
    DTYPE="bf16",
):
    """Gather image (kv [T, S, D] in DTYPE, bias f32 [T, S]); returns (kv, bias)."""
    dtype = storage_dtype(DTYPE)
    tensors = {
        "ori_kv": ori_kv,
        "cmp_kv": cmp_kv,
        "cmp_sparse_indices": cmp_sparse_indices,
        "ori_block_table": ori_block_table,
        "cmp_block_table": cmp_block_table,
        "cu_seqlens_q": cu_seqlens_q,
        "seqused_ori_kv": seqused_ori_kv,
        "seqused_cmp_kv": seqused_cmp_kv,
        "cmp_residual_kv": cmp_residual_kv,
        "ori_topk_length": ori_topk_length,
    }
    device = check_inputs(
        tensors, B=B, T=T, H=1, D=D, PAGE=PAGE, RATIO=RATIO, MAX_SEQ=MAX_SEQ,
        ORI_BLOCKS=ORI_BLOCKS, CMP_BLOCKS=CMP_BLOCKS, TOPK=TOPK, dtype=dtype,
    )
    if kv_out is None:
        kv_out = torch.empty((T, S, D), dtype=DTYPES[dtype], device=device)
    if bias_out is None:
        bias_out = torch.empty((T, S), dtype=torch.float32, device=device)
    check_tensor("kv_out", kv_out, (T, S, D), DTYPES[dtype], device)
    check_tensor("bias_out", bias_out, (T, S), torch.float32, device)
    params = make_params(B, T, 64, D, PAGE, RATIO, MAX_SEQ, ORI_BLOCKS, CMP_BLOCKS, WINDOW, TOPK, S, 64, dtype, 1.0)
    status = _native.library().launch_sparse_mla_gather(
        stream_handle(device),
        *(t.data_ptr() for t in tensors.values()),
        kv_out.data_ptr(),
        bias_out.data_ptr(),
        ct.byref(params),
    )
    _native.check(status, "launch_sparse_mla_gather")
    return kv_out, bias_out
