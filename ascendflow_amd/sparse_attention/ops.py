"""Framework-facing sparse MLA: the functional call of a serving framework.

``sparse_flash_mla`` takes the argument convention of the vendor operator the
reference benchmarks against, ``aclnnSparseFlashMla`` as vllm-ascend's
DeepSeek-V4.1 attention calls it (``benchmarks/references/sparse_mla_aclnn.py:40-130``;
``docs/operators/sparse-mla.md:10-14``): TND queries, PA_BBND paged caches,
the original cache under band mask mode 4 with a left window of WINDOW - 1
and no right window, the compressed cache under causal mask mode 3, one sink
per head, and an optional softmax LSE output. Sizes come from the tensor
shapes; the output and the LSE are allocated here. It is registered as the
torch custom op ``ascendflow_amd::sparse_flash_mla`` (with a shape-only fake
implementation, so graph capture and ``torch.compile`` can trace it) and runs
the same gfx950 kernels as ``sparse_mla``.

Only the configuration the reference operator asserts is accepted
(``examples/sparse_attention/attention.py:253-262``): WINDOW = PAGE = 128,
RATIO in {1, 2}, H a multiple of 32, D in {128, 256, 512}. The vendor
metadata tensor (``aclnnSparseFlashMlaMetadata``, a scheduling precomputation)
is accepted and not read: the row-list plan is built on the device per call.
"""

from __future__ import annotations

from typing import Optional

import torch

from .._tensors import require, storage_dtype
from .attention import sparse_mla

ORI_MASK_MODE = 4   # band (sliding window) over the original cache
CMP_MASK_MODE = 3   # causal selection over the compressed cache
BK = 512            # selected-capacity block of the reference kernel (attention.py:258)


def _sizes(q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table, cu_seqlens_q, cmp_ratio, ori_win_left):
    require(q.dim() == 3, "layout_q TND: q must be [T, H, D]")
    T, H, D = (int(v) for v in q.shape)
    require(ori_kv.dim() == 4 and cmp_kv.dim() == 4, "layout_kv PA_BBND: caches must be [blocks, page, 1, D]")
    page = int(ori_kv.shape[1])
    require(cmp_ratio in (1, 2) and page % cmp_ratio == 0, "cmp_ratio must be 1 or 2")
    require(tuple(cmp_kv.shape[1:]) == (page // cmp_ratio, 1, D), "cmp_kv must be [blocks, page / cmp_ratio, 1, D]")
    topk = int(cmp_sparse_indices.shape[-1])
    window = int(ori_win_left) + 1
    return dict(
        B=int(cu_seqlens_q.numel()) - 1,
        T=T,
        H=H,
        D=D,
        PAGE=page,
        RATIO=int(cmp_ratio),
        MAX_SEQ=int(ori_block_table.shape[1]) * page,
        ORI_BLOCKS=int(ori_kv.shape[0]),
        CMP_BLOCKS=int(cmp_kv.shape[0]),
        WINDOW=window,
        TOPK=topk,
        S=window + -(-topk // BK) * BK,
        BM=64 if H % 64 == 0 else 32,
    )


@torch.library.custom_op("ascendflow_amd::sparse_flash_mla", mutates_args=())
def sparse_flash_mla(
    q: torch.Tensor,
    ori_kv: torch.Tensor,
    cmp_kv: torch.Tensor,
    cmp_sparse_indices: torch.Tensor,
    ori_block_table: torch.Tensor,
    cmp_block_table: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    seqused_ori_kv: torch.Tensor,
    seqused_cmp_kv: torch.Tensor,
    cmp_residual_kv: torch.Tensor,
    ori_topk_length: torch.Tensor,
    sinks: torch.Tensor,
    softmax_scale: float,
    cmp_ratio: int,
    metadata: Optional[torch.Tensor] = None,
    ori_mask_mode: int = ORI_MASK_MODE,
    cmp_mask_mode: int = CMP_MASK_MODE,
    ori_win_left: int = 127,
    ori_win_right: int = 0,
    layout_q: str = "TND",
    layout_kv: str = "PA_BBND",
    return_softmax_lse: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns ``(attention_out [T, H, D], softmax_lse)``; ``softmax_lse`` is
    float32 [T, H] (ln of the softmax denominator, sink included) when
    ``return_softmax_lse`` is set, else an empty tensor."""
    require(layout_q == "TND" and layout_kv == "PA_BBND", "supported layouts: layout_q TND, layout_kv PA_BBND")
    require(ori_mask_mode == ORI_MASK_MODE and cmp_mask_mode == CMP_MASK_MODE,
            "supported masks: ori_mask_mode 4 (band), cmp_mask_mode 3 (causal)")
    require(ori_win_right == 0, "the original-cache window ends at the query (ori_win_right 0)")
    sizes = _sizes(q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table, cu_seqlens_q, cmp_ratio, ori_win_left)
    out = torch.empty_like(q)
    lse = (torch.empty((sizes["T"], sizes["H"]), dtype=torch.float32, device=q.device) if return_softmax_lse
           else torch.empty(0, dtype=torch.float32, device=q.device))
    sparse_mla(q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table, cmp_block_table, cu_seqlens_q, seqused_ori_kv,
               seqused_cmp_kv, cmp_residual_kv, ori_topk_length, sinks, out, **sizes,
               VR=16 if sizes["BM"] == 64 else 8, DTYPE=storage_dtype(q.dtype), SCALE=float(softmax_scale),
               softmax_lse=lse if return_softmax_lse else None)
    return out, lse


@sparse_flash_mla.register_fake
def _(q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table, cmp_block_table, cu_seqlens_q, seqused_ori_kv,
      seqused_cmp_kv, cmp_residual_kv, ori_topk_length, sinks, softmax_scale, cmp_ratio, metadata=None,
      ori_mask_mode=ORI_MASK_MODE, cmp_mask_mode=CMP_MASK_MODE, ori_win_left=127, ori_win_right=0, layout_q="TND",
      layout_kv="PA_BBND", return_softmax_lse=False):
    T, H = q.shape[0], q.shape[1]
    lse = q.new_empty((T, H), dtype=torch.float32) if return_softmax_lse else q.new_empty(0, dtype=torch.float32)
    return torch.empty_like(q), lse
