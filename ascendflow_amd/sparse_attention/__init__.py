"""Sparse MLA (examples/sparse_attention in the reference) on MI355X."""

from .attention import sparse_mla, sparse_mla_planned
from .gather import sparse_mla_gather
from .indexer import sparse_topk_indices
from .ops import sparse_flash_mla

__all__ = ["sparse_mla", "sparse_mla_planned", "sparse_mla_gather", "sparse_flash_mla", "sparse_topk_indices"]
