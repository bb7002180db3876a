"""NSA top-k + page-table translation entry points, on MI355X.

Same signatures and error behaviour as
dlengine/runtime/kernel/jit/sgl/deepseek_v4.py:324-400 (``topk_transform``,
``topk_transform_ragged``, ``topk_transform_512``). The selection is exact at
every context length (the reference's fused kernel is exact only up to 16K and
its ragged variant may differ by a few entries) and emits positions in
ascending order.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops


def topk_transform(scores: torch.Tensor, seq_lens: torch.Tensor, page_tables: torch.Tensor,
                   out_page_indices: torch.Tensor, page_size: int, top_k: int,
                   out_raw_indices: Optional[torch.Tensor] = None) -> None:
    """Select the top ``top_k`` positions of ``scores[b, :seq_lens[b]]`` and write
    them as physical slots ``page_tables[b, p // page_size] * page_size + p %
    page_size`` into ``out_page_indices`` (and as positions into
    ``out_raw_indices``), padding with -1. ``top_k`` in {512, 2048}."""
    if top_k not in (512, 2048):
        raise ValueError(f"top_k must be 512 or 2048, got {top_k}")
    ops.topk_transform(scores, seq_lens, page_tables, out_page_indices, page_size, top_k, out_raw_indices)


def topk_transform_ragged(scores: torch.Tensor, seq_lens: torch.Tensor, row_starts: torch.Tensor,
                          offsets: torch.Tensor, out_indices: torch.Tensor, top_k: int) -> None:
    """Top-2048 over ``scores[b, row_start : row_start + len]``, written as
    ``position + offsets[b]``."""
    if top_k != 2048:
        raise ValueError(f"ragged Indexer top_k must be 2048, got {top_k}")
    ops.topk_transform_ragged(scores, seq_lens, row_starts, offsets, out_indices, top_k)


def topk_transform_512(scores: torch.Tensor, seq_lens: torch.Tensor, page_tables: torch.Tensor,
                       out_page_indices: torch.Tensor, page_size: int,
                       out_raw_indices: Optional[torch.Tensor] = None) -> None:
    """Backward-compatible TopK=512 wrapper."""
    topk_transform(scores, seq_lens, page_tables, out_page_indices, page_size, 512, out_raw_indices)
