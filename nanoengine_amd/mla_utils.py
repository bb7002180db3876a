"""``topk_indices_to_physical`` and ``merge_attention_states`` on MI355X.

Mirrors dlengine/runtime/layers/backends/attention/mla_utils.py:12-23 and
:237-272.
"""
from __future__ import annotations

import torch

from . import ops


def topk_indices_to_physical(topk_indices: torch.Tensor, block_table: torch.Tensor,
                             block_size: int) -> torch.Tensor:
    """Logical token positions [rows, topk] int32 (-1 = padding) -> physical
    slots ``block_table[row, idx // block_size] * block_size + idx % block_size``
    with -1 preserved. ``block_table`` has one row per ``topk_indices`` row, or
    one row per ``next_n`` consecutive rows (the MTP layout that the reference
    builds with ``repeat_interleave``)."""
    if topk_indices.dtype != torch.int32:
        topk_indices = topk_indices.to(torch.int32)
    rows = topk_indices.shape[0]
    if block_table.shape[0] == 0 or rows % block_table.shape[0]:
        raise RuntimeError(f"block_table rows {block_table.shape[0]} do not divide index rows {rows}")
    return ops.topk_to_physical(topk_indices, block_table, block_size,
                                rows_per_table=rows // block_table.shape[0])


def merge_attention_states(left: torch.Tensor, left_lse: torch.Tensor, right: torch.Tensor,
                           right_lse: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Merge two attention outputs [T, H, D] by their LSEs [H, T] (natural log)."""
    merged_lse = torch.logaddexp(left_lse, right_lse)
    left_scale = torch.exp(left_lse - merged_lse).transpose(0, 1).unsqueeze(-1)
    right_scale = torch.exp(right_lse - merged_lse).transpose(0, 1).unsqueeze(-1)
    merged = left.float() * left_scale + right.float() * right_scale
    return merged.to(left.dtype), merged_lse
