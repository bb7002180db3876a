"""Indexer query prologue and NSA top-k + page-table translation entry points, on MI355X.

Same signatures and error behaviour as
dlengine/runtime/kernel/jit/sgl/deepseek_v4.py:290-400
(``indexer_q_rope_hadamard_quant``, ``topk_transform``,
``topk_transform_ragged``, ``topk_transform_512``). The selection is exact at
every context length (the reference's fused kernel is exact only up to 16K and
its ragged variant may differ by a few entries) and emits positions in
ascending order.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops


def indexer_q_rope_hadamard_quant(query: torch.Tensor, gate_weight: torch.Tensor, weight_scale: float,
                                  cos_sin_cache: torch.Tensor, positions: torch.Tensor,
                                  rope_interleaved: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """Fuse RoPE-first, Hadamard-128, UE8M0 quant, and gate scaling.

    query [T, H, 128] bf16 with dims 0..63 as interleaved RoPE pairs (the
    reference's only layout; ``rope_interleaved=False`` takes them already in
    the half layout), gate_weight [T, H] bf16, cos_sin_cache [max_pos, (1,) 64]
    f32, positions [T] int32/int64. Returns (q_fp8 [T, H, 128] e4m3fn,
    weights [T, H, 1] f32 = gate * weight_scale * q_scale)."""
    if query.shape[-1] != 128:
        raise ValueError(f"Indexer query head dim must be 128, got {query.shape[-1]}")
    if gate_weight.shape != query.shape[:-1]:
        raise ValueError(
            f"gate weight shape {tuple(gate_weight.shape)} does not match "
            f"query shape {tuple(query.shape[:-1])}")
    query = query.contiguous()
    q_fp8 = torch.empty_like(query, dtype=torch.float8_e4m3fn)
    weights_out = torch.empty((*query.shape[:-1], 1), dtype=torch.float32, device=query.device)
    ops.indexer_q_prologue(query, gate_weight, weight_scale, cos_sin_cache, positions, q_fp8, weights_out,
                           rope_interleaved)
    return q_fp8, weights_out


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
