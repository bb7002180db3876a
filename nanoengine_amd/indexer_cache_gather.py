"""Fused paged-to-ragged gather for the fp8 indexer cache, on MI355X.

Mirrors ``gather_indexer_cache``
(dlengine/runtime/kernel/triton/generic/indexer_cache_gather.py:60-114): same
signature, checks and error messages; one HIP launch (dsa_gather_indexer_cache).
"""
from __future__ import annotations

import torch

from . import ops


def gather_indexer_cache(cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_k: torch.Tensor, *,
                         page_size: int, head_dim: int, total_k: int | None = None,
                         max_seqlen_k: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather paged indexer fp8 keys and scales into contiguous ragged rows.

    Each cache page stores all ``page_size * head_dim`` fp8 key bytes first,
    followed by one four-byte f32 scale per token. Returns (keys uint8
    [total_k, head_dim], scales uint8 [total_k, 4]). ``max_seqlen_k`` is
    accepted for signature parity; the HIP kernel does not need it.
    """
    if cache.ndim != 2 or cache.dtype != torch.uint8 or not cache.is_contiguous():
        raise ValueError("cache must be a contiguous 2D uint8 tensor")
    if block_table.ndim != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be 2D and contiguous in its last dimension")
    if cu_seqlens_k.ndim != 1 or not cu_seqlens_k.is_contiguous():
        raise ValueError("cu_seqlens_k must be a contiguous 1D tensor")
    if cu_seqlens_k.numel() != block_table.shape[0] + 1:
        raise ValueError("cu_seqlens_k and block_table batch dimensions differ")
    expected_page_bytes = page_size * (head_dim + 4)
    if cache.shape[1] != expected_page_bytes:
        raise ValueError(f"Indexer cache page has {cache.shape[1]} bytes, expected {expected_page_bytes}")
    if total_k is None:
        total_k = int(cu_seqlens_k[-1].item())
    key_out = torch.empty((total_k, head_dim), dtype=torch.uint8, device=cache.device)
    scale_out = torch.empty((total_k, 4), dtype=torch.uint8, device=cache.device)
    if total_k == 0:
        return key_out, scale_out
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    ops.gather_indexer_cache(cache, bt, cu_seqlens_k, page_size, total_k, key_out, scale_out)
    return key_out, scale_out
