"""Indexer key transform + cache store, on MI355X.

Mirrors ``indexer_k_transform_store_fp8``
(dlengine/runtime/kernel/triton/generic/indexer_transform.py:262-288): one
launch of LayerNorm, RoPE on the leading 64 (interleaved) dims, Hadamard-128,
UE8M0 fp8 quantisation and the store into the indexer's split page layout.
Slots < 0 are skipped (the reference writes them to slot 0).
"""
from __future__ import annotations

import torch

from . import ops


def indexer_k_transform_store_fp8(key: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float,
                                  positions: torch.Tensor, cos_sin_cache: torch.Tensor, cache: torch.Tensor,
                                  slot_mapping: torch.Tensor, page_size: int) -> None:
    """Fuse the complete decode-time Indexer K transform and cache store."""
    if key.dtype != torch.bfloat16 or key.ndim != 2 or key.shape[1] != 128:
        raise ValueError("fused Indexer K path requires a bfloat16 [T, 128] key")
    ops.indexer_k_transform_store(key, weight, bias, eps, positions, cos_sin_cache, cache.view(-1), slot_mapping,
                                  page_size)
