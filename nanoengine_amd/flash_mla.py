"""The FlashMLA entry points the sparse fp8 decode path calls, on MI355X.

``flash_mla_with_kvcache(..., is_fp8_kvcache=True, indices=...)`` with the
argument order used at dlengine/runtime/layers/backends/mla/flash_mla.py:86-97,
and ``get_mla_metadata()`` (:80-81). Only the sparse fp8 decode is provided:
the dense paged decode is not on the DSA path and raises.
"""
from __future__ import annotations

import torch

from . import ops


class SparseMlaSchedule:
    """Opaque per-shape schedule: the split count and a reusable workspace."""

    def __init__(self) -> None:
        self.num_splits: int | None = None
        self.workspace: torch.Tensor | None = None
        self.key: tuple | None = None

    def prepare(self, num_tokens: int, num_heads: int, topk: int, device: torch.device) -> None:
        key = (num_tokens, num_heads, topk, device)
        if self.key == key:
            return
        self.num_splits = ops.sparse_mla_num_splits(num_tokens, num_heads, topk, device)
        need = ops.sparse_mla_workspace_bytes(num_tokens, num_heads, self.num_splits)
        self.workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
        self.key = key


def get_mla_metadata(*args, **kwargs):
    """Returns (schedule, None); the schedule is filled on first use and must be
    reused across graph replays (allocate it before capture)."""
    return SparseMlaSchedule(), None


def flash_mla_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, block_table, cache_seqlens,
                           head_dim_v: int, tile_scheduler_metadata, num_splits, softmax_scale: float,
                           causal: bool = False, is_fp8_kvcache: bool = False,
                           indices: torch.Tensor | None = None):
    """Sparse MLA decode. q [B, n, H, 576] bf16; k_cache [blocks, block_size, 1, 656]
    fp8 bytes (block stride may include the padding row); indices [B, n, topk]
    int32 physical slots (-1 = skip). Returns (o [B, n, H, 512] bf16,
    lse [B, H, n] f32, natural log)."""
    if indices is None or not is_fp8_kvcache:
        raise NotImplementedError("only the sparse fp8 MLA decode (indices=..., is_fp8_kvcache=True) "
                                  "is implemented on MI355X")
    if causal:
        raise ValueError("causal must be False for sparse decode")
    if head_dim_v != ops.MLA_D_V:
        raise ValueError(f"head_dim_v must be {ops.MLA_D_V}, got {head_dim_v}")
    B, n, H, D = q.shape
    topk = indices.shape[-1]
    q3 = q.reshape(B * n, H, D)
    idx = indices.reshape(B * n, topk)
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    sched = tile_scheduler_metadata
    splits, ws = None, None
    if isinstance(sched, SparseMlaSchedule):
        sched.prepare(B * n, H, topk, q.device)
        splits, ws = sched.num_splits, sched.workspace
    if num_splits is not None:
        splits = int(num_splits)
    o, lse = ops.sparse_mla_decode(q3, k_cache, idx, softmax_scale, num_splits=splits, workspace=ws)
    return o.view(B, n, H, ops.MLA_D_V), lse.view(B, n, H).permute(0, 2, 1)
