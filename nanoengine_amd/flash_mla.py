"""The FlashMLA entry points the DSA path calls, on MI355X.

``flash_mla_with_kvcache(..., is_fp8_kvcache=True, indices=...)`` with the
argument order used at dlengine/runtime/layers/backends/mla/flash_mla.py:86-97,
``get_mla_metadata()`` (:80-81), and the sparse prefill
``flash_mla_sparse_fwd(q, kv, indices, sm_scale, d_v)`` as called at
dlengine/runtime/models/deepseek_v2/deepseek_v2.py:1644-1650. The dense paged
decode is not on the DSA path and raises.
"""
from __future__ import annotations

import torch

from . import ops


class SparseMlaSchedule:
    """Opaque schedule: the split count and a workspace per shape. Every
    shape's workspace is kept for the schedule's lifetime, because a HIP graph
    captured at one shape holds that workspace's address: freeing it when the
    shape changes would let later replays write their split partials over
    whatever the allocator put there next."""

    def __init__(self) -> None:
        self.num_splits: int | None = None
        self.workspace: torch.Tensor | None = None
        self.key: tuple | None = None
        self._by_key: dict = {}

    def prepare(self, num_tokens: int, num_heads: int, topk: int, device: torch.device) -> None:
        key = (num_tokens, num_heads, topk, device)
        if self.key == key:
            return
        if key not in self._by_key:
            splits = ops.sparse_mla_num_splits(num_tokens, num_heads, topk, device)
            need = ops.sparse_mla_workspace_bytes(num_tokens, num_heads, splits)
            self._by_key[key] = (splits, torch.empty(max(need, 1), dtype=torch.uint8, device=device))
        self.num_splits, self.workspace = self._by_key[key]
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


def flash_mla_sparse_fwd(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor, sm_scale: float,
                         d_v: int = 512):
    """Sparse MLA prefill. q [s_q, h_q, 576] bf16; kv [s_kv, h_kv=1, 576] bf16
    (the chunk's cached + fresh keys, ragged order); indices [s_q, h_kv=1, topk]
    int32 logical indices into kv (-1 or >= s_kv = skip). Returns
    (out [s_q, h_q, d_v] bf16, max_logits [s_q, h_q] f32, lse [s_q, h_q] f32,
    natural log)."""
    if d_v != ops.MLA_D_V:
        raise ValueError(f"d_v must be {ops.MLA_D_V}, got {d_v}")
    if kv.dim() != 3 or kv.shape[1] != 1:
        raise ValueError(f"kv must be [s_kv, 1, 576] (one KV head), got {tuple(kv.shape)}")
    if indices.dim() != 3 or indices.shape[1] != 1 or indices.shape[0] != q.shape[0]:
        raise ValueError(f"indices must be [s_q, 1, topk], got {tuple(indices.shape)}")
    idx = indices[:, 0, :]
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    return ops.sparse_mla_prefill(q, kv[:, 0, :], idx, sm_scale)


def flash_mla_sparse_fwd_paged(q: torch.Tensor, k_cache: torch.Tensor, block_table: torch.Tensor,
                               cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, key_states: torch.Tensor,
                               indices: torch.Tensor, sm_scale: float, d_v: int = 512,
                               total_k: int | None = None):
    """The chunked prefill's key assembly and sparse MLA in one call
    (models/deepseek_v2/deepseek_v2.py:1573-1650: _gather_cache_cached_only,
    restore_mla_fp8_cache_rows and _interleave_cached_fresh, then
    flash_mla_sparse_fwd): the cached keys are read from the paged fp8 cache,
    the fresh ones from key_states [total_q, (1,) 576] bf16. indices
    [s_q, 1, topk] are positions in the ragged key order. Returns
    (out [s_q, h_q, d_v] bf16, max_logits [s_q, h_q] f32, lse [s_q, h_q] f32)."""
    if d_v != ops.MLA_D_V:
        raise ValueError(f"d_v must be {ops.MLA_D_V}, got {d_v}")
    if indices.dim() != 3 or indices.shape[1] != 1 or indices.shape[0] != q.shape[0]:
        raise ValueError(f"indices must be [s_q, 1, topk], got {tuple(indices.shape)}")
    idx = indices[:, 0, :]
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    if total_k is None:
        total_k = int(cu_seqlens_k[-1].item())
    dt = torch.int64 if torch.int64 in (cu_seqlens_q.dtype, cu_seqlens_k.dtype) else torch.int32
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    return ops.sparse_mla_prefill_paged(q, k_cache, bt, cu_seqlens_q.to(dt).contiguous(),
                                        cu_seqlens_k.to(dt).contiguous(), key_states, idx, sm_scale, total_k)
