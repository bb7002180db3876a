"""MLA attention backend for the "mi355x" hardware tier (sparse fp8 decode).

Mirrors the reference contract:
- ``MlaAttentionBase`` (dlengine/runtime/layers/backends/mla/base.py:18-49);
- ``FlashMlaAttention.forward`` (dlengine/runtime/layers/backends/mla/flash_mla.py:22-121):
  store the new token's KV into the fp8 cache, then run sparse decode over the
  caller's top-k physical slots (all -1 when none are given, as during graph
  capture warm-up, flash_mla.py:64-74).
It reads the same batch fields through ``get_batch_context()``
(dlengine/runtime/context/batch.py:10-80); ``resolve_mla_plan`` / ``create_mla``
add the tier beside "blackwell" and "hopper" (layers/backends/selector.py:195-223).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from . import flash_mla, ops


@dataclass
class BatchContext:
    """The batch fields the DSA decode path reads (a subset of the reference's
    BatchContext; names and meaning unchanged)."""
    is_prefill: bool = False
    is_dummy: bool = False
    context_lens: torch.Tensor | None = None     # [1, B] int32
    block_tables: torch.Tensor | None = None     # [1, B, M] int32
    slot_mapping: torch.Tensor | None = None     # [T] slots of the new tokens
    num_tokens_per_seq: int = 1
    hisparse_slot_mapping: torch.Tensor | None = None
    indexer_schedule_meta: torch.Tensor | tuple | None = None


_CONTEXT = BatchContext()


def get_batch_context() -> BatchContext:
    return _CONTEXT


def set_batch_context(**fields) -> BatchContext:
    global _CONTEXT
    _CONTEXT = BatchContext(**fields)
    return _CONTEXT


def reset_batch_context() -> None:
    set_batch_context()


class MlaAttentionBase(nn.Module):
    """Contract for MLA attention backends (base.py:18-49)."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int, v_head_dim: int,
                 attention_type: str = "MLA", nsa_index_topk: int = 0, **kwargs) -> None:
        super().__init__()
        if attention_type != "MLA":
            raise ValueError(f"{type(self).__name__} requires MLA attention, got {attention_type!r}.")
        if num_kv_heads != 1:
            raise ValueError(f"MLA requires one compressed KV head, got {num_kv_heads}.")
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.v_head_dim = v_head_dim
        self.nsa_index_topk = nsa_index_topk
        # cache tensors are injected by the model runner after construction
        self.k_cache = self.v_cache = torch.tensor([])


class Mi355xSparseMlaAttention(MlaAttentionBase):
    """Sparse fp8 MLA decode on MI355X (the DSA decode branch of
    FlashMlaAttention.forward, flash_mla.py:30-99)."""

    def __init__(self, *args, **kwargs) -> None:
        kwargs.pop("mla_qk_nope_head_dim", None)
        kwargs.pop("mla_kv_lora_rank", None)
        super().__init__(*args, **kwargs)
        self.sparse_meta = None  # schedule + workspace, reused across steps and graph replays

    def forward(self, q: torch.Tensor, k: torch.Tensor | None, v: torch.Tensor | None,
                sparse_indices: torch.Tensor | None = None, write_kv_cache: bool = True) -> torch.Tensor:
        k_cache = self.k_cache
        context = get_batch_context()
        if write_kv_cache and k is not None and k_cache.numel() and not context.is_dummy:
            slot_mapping = (context.hisparse_slot_mapping if context.hisparse_slot_mapping is not None
                            else context.slot_mapping)
            ops.mla_kv_store(k, k_cache, slot_mapping)
        if context.is_prefill:
            raise RuntimeError("Mi355xSparseMlaAttention.forward serves decode only; MLA prefill is "
                               "handled by the model's non-absorbed path.")
        ntps = context.num_tokens_per_seq
        total_tokens, num_head, head_dim = q.shape
        bs = total_tokens // ntps
        q = q[: bs * ntps]
        if sparse_indices is None:
            if self.nsa_index_topk <= 0:
                raise RuntimeError("the mi355x MLA backend implements the sparse (DSA) decode only")
            sparse_indices = torch.full((bs * ntps, self.nsa_index_topk), -1, dtype=torch.int32, device=q.device)
        topk = sparse_indices.shape[-1]
        if self.sparse_meta is None:
            self.sparse_meta, _ = flash_mla.get_mla_metadata()
        o, _ = flash_mla.flash_mla_with_kvcache(q.reshape(bs, ntps, num_head, head_dim), k_cache, None, None,
                                                self.v_head_dim, self.sparse_meta, None, self.scale, False,
                                                is_fp8_kvcache=True,
                                                indices=sparse_indices.view(bs, ntps, topk))
        return o.reshape(bs * ntps, o.shape[2], o.shape[3])


def resolve_mla_plan(hardware_backend: str = "gpu_generic", capability=None) -> str:
    """selector.py:195-205 with the MI355X tier added."""
    if hardware_backend == "mi355x":
        return "mi355x_sparse"
    if hardware_backend == "blackwell":
        return "trtllm"
    if hardware_backend == "hopper":
        return "flash_mla"
    return "reference"


def create_mla(*, hardware_backend: str = "gpu_generic", **kwargs) -> MlaAttentionBase:
    plan = resolve_mla_plan(hardware_backend)
    if plan == "mi355x_sparse":
        return Mi355xSparseMlaAttention(**kwargs)
    raise RuntimeError(f"this package provides only the mi355x tier (requested plan {plan!r})")
