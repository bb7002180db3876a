"""``topk_indices_to_physical`` and ``merge_attention_states`` on MI355X.

Mirrors dlengine/runtime/layers/backends/attention/mla_utils.py:12-23 and
:237-272, plus the prefill's key assembly from the fp8 cache (:118-236).
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


def assemble_prefill_kv(k_cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_q: torch.Tensor,
                        cu_seqlens_k: torch.Tensor, key_states: torch.Tensor,
                        total_k: int | None = None) -> torch.Tensor:
    """The sparse prefill's keys [total_k, 1, 576] bf16 in ragged order: each
    sequence's cached prefix restored from the fp8 cache, then its fresh rows
    (``key_states`` [total_q, (1,) 576] bf16). One HIP pass does what the
    reference does with _gather_cache_cached_only, restore_mla_fp8_cache_rows
    and _interleave_cached_fresh (mla_utils.py:118-236, called at
    models/deepseek_v2/deepseek_v2.py:1573-1604). ``total_k`` (= cu_seqlens_k[-1])
    saves a device read when the caller knows it."""
    fresh = key_states.reshape(key_states.shape[0], -1)
    if total_k is None:
        total_k = int(cu_seqlens_k[-1].item())
    dt = torch.int64 if torch.int64 in (cu_seqlens_q.dtype, cu_seqlens_k.dtype) else torch.int32
    out = torch.empty(total_k, ops.MLA_D_QK, dtype=torch.bfloat16, device=key_states.device)
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    ops.mla_prefill_kv(k_cache, bt, cu_seqlens_q.to(dt).contiguous(), cu_seqlens_k.to(dt).contiguous(), fresh,
                       total_k, out)
    return out.view(total_k, 1, ops.MLA_D_QK)
