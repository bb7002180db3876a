"""The four DeepGEMM entry points the DSA indexer calls, on MI355X.

Same names, arguments and results as the calls at
dlengine/runtime/layers/backends/dsa/indexer/lightning.py:633 (``get_num_sms``),
:668-676 (``get_paged_mqa_logits_metadata``), :1395-1406
(``fp8_paged_mqa_logits``) and :1212-1219 (``fp8_mqa_logits``, prefill), so the
caller's code stays unchanged.
"""
from __future__ import annotations

import torch

from . import ops


def get_num_sms() -> int:
    """Compute units of the current device (256 on MI355X)."""
    return ops.num_cus()


def get_paged_mqa_logits_metadata(context_lens: torch.Tensor, block_size: int,
                                  num_sms: int | None = None) -> torch.Tensor:
    """Per-step schedule: exclusive prefix sum of per-sequence page counts
    (int32 [B+1]). The logits kernel does not depend on it; it exists so the
    once-per-forward schedule step (deepseek_v2.py:807-840) keeps its shape."""
    return ops.indexer_schedule(context_lens, block_size)


def fp8_paged_mqa_logits(q_fp8: torch.Tensor, kv_cache: torch.Tensor, weights: torch.Tensor,
                         context_lens: torch.Tensor, block_tables: torch.Tensor,
                         schedule_meta: torch.Tensor | None, max_context_len: int,
                         clean_logits: bool = False) -> torch.Tensor:
    """Weighted-ReLU MQA logits over the paged fp8 indexer cache.

    q_fp8 [B, next_n, 64, 128] float8_e4m3fn; kv_cache [pages, page_size, 1, 132]
    (or [pages, page_size*132]) uint8; weights [B*next_n, 64] f32;
    context_lens [B, next_n] int32; block_tables [B, M] int32.
    Returns logits [B*next_n, max_context_len] f32. With ``clean_logits``
    every position at or past the context is -inf; otherwise only the tail of
    the last page is (later positions hold whatever the buffer held).
    """
    B, n = q_fp8.shape[:2]
    kv = kv_cache.reshape(kv_cache.shape[0], -1)
    cl = context_lens.reshape(B, -1)
    if cl.shape[1] != n:
        raise ValueError(f"context_lens must be [B, next_n]; got {tuple(context_lens.shape)} for next_n={n}")
    if clean_logits:
        out = torch.full((B * n, max_context_len), float("-inf"), dtype=torch.float32, device=q_fp8.device)
    else:
        out = None
    if n <= 2:
        return ops.indexer_logits(q_fp8, kv, weights, cl, block_tables, max_context_len, out=out)
    # wider next_n: one launch per query position, sequence-major rows
    if out is None:
        out = torch.empty(B * n, max_context_len, dtype=torch.float32, device=q_fp8.device)
    rows = out.view(B, n, max_context_len)
    w = weights.view(B, n, -1)
    for j in range(n):
        ops.indexer_logits(q_fp8[:, j:j + 1].contiguous(), kv, w[:, j].contiguous(),
                           cl[:, j:j + 1].contiguous(), block_tables, max_context_len, out=rows[:, j])
    return out


def fp8_mqa_logits(q: torch.Tensor, kv: tuple[torch.Tensor, torch.Tensor], weights: torch.Tensor,
                   cu_seq_len_k_start: torch.Tensor, cu_seq_len_k_end: torch.Tensor,
                   clean_logits: bool = True) -> torch.Tensor:
    """Ragged weighted-ReLU MQA logits for prefill.

    q [M, 64, 128] float8_e4m3fn; kv = (keys [N, 128] float8_e4m3fn, scales [N] f32);
    weights [M, 64] f32; cu_seq_len_k_start / _end [M] int32: row i scores keys
    [start[i], end[i]). Returns logits [M, N] f32; with ``clean_logits`` every
    entry outside a row's window is -inf, otherwise those entries are unspecified.
    """
    keys, scales = kv
    out = torch.empty(q.shape[0], keys.shape[0], dtype=torch.float32, device=q.device)
    ops.mqa_logits(q, keys, scales, weights, cu_seq_len_k_start, cu_seq_len_k_end, out, clean_logits)
    return out
