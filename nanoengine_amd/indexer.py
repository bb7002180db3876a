"""Decode-time lightning-indexer selection on MI355X.

Mirrors the selection half of ``Indexer.forward``
(dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1357-1492): paged
fp8 logits, top-k, and (optionally) the logical->physical translation, with the
reference's helper names and checks. The q/k projections, RoPE, Hadamard and
cache writes that precede it in the reference are not part of this path.
"""
from __future__ import annotations

import torch

from . import deep_gemm, deepseek_v4, ops

INDEXER_QUANT_BLOCK_SIZE = 128


def _uses_linear_mtp_indexer_path(*, is_prefill: bool, ntps: int) -> bool:
    """Return whether the wide per-position MTP scoring path is required
    (lightning.py:72-74)."""
    return not is_prefill and ntps > 2


def _expand_decode_context_lens(context_lens: torch.Tensor, next_n: int) -> torch.Tensor:
    """[batch] or [batch, 1] final lengths -> per-query causal lengths
    [batch, next_n] int32, ``ctx - (next_n - 1 - j)`` clamped to >= 1
    (lightning.py:350-378)."""
    if context_lens.dim() == 1:
        context_lens = context_lens[:, None]
    if context_lens.dim() != 2 or context_lens.shape[1] not in (1, next_n):
        raise ValueError(
            "Indexer context_lens must have shape [batch], [batch, 1], or "
            f"[batch, next_n]; got {tuple(context_lens.shape)} for next_n={next_n}")
    if context_lens.shape[1] == next_n:
        return context_lens.to(torch.int32)
    offsets = torch.arange(next_n - 1, -1, -1, dtype=context_lens.dtype, device=context_lens.device)
    return (context_lens - offsets).clamp_min(1).to(torch.int32)


class IndexerCache:
    """Per-layer fp8 indexer key cache, one contiguous uint8 buffer
    ``[num_layers, num_pages, page_size * (head_dim + 4)]``; each page holds
    ``page_size`` fp8 keys followed by ``page_size`` f32 scales
    (lightning.py:408-448)."""

    def __init__(self, num_layers: int, num_pages: int, page_size: int, head_dim: int,
                 device: str | torch.device = "cuda", buffer: torch.Tensor | None = None):
        self.num_layers = num_layers
        self.num_pages = num_pages
        self.page_size = page_size
        self.head_dim = head_dim
        self.quant_block_size = INDEXER_QUANT_BLOCK_SIZE
        self.bytes_per_token = head_dim + head_dim // self.quant_block_size * 4
        shape = (num_layers, num_pages, page_size * self.bytes_per_token)
        self.buffer = torch.zeros(shape, dtype=torch.uint8, device=device) if buffer is None else buffer
        if tuple(self.buffer.shape) != shape or self.buffer.dtype != torch.uint8:
            raise ValueError(f"IndexerCache buffer must be uint8 with shape {shape}, "
                             f"got dtype={self.buffer.dtype}, shape={tuple(self.buffer.shape)}")

    @property
    def buffers(self) -> list[torch.Tensor]:
        return [self.buffer[i] for i in range(self.num_layers)]

    def get_buffer(self, layer_id: int) -> torch.Tensor:
        return self.buffer[layer_id]

    def store_key_fp8(self, layer_id: int, key_bf16: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Quantise keys [N, head_dim] bf16 (UE8M0 per-token scale) and write them
        into the split page layout (lightning.py:449-535), on the GPU."""
        ops.indexer_k_store(key_bf16, self.buffer[layer_id], slot_mapping, self.page_size)


def indexer_decode_topk(q_fp8: torch.Tensor, weights: torch.Tensor, kv_cache_buf: torch.Tensor,
                        context_lens: torch.Tensor, block_tables: torch.Tensor, index_topk: int,
                        page_size: int = 64, *, is_prefill: bool = False, schedule_meta=None,
                        translate_topk: bool = False, topk_page_size: int | None = None,
                        logits_out: torch.Tensor | None = None):
    """Steps 8-9 of ``Indexer.forward`` for decode (lightning.py:1357-1492).

    q_fp8 [num_tokens, 64, 128] (num_tokens = batch * next_n); weights
    [num_tokens, 64] f32; kv_cache_buf [num_pages, page_size * 132] uint8;
    context_lens [batch] int (length after the last query token); block_tables
    [batch, M] int32. Returns logical top-k positions [num_tokens, index_topk]
    int32 (ascending, -1 padded), or (logical, physical) when ``translate_topk``.
    Selection always runs on the exact HIP top-k, at every context length.
    """
    num_tokens = q_fp8.shape[0]
    batch = context_lens.shape[0]
    ntps = num_tokens // batch
    n_heads, head_dim = q_fp8.shape[1], q_fp8.shape[2]
    q4 = q_fp8.view(batch, ntps, n_heads, head_dim)
    kv_cache = kv_cache_buf.view(kv_cache_buf.shape[0], page_size, 1, -1)
    max_context_len = block_tables.shape[-1] * page_size
    ctx = _expand_decode_context_lens(context_lens.to(torch.int32), ntps)
    bt = block_tables.to(torch.int32)
    if not _uses_linear_mtp_indexer_path(is_prefill=is_prefill, ntps=ntps):
        if schedule_meta is None:
            schedule_meta = deep_gemm.get_paged_mqa_logits_metadata(ctx, page_size, None)
    logits = deep_gemm.fp8_paged_mqa_logits(q4, kv_cache, weights, ctx, bt, schedule_meta,
                                            max_context_len, clean_logits=False) \
        if logits_out is None else _logits_into(q4, kv_cache, weights, ctx, bt, max_context_len, logits_out)

    seq_lens = ctx.reshape(-1).contiguous()
    logical = torch.empty((num_tokens, index_topk), dtype=torch.int32, device=q_fp8.device)
    if translate_topk:
        if topk_page_size is None:
            raise ValueError("topk_page_size is required when translate_topk=True")
        page_tables = bt if ntps == 1 else bt.repeat_interleave(ntps, dim=0)
        physical = torch.empty_like(logical)
        deepseek_v4.topk_transform(logits, seq_lens, page_tables, physical, topk_page_size, index_topk,
                                   logical)
        return logical, physical
    if index_topk not in (512, 2048):
        raise ValueError(f"top_k must be 512 or 2048, got {index_topk}")
    ops.topk_transform_raw(logits, seq_lens, logical, index_topk)
    return logical


def _logits_into(q4, kv_cache, weights, ctx, bt, max_context_len, out):
    kv = kv_cache.reshape(kv_cache.shape[0], -1)
    return ops.indexer_logits(q4, kv, weights, ctx, bt, max_context_len, out=out)
