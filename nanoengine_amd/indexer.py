"""Lightning-indexer selection on MI355X: decode and chunked prefill.

Mirrors the selection half of ``Indexer.forward``
(dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1357-1492): paged
fp8 logits, top-k, and (optionally) the logical->physical translation, with the
reference's helper names and checks. The q/k projections, RoPE, Hadamard and
cache writes that precede it in the reference are not part of this path.
"""
from __future__ import annotations

import torch

from . import deep_gemm, deepseek_v4, ops
from .deepseek_v4 import topk_transform_ragged
from .indexer_cache_gather import gather_indexer_cache

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
    if index_topk in (512, 2048):
        ops.indexer_select(logits, seq_lens, logical, index_topk)
        return logical
    return _select_other_k(logits, seq_lens, index_topk, logical)


def _select_other_k(logits: torch.Tensor, seq_lens: torch.Tensor, index_topk: int,
                    out: torch.Tensor) -> torch.Tensor:
    """Top-k sizes the HIP select does not instantiate (the model uses 2048):
    the same masking rules with torch's own GPU sort, then ascending order and
    -1 padding as the HIP select writes them (lightning.py:1468-1492)."""
    width = logits.shape[1]
    pos = torch.arange(width, device=logits.device)
    ok = (pos[None, :] < seq_lens[:, None]) & torch.isfinite(logits) & (logits.abs() < 1e30)
    masked = torch.where(ok, logits, torch.full_like(logits, float("-inf")))
    k = min(index_topk, width)
    # a stable descending sort breaks ties by the lowest position, as the HIP select does
    idx = torch.sort(masked, dim=-1, descending=True, stable=True).indices[:, :k]
    idx = torch.where(idx < seq_lens[:, None], idx, torch.full_like(idx, width))
    idx = idx.sort(dim=-1).values.to(torch.int32)
    out.fill_(-1)
    out[:, :k] = torch.where(idx < width, idx, torch.full_like(idx, -1))
    return out


def _logits_into(q4, kv_cache, weights, ctx, bt, max_context_len, out):
    kv = kv_cache.reshape(kv_cache.shape[0], -1)
    return ops.indexer_logits(q4, kv, weights, ctx, bt, max_context_len, out=out)


def _prefill_mqa_chunk_rows(num_queries: int, num_keys: int, device: torch.device,
                            max_rows: int | None = None) -> int:
    """Query rows per ragged-logits chunk, from the memory a [rows, num_keys]
    f32 logits tensor needs (lightning.py:381-405)."""
    if num_queries <= 0:
        return 0
    if num_keys <= 0:
        raise ValueError("prefill Indexer requires at least one key")
    if max_rows is not None and max_rows <= 0:
        raise ValueError(f"max_rows must be positive, got {max_rows}")
    rows = num_queries
    logits_elements = num_queries * num_keys
    if logits_elements >= 8_000_000:
        free_mem, total_mem = torch.cuda.mem_get_info(device)
        logits_bytes = logits_elements * 4
        if logits_bytes * 2 > free_mem or logits_bytes > total_mem * 0.3:
            bytes_per_row = num_keys * 4
            rows = max(1, int((free_mem * 0.45) // bytes_per_row))
    if max_rows is not None:
        rows = min(rows, max_rows)
    return min(rows, num_queries)


def compute_prefill_topk_paged(q_fp8: torch.Tensor, weights: torch.Tensor, cu_seqlens_q: torch.Tensor,
                               cu_seqlens_k: torch.Tensor, block_table: torch.Tensor,
                               cache_buf: torch.Tensor, *, page_size: int = 64, index_topk: int = 2048,
                               query_chunk: int | None = None) -> torch.Tensor:
    """Prefill top-k with ragged fp8 MQA logits: the selection half of
    ``Indexer.compute_prefill_topk_paged`` (lightning.py:1081-1250), from the
    quantised queries on.

    q_fp8 [num_queries, 64, 128] float8_e4m3fn and weights [num_queries, 64]
    f32 (the q prologue's outputs); cu_seqlens_q / cu_seqlens_k [num_seqs + 1]
    (each sequence's fresh queries are the last q_len of its k_len keys, whose
    keys are already in the paged cache); block_table [num_seqs, pages] int32;
    cache_buf [num_pages, page_size * 132] uint8. Returns packed global
    logical indices [num_queries, index_topk] int32 into the ragged key order
    (sequence b's keys at cu_seqlens_k[b] ...), -1 padded.
    """
    if query_chunk is not None and query_chunk <= 0:
        raise ValueError(f"query_chunk must be positive, got {query_chunk}")
    if cu_seqlens_q.shape != cu_seqlens_k.shape:
        raise RuntimeError("cu_seqlens_q/cu_seqlens_k shape mismatch: "
                           f"{cu_seqlens_q.shape} vs {cu_seqlens_k.shape}")
    num_queries = q_fp8.shape[0]
    indices = torch.full((num_queries, index_topk), -1, dtype=torch.int32, device=q_fp8.device)
    if num_queries == 0:
        return indices
    head_dim = q_fp8.shape[-1]
    num_seqs = cu_seqlens_q.numel() - 1
    if block_table.shape[0] != num_seqs:
        raise RuntimeError(f"block_table/cu_seqlens batch mismatch: {block_table.shape[0]} vs {num_seqs}")
    q_first = int(cu_seqlens_q[0].item())
    k_first = int(cu_seqlens_k[0].item())
    q_total = int(cu_seqlens_q[-1].item())
    if q_first != 0 or k_first != 0:
        raise RuntimeError("ragged Indexer cu_seqlens must start at zero")
    if q_total != num_queries:
        raise RuntimeError(f"cu_seqlens_q does not cover the packed queries: {q_total} vs {num_queries}")
    q_lens = (cu_seqlens_q[1:] - cu_seqlens_q[:-1]).to(torch.int32)
    k_lens = (cu_seqlens_k[1:] - cu_seqlens_k[:-1]).to(torch.int32)
    if bool(torch.any(q_lens < 0).item()) or bool(torch.any(k_lens < q_lens).item()):
        raise RuntimeError("Invalid prefill ragged lengths: K length must cover every Q length")
    used_pages = torch.div(k_lens + page_size - 1, page_size, rounding_mode="floor")
    if int(used_pages.max().item()) > block_table.shape[1]:
        raise RuntimeError("Indexer block table is too short for the longest sequence")

    total_k = int(cu_seqlens_k[-1].item())
    max_seqlen_k = int(k_lens.max().item())
    key_bytes, scale_bytes = gather_indexer_cache(cache_buf, block_table, cu_seqlens_k, page_size=page_size,
                                                  head_dim=head_dim, total_k=total_k, max_seqlen_k=max_seqlen_k)
    kv_fp8 = (key_bytes.view(torch.float8_e4m3fn), scale_bytes.view(torch.float32).reshape(-1))

    q_to_seq = torch.repeat_interleave(torch.arange(num_seqs, dtype=torch.int64, device=q_fp8.device),
                                       q_lens.to(torch.int64), output_size=num_queries)
    q_starts = cu_seqlens_q[:-1].index_select(0, q_to_seq).to(torch.int32)
    k_starts = cu_seqlens_k[:-1].index_select(0, q_to_seq).to(torch.int32)
    cached_lens = (k_lens - q_lens).index_select(0, q_to_seq)
    local_q = torch.arange(num_queries, dtype=torch.int32, device=q_fp8.device) - q_starts
    ks = k_starts.contiguous()
    ke = (ks + cached_lens + local_q + 1).contiguous()

    chunk_rows = _prefill_mqa_chunk_rows(num_queries, total_k, q_fp8.device, max_rows=query_chunk)
    use_fused_topk = index_topk == 2048
    valid_lens = (ke - ks).contiguous()
    for start in range(0, num_queries, chunk_rows):
        end = min(start + chunk_rows, num_queries)
        logits = deep_gemm.fp8_mqa_logits(q_fp8[start:end], kv_fp8, weights[start:end], ks[start:end],
                                          ke[start:end], clean_logits=not use_fused_topk)
        if use_fused_topk:
            topk_transform_ragged(logits, valid_lens[start:end], ks[start:end], ks[start:end],
                                  indices[start:end], index_topk)
        else:
            actual_topk = min(index_topk, total_k)
            top_values, logical = logits.topk(actual_topk, dim=-1)
            logical = logical.to(torch.int32).masked_fill_(~torch.isfinite(top_values), -1)
            if actual_topk < index_topk:
                logical = torch.nn.functional.pad(logical, (0, index_topk - actual_topk), value=-1)
            indices[start:end] = logical
            del top_values, logical
        del logits
    return indices
