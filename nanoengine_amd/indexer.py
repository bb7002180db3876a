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


# Logits workspace of one prefill call: at most this fraction of the device's
# HBM (9 GB on a 288 GB MI355X, a whole 8K x 128K chunk of f32 logits). The rows
# of a chunk follow from it; the buffer is allocated once per call and reused.
PREFILL_LOGITS_HBM_FRACTION = 1 / 32
_HBM_BYTES: dict = {}


def _prefill_chunk_rows(num_queries: int, num_keys: int, device: torch.device,
                        query_chunk: int | None = None) -> int:
    """Query rows per logits chunk: as many [rows, num_keys] f32 rows as fit in
    the call's logits workspace, capped by ``query_chunk``."""
    if num_keys <= 0:
        raise ValueError("prefill Indexer requires at least one key")
    dev = torch.device(device)
    key = (dev.type, dev.index if dev.index is not None else torch.cuda.current_device())
    if key not in _HBM_BYTES:
        _HBM_BYTES[key] = torch.cuda.get_device_properties(key[1]).total_memory
    budget = int(_HBM_BYTES[key] * PREFILL_LOGITS_HBM_FRACTION)
    rows = max(1, budget // (4 * num_keys))
    if query_chunk is not None:
        rows = min(rows, query_chunk)
    return min(rows, num_queries)


def _select_rows_descending(logits: torch.Tensor, out: torch.Tensor, top_k: int) -> None:
    """Top-k sizes other than 2048 on window-cleaned logits: positions by
    descending logit, non-finite picks as -1, -1 padding past the key count
    (lightning.py:1232-1245). ``out`` arrives filled with -1."""
    k = min(top_k, logits.shape[1])
    vals, pos = torch.topk(logits, k, dim=-1)
    out[:, :k] = torch.where(torch.isfinite(vals), pos.to(torch.int32), -1)


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

    The windows and the batch checks run in one kernel (``ops.prefill_windows``);
    the host reads its 32-byte status once, which is the call's only
    synchronisation. The paged keys are gathered to ragged order once, then
    for top-2048 the logits kernel feeds the exact select directly
    (``ops.mqa_topk``: no logits buffer); for other k the logits go chunk by
    chunk through one reused buffer, each chunk followed by its top-k.
    """
    if query_chunk is not None and query_chunk <= 0:
        raise ValueError(f"query_chunk must be positive, got {query_chunk}")
    if cu_seqlens_q.shape != cu_seqlens_k.shape:
        raise RuntimeError("cu_seqlens_q/cu_seqlens_k shape mismatch: "
                           f"{cu_seqlens_q.shape} vs {cu_seqlens_k.shape}")
    dev = q_fp8.device
    num_queries = q_fp8.shape[0]
    indices = torch.full((num_queries, index_topk), -1, dtype=torch.int32, device=dev)
    if num_queries == 0:
        return indices
    num_seqs = cu_seqlens_q.numel() - 1
    if block_table.shape[0] != num_seqs:
        raise RuntimeError(f"block_table/cu_seqlens batch mismatch: {block_table.shape[0]} vs {num_seqs}")

    cu_dtype = torch.int64 if torch.int64 in (cu_seqlens_q.dtype, cu_seqlens_k.dtype) else torch.int32
    cu_q = cu_seqlens_q.to(cu_dtype).contiguous()
    cu_k = cu_seqlens_k.to(cu_dtype).contiguous()
    windows = torch.empty(2, num_queries, dtype=torch.int32, device=dev)
    ks, ke = windows[0], windows[1]
    status = torch.empty(4, dtype=torch.int64, device=dev)
    ops.prefill_windows(cu_q, cu_k, num_queries, page_size, ks, ke, status)
    faults, total_k, max_seqlen_k, max_pages = status.tolist()
    if faults & 1:
        raise RuntimeError("ragged Indexer cu_seqlens must start at zero")
    if faults & 2:
        q_total = int(cu_q[-1])
        raise RuntimeError(f"cu_seqlens_q does not cover the packed queries: {q_total} vs {num_queries}")
    if faults & 4:
        raise RuntimeError("Invalid prefill ragged lengths: K length must cover every Q length")
    if max_pages > block_table.shape[1]:
        raise RuntimeError("Indexer block table is too short for the longest sequence")

    key_bytes, scale_bytes = gather_indexer_cache(cache_buf, block_table, cu_k, page_size=page_size,
                                                  head_dim=q_fp8.shape[-1], total_k=total_k,
                                                  max_seqlen_k=max_seqlen_k)
    keys = key_bytes.view(torch.float8_e4m3fn)
    key_scales = scale_bytes.view(torch.float32).reshape(-1)

    if index_topk == 2048 and PREFILL_FUSED_TOPK:
        # logits and top-k in one pass: no [rows, total_k] logits buffer
        rows = min(query_chunk or num_queries, num_queries)
        workspace = torch.empty(ops.mqa_topk_workspace_bytes(rows, total_k), dtype=torch.uint8, device=dev)
        for r0 in range(0, num_queries, rows):
            r1 = min(r0 + rows, num_queries)
            ops.mqa_topk(q_fp8[r0:r1], keys, key_scales, weights[r0:r1], ks[r0:r1], ke[r0:r1], max_seqlen_k,
                         indices[r0:r1], index_topk, workspace=workspace)
        return indices

    fused = index_topk == 2048
    rows = _prefill_chunk_rows(num_queries, total_k, dev, query_chunk)
    workspace = torch.empty(rows, total_k, dtype=torch.float32, device=dev)
    lens = (ke - ks) if fused else None
    for r0 in range(0, num_queries, rows):
        r1 = min(r0 + rows, num_queries)
        logits = workspace[:r1 - r0]
        _score_chunk(q_fp8[r0:r1], keys, key_scales, weights[r0:r1], ks[r0:r1], ke[r0:r1], logits,
                     clean=not fused)
        if fused:
            # positions come back relative to the window start; adding ks makes them global
            ops.topk_transform_ragged(logits, lens[r0:r1], ks[r0:r1], ks[r0:r1], indices[r0:r1], index_topk)
        else:
            _select_rows_descending(logits, indices[r0:r1], index_topk)
    return indices


# top-2048 through ops.mqa_topk (logits never stored); False scores each chunk
# of rows into a logits buffer and selects with the ragged top-k
PREFILL_FUSED_TOPK = True


def _score_chunk(q, keys, key_scales, weights, ks, ke, out, clean: bool) -> None:
    """Ragged logits of one chunk of queries into ``out`` (the weighted-ReLU
    fp8 MQA score of lightning.py:116-162, every key j in [ks, ke))."""
    ops.mqa_logits(q, keys, key_scales, weights, ks, ke, out, clean_logits=clean)
