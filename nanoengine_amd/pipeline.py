"""The full DSA decode step on one GPU: indexer logits -> exact top-k with page
translation -> sparse MLA decode.

This is the composition ``DeepseekV2Attention.forward`` performs per layer in
decode (dlengine/runtime/models/deepseek_v2/deepseek_v2.py:1860-2018 calling
``Indexer.forward`` lightning.py:1357-1466 with ``translate_topk=True`` and then
``FlashMlaAttention.forward`` flash_mla.py:76-99). Every buffer is allocated
once in the constructor, so a step allocates nothing (capturable in a HIP
graph). By default the indexer and the top-k run fused (``ops.indexer_topk``:
the logits are never written to memory); ``fused=False`` runs them as the two
separate reference operators over a logits buffer.

Buffer ownership: a call returns views of the object's own buffers (o, lse,
logical, physical), and the next call on the same object overwrites them. A
model that runs several layers through one object passes ``out=`` / ``lse=``
per layer (its own [rows, H, 512] bf16 and [rows, H] f32 tensors) to keep each
layer's attention output. The (logical, physical) pair a full layer publishes
to an ``IndexerTopKState`` is held by reference: the next full layer on the
same object rewrites it in place, which is also the moment the reference's
state moves on to the new layer's selection (deepseek_v2.py:1917-1950), so the
shared layers in between read the pair of the full layer before them.
"""
from __future__ import annotations

import torch

from . import ops
from .state import IndexerTopKState


class DsaDecodeStep:
    def __init__(self, batch: int, next_n: int, max_context_len: int, num_heads: int = 128,
                 index_topk: int = 2048, page_size: int = 64, device="cuda", fused: bool = True):
        self.batch, self.next_n, self.max_ctx = batch, next_n, max_context_len
        self.num_heads, self.topk, self.page_size = num_heads, index_topk, page_size
        self.fused = fused
        if fused and page_size != 64:
            # the fused kernel translates through the indexer's 64-token pages
            raise ValueError(f"the fused indexer + top-k step needs page_size 64 (the indexer page), got {page_size}")
        rows = batch * next_n
        dev = torch.device(device)
        if fused:
            self.logits = None
            self.fused_workspace = torch.zeros(ops.indexer_topk_workspace_bytes(batch, next_n, max_context_len),
                                               dtype=torch.uint8, device=dev)
        else:
            self.logits = torch.empty(rows, max_context_len, dtype=torch.float32, device=dev)
        self.logical = torch.empty(rows, index_topk, dtype=torch.int32, device=dev)
        self.physical = torch.empty(rows, index_topk, dtype=torch.int32, device=dev)
        self.out = torch.empty(rows, num_heads, ops.MLA_D_V, dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty(rows, num_heads, dtype=torch.float32, device=dev)
        self.num_splits = ops.sparse_mla_num_splits(rows, num_heads, index_topk, dev)
        need = ops.sparse_mla_workspace_bytes(rows, num_heads, self.num_splits)
        self.workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        self.topk_workspace = torch.empty(max(ops.topk_workspace_bytes(rows), 16), dtype=torch.uint8, device=dev)

    def expand_lens(self, context_lens: torch.Tensor) -> torch.Tensor:
        """Per-query causal lengths, flattened [batch*next_n] int32."""
        n = self.next_n
        if n == 1:
            return context_lens.to(torch.int32).reshape(-1).contiguous()
        offs = torch.arange(n - 1, -1, -1, dtype=torch.int32, device=context_lens.device)
        return (context_lens.to(torch.int32)[:, None] - offs).clamp_min(1).reshape(-1).contiguous()

    def __call__(self, q_idx_fp8: torch.Tensor, weights: torch.Tensor, indexer_cache: torch.Tensor,
                 seq_lens: torch.Tensor, block_tables: torch.Tensor, page_tables: torch.Tensor,
                 q_mla: torch.Tensor, kv_cache: torch.Tensor, sm_scale: float, *,
                 layer_idx: int | None = None, indexer_state: IndexerTopKState | None = None,
                 shared: bool = False, out: torch.Tensor | None = None, lse: torch.Tensor | None = None):
        """q_idx_fp8 [B*n, 64, 128] fp8; weights [B*n, 64] f32; indexer_cache
        [pages, 8448] uint8; seq_lens [B*n] int32 per-query lengths;
        block_tables [B, M] int32; page_tables [B*n, M] int32 (block_tables
        repeated per query token); q_mla [B*n, H, 576] bf16; kv_cache
        [blocks, 64, 1, 656] fp8 bytes. Returns (o, lse, logical, physical).

        With an ``indexer_state``, a full layer (``shared=False``) publishes its
        (logical, physical) pair under ``layer_idx``; a shared layer
        (``shared=True``) runs no indexer and attends over the published pair,
        which must match this batch's shape (deepseek_v2.py:1865-1950). The
        indexer inputs are not read on a shared layer and may be None.
        ``out`` [B*n, H, 512] bf16 and ``lse`` [B*n, H] f32, when given, receive
        this call's attention output instead of the object's own buffers."""
        o_buf = self.out if out is None else out
        lse_buf = self.lse if lse is None else lse
        if shared:
            if indexer_state is None:
                raise ValueError("a shared indexer layer needs the indexer_state of a preceding full layer")
            logical, physical = indexer_state.require(layer_idx, self.batch * self.next_n, self.topk,
                                                      require_physical=True)
            ops.sparse_mla_decode(q_mla, kv_cache, physical, sm_scale, out=o_buf, lse=lse_buf,
                                  num_splits=self.num_splits, workspace=self.workspace)
            return o_buf, lse_buf, logical, physical
        B, n = self.batch, self.next_n
        q4 = q_idx_fp8.view(B, n, *q_idx_fp8.shape[1:])
        if self.fused:
            ops.indexer_topk(q4, indexer_cache, weights, seq_lens.view(B, n), block_tables, self.max_ctx,
                             self.topk, self.physical, self.logical, workspace=self.fused_workspace)
        else:
            ops.indexer_logits(q4, indexer_cache, weights, seq_lens.view(B, n), block_tables, self.max_ctx,
                               out=self.logits)
            ops.topk_transform(self.logits, seq_lens, page_tables, self.physical, self.page_size, self.topk,
                               self.logical, workspace=self.topk_workspace)
        if indexer_state is not None:
            indexer_state.publish(layer_idx, self.logical, self.physical)
        ops.sparse_mla_decode(q_mla, kv_cache, self.physical, sm_scale, out=o_buf, lse=lse_buf,
                              num_splits=self.num_splits, workspace=self.workspace)
        return o_buf, lse_buf, self.logical, self.physical
