"""Tensor-level adapters over the C ABI (include/dsa_amd.h).

Every function here validates shapes, dtypes, devices and strides the way the
reference's ``TensorMatcher`` checks do (dlengine/runtime/kernel/jit/sgl/
csrc/deepseek_v4/topk.cuh:350-378), then launches on the current HIP stream.
Outputs are caller-allocated wherever the reference's are; nothing here
synchronises the host, so the calls are capturable in a HIP graph.
"""
from __future__ import annotations

import torch

from . import _lib

MLA_ROW_BYTES = 656
MLA_D_QK = 576
MLA_D_V = 512
INDEXER_HEADS = 64
INDEXER_HEAD_DIM = 128
INDEXER_ROW_BYTES = INDEXER_HEAD_DIM + 4


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require(cond: bool, msg: str, exc=RuntimeError) -> None:
    if not cond:
        raise exc(msg)


def _check_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        _require(t.is_cuda, f"tensor on {t.device}: the DSA path runs on the GPU only")
        _require(t.device == dev, f"tensors on different devices: {t.device} vs {dev}")
    return dev


def _as_bytes(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


# --------------------------------------------------------------------------- device info
def num_cus(device: int | torch.device | None = None) -> int:
    if device is None:
        device = torch.cuda.current_device()
    if isinstance(device, torch.device):
        device = device.index if device.index is not None else torch.cuda.current_device()
    return int(_lib.load().dsa_num_cus(int(device)))


def topk_max_len() -> int:
    return int(_lib.load().dsa_topk_max_len())


# --------------------------------------------------------------------------- indexer
def indexer_schedule(context_lens: torch.Tensor, page_size: int) -> torch.Tensor:
    cl = context_lens if context_lens.dim() == 2 else context_lens.reshape(-1, 1)
    cl = cl.to(torch.int32).contiguous()
    dev = _check_cuda(cl)
    out = torch.empty(cl.shape[0] + 1, dtype=torch.int32, device=dev)
    _lib.call("dsa_indexer_schedule", cl.data_ptr(), cl.shape[0], cl.shape[1], int(page_size),
              out.data_ptr(), _stream(dev))
    return out


def indexer_logits(q_fp8: torch.Tensor, kv_cache: torch.Tensor, weights: torch.Tensor,
                   context_lens: torch.Tensor, block_tables: torch.Tensor, max_context_len: int,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """fp8 paged indexer logits [B*n, max_context_len] f32 (see dsa_indexer_logits)."""
    _require(q_fp8.dim() == 4, f"q_fp8 must be [B, next_n, H, D], got {tuple(q_fp8.shape)}")
    B, n, H, D = q_fp8.shape
    _require(q_fp8.dtype in (torch.float8_e4m3fn, torch.uint8), f"q_fp8 dtype {q_fp8.dtype}")
    _require(q_fp8.is_contiguous(), "q_fp8 must be contiguous")
    _require(kv_cache.dtype in (torch.uint8, torch.float8_e4m3fn), f"kv_cache dtype {kv_cache.dtype}")
    _require(kv_cache.is_contiguous(), "kv_cache must be contiguous")
    num_pages = kv_cache.shape[0]
    _require(kv_cache.numel() % max(num_pages, 1) == 0, "kv_cache shape")
    page_bytes = kv_cache.numel() // max(num_pages, 1)
    _require(page_bytes % (D + 4) == 0, f"kv_cache page of {page_bytes} B is not page_size*{D + 4}")
    page_size = page_bytes // (D + 4)
    _require(weights.dtype == torch.float32 and tuple(weights.shape) == (B * n, H),
             f"weights must be f32 [{B * n}, {H}], got {weights.dtype} {tuple(weights.shape)}")
    weights = weights.contiguous()
    cl = context_lens.reshape(B, -1)
    _require(cl.shape[1] == n, f"context_lens must be [B, next_n]={B, n}, got {tuple(context_lens.shape)}")
    cl = cl.to(torch.int32).contiguous()
    _require(block_tables.dim() == 2 and block_tables.shape[0] == B, "block_tables must be [B, M]")
    bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    _require(bt.stride(1) == 1, "block_tables rows must be contiguous")
    _require(bt.shape[1] * page_size >= max_context_len, "block_tables too narrow for max_context_len")
    dev = _check_cuda(q_fp8, kv_cache, weights, cl, bt)
    if out is None:
        out = torch.empty(B * n, max_context_len, dtype=torch.float32, device=dev)
    _require(out.dtype == torch.float32 and out.shape[0] == B * n and out.shape[1] >= max_context_len
             and out.stride(1) == 1, "logits output must be f32 [B*n, >=max_ctx] with unit column stride")
    _lib.call("dsa_indexer_logits", _as_bytes(q_fp8).data_ptr(), _as_bytes(kv_cache).data_ptr(),
              weights.data_ptr(), cl.data_ptr(), bt.data_ptr(), bt.stride(0), B, n, H, D, page_size,
              int(max_context_len), out.data_ptr(), out.stride(0), _stream(dev))
    return out


def indexer_topk_workspace_bytes(batch: int, next_n: int, max_context_len: int) -> int:
    return int(_lib.load().dsa_indexer_topk_workspace_bytes(batch, next_n, int(max_context_len)))


def indexer_topk(q_fp8: torch.Tensor, kv_cache: torch.Tensor, weights: torch.Tensor,
                 context_lens: torch.Tensor, block_tables: torch.Tensor, max_context_len: int, top_k: int,
                 out_physical: torch.Tensor, out_logical: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None,
                 phase_events: list | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Fused indexer + exact top-k + page translation (see dsa_indexer_topk):
    the same result as topk_transform over indexer_logits, without the logits.
    ``phase_events``: optional five torch.cuda.Event recorded before the first
    launch and after the sample, filter and select phases (the last two both
    after the select, which also redoes rows whose list was unusable), on the
    current stream."""
    _require(q_fp8.dim() == 4, f"q_fp8 must be [B, next_n, H, D], got {tuple(q_fp8.shape)}")
    B, n, H, D = q_fp8.shape
    _require(q_fp8.dtype in (torch.float8_e4m3fn, torch.uint8) and q_fp8.is_contiguous(), "q_fp8 fp8 contiguous")
    _require(kv_cache.dtype in (torch.uint8, torch.float8_e4m3fn) and kv_cache.is_contiguous(), "kv_cache bytes")
    num_pages = kv_cache.shape[0]
    page_bytes = kv_cache.numel() // max(num_pages, 1)
    _require(page_bytes % (D + 4) == 0, f"kv_cache page of {page_bytes} B is not page_size*{D + 4}")
    page_size = page_bytes // (D + 4)
    _require(weights.dtype == torch.float32 and tuple(weights.shape) == (B * n, H), "weights must be f32 [B*n, H]")
    weights = weights.contiguous()
    cl = context_lens.reshape(B, -1)
    _require(cl.shape[1] == n, f"context_lens must be [B, next_n]={B, n}, got {tuple(context_lens.shape)}")
    cl = cl.to(torch.int32).contiguous()
    _require(block_tables.dim() == 2 and block_tables.shape[0] == B, "block_tables must be [B, M]")
    bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    _require(bt.stride(1) == 1, "block_tables rows must be contiguous")
    _require(bt.shape[1] * page_size >= max_context_len, "block_tables too narrow for max_context_len")
    for o in (out_physical, out_logical):
        if o is not None:
            _require(o.dtype == torch.int32 and tuple(o.shape) == (B * n, top_k) and o.is_contiguous(),
                     f"outputs must be int32 [{B * n}, {top_k}] contiguous")
    dev = _check_cuda(q_fp8, kv_cache, weights, cl, bt, out_physical)
    need = indexer_topk_workspace_bytes(B, n, max_context_len)
    if workspace is None:
        workspace = torch.zeros(need, dtype=torch.uint8, device=dev)
    _require(workspace.dtype == torch.uint8 and workspace.numel() >= need, f"workspace needs {need} bytes")
    _lib.call("dsa_indexer_topk", _as_bytes(q_fp8).data_ptr(), _as_bytes(kv_cache).data_ptr(),
              weights.data_ptr(), cl.data_ptr(), bt.data_ptr(), bt.stride(0), B, n, H, D, page_size,
              int(max_context_len), int(top_k), out_physical.data_ptr(),
              out_logical.data_ptr() if out_logical is not None else None, workspace.data_ptr(),
              workspace.numel(), _stream(dev), _event_array(phase_events))
    return out_physical, out_logical


def _event_array(events):
    if not events:
        return None
    import ctypes
    handles = []
    for e in events:
        if e is None:
            handles.append(None)
        else:
            if e.cuda_event == 0:  # torch creates the HIP event lazily
                e.record()
            handles.append(e.cuda_event)
    return (ctypes.c_void_p * len(handles))(*handles)


# --------------------------------------------------------------------------- top-k
_TOPK_WS: dict = {}
# buffers replaced by a larger one: kept alive because a captured HIP graph may
# still hold their addresses (never freed before the process ends)
_TOPK_WS_RETIRED: list = []


def topk_workspace_bytes(batch: int) -> int:
    return int(_lib.load().dsa_topk_workspace_bytes(batch))


def topk_workspace(batch: int, device: torch.device) -> torch.Tensor:
    """Workspace for the top-k entry points, cached per (device, stream) and
    grown on demand; calls on one stream are ordered, so sharing is safe. A
    buffer that is outgrown stays allocated (graphs may have captured it)."""
    need = int(_lib.load().dsa_topk_workspace_bytes(batch))
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _TOPK_WS.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _TOPK_WS_RETIRED.append(ws)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
        _TOPK_WS[key] = ws
    return ws


def _ws_args(ws):
    """(pointer, bytes) for a workspace tensor; False selects the path that
    needs no workspace (the full multi-pass exact select)."""
    return (None, 0) if ws is None or ws is False else (ws.data_ptr(), ws.numel())


def topk_transform(scores: torch.Tensor, seq_lens: torch.Tensor, page_tables: torch.Tensor,
                   out_page_indices: torch.Tensor, page_size: int, top_k: int,
                   out_raw_indices: torch.Tensor | None = None,
                   workspace=None) -> None:
    if top_k not in (512, 2048):
        raise ValueError(f"top_k must be 512 or 2048, got {top_k}")
    _require(scores.dim() == 2 and scores.dtype == torch.float32 and scores.stride(1) == 1,
             "scores must be f32 [B, S] with unit column stride")
    B = scores.shape[0]
    _require(seq_lens.dtype == torch.int32 and tuple(seq_lens.shape) == (B,) and seq_lens.is_contiguous(),
             "seq_lens must be contiguous int32 [B]")
    _require(page_tables.dim() == 2 and page_tables.shape[0] == B and page_tables.dtype == torch.int32
             and page_tables.stride(1) == 1, "page_tables must be int32 [B, P] with unit column stride")
    for name, t in (("out_page_indices", out_page_indices), ("out_raw_indices", out_raw_indices)):
        if t is not None:
            _require(t.dtype == torch.int32 and tuple(t.shape) == (B, top_k) and t.is_contiguous(),
                     f"{name} must be contiguous int32 [{B}, {top_k}]")
    if page_size <= 0 or page_size & (page_size - 1):
        raise RuntimeError("page_size must be power of 2")
    dev = _check_cuda(scores, seq_lens, page_tables, out_page_indices)
    if workspace is None:
        workspace = topk_workspace(B, dev)
    _lib.call("dsa_topk_transform", scores.data_ptr(), scores.stride(0), seq_lens.data_ptr(),
              page_tables.data_ptr(), page_tables.stride(0), out_page_indices.data_ptr(),
              _ptr(out_raw_indices), B, scores.shape[1], int(page_size), int(top_k), *_ws_args(workspace),
              _stream(dev))


def topk_transform_raw(scores: torch.Tensor, seq_lens: torch.Tensor, out_indices: torch.Tensor,
                       top_k: int, workspace=None) -> None:
    """Exact top-k positions without translation (``page_table`` NULL in the C ABI)."""
    if top_k not in (512, 2048):
        raise ValueError(f"top_k must be 512 or 2048, got {top_k}")
    _require(scores.dim() == 2 and scores.dtype == torch.float32 and scores.stride(1) == 1,
             "scores must be f32 [B, S] with unit column stride")
    B = scores.shape[0]
    _require(seq_lens.dtype == torch.int32 and tuple(seq_lens.shape) == (B,) and seq_lens.is_contiguous(),
             "seq_lens must be contiguous int32 [B]")
    _require(out_indices.dtype == torch.int32 and tuple(out_indices.shape) == (B, top_k)
             and out_indices.is_contiguous(), f"out_indices must be contiguous int32 [{B}, {top_k}]")
    dev = _check_cuda(scores, seq_lens, out_indices)
    if workspace is None:
        workspace = topk_workspace(B, dev)
    _lib.call("dsa_topk_transform", scores.data_ptr(), scores.stride(0), seq_lens.data_ptr(), None, 0,
              out_indices.data_ptr(), None, B, scores.shape[1], 1, int(top_k), *_ws_args(workspace),
              _stream(dev))


def indexer_select(logits: torch.Tensor, context_lens: torch.Tensor, out_indices: torch.Tensor,
                   top_k: int, workspace=None) -> None:
    """The portable selection tail of the decode indexer: exact top-k positions
    among [0, context_lens[r]) with non-finite and |x| >= 1e30 logits ranked as
    -inf, ascending, -1 padded (``dsa_indexer_select``)."""
    if top_k not in (512, 2048):
        raise ValueError(f"top_k must be 512 or 2048, got {top_k}")
    _require(logits.dim() == 2 and logits.dtype == torch.float32 and logits.stride(1) == 1,
             "logits must be f32 [rows, S] with unit column stride")
    R = logits.shape[0]
    _require(context_lens.dtype == torch.int32 and tuple(context_lens.shape) == (R,)
             and context_lens.is_contiguous(), "context_lens must be contiguous int32 [rows]")
    _require(out_indices.dtype == torch.int32 and tuple(out_indices.shape) == (R, top_k)
             and out_indices.is_contiguous(), f"out_indices must be contiguous int32 [{R}, {top_k}]")
    dev = _check_cuda(logits, context_lens, out_indices)
    if workspace is None:
        workspace = topk_workspace(R, dev)
    _lib.call("dsa_indexer_select", logits.data_ptr(), logits.stride(0), context_lens.data_ptr(),
              out_indices.data_ptr(), R, logits.shape[1], int(top_k), *_ws_args(workspace), _stream(dev))


def topk_transform_ragged(scores: torch.Tensor, seq_lens: torch.Tensor, row_starts: torch.Tensor,
                          offsets: torch.Tensor, out_indices: torch.Tensor, top_k: int,
                          workspace=None) -> None:
    if top_k != 2048:
        raise ValueError(f"ragged Indexer top_k must be 2048, got {top_k}")
    _require(scores.dim() == 2 and scores.dtype == torch.float32 and scores.stride(1) == 1,
             "scores must be f32 [B, S] with unit column stride")
    B = scores.shape[0]
    for name, t in (("seq_lens", seq_lens), ("row_starts", row_starts), ("offsets", offsets)):
        _require(t.dtype == torch.int32 and tuple(t.shape) == (B,) and t.is_contiguous(),
                 f"{name} must be contiguous int32 [B]")
    _require(out_indices.dtype == torch.int32 and tuple(out_indices.shape) == (B, top_k)
             and out_indices.is_contiguous(), "out_indices must be contiguous int32 [B, top_k]")
    dev = _check_cuda(scores, seq_lens, row_starts, offsets, out_indices)
    if workspace is None:
        workspace = topk_workspace(B, dev)
    _lib.call("dsa_topk_transform_ragged", scores.data_ptr(), scores.stride(0), seq_lens.data_ptr(),
              row_starts.data_ptr(), offsets.data_ptr(), out_indices.data_ptr(), B, scores.shape[1],
              int(top_k), *_ws_args(workspace), _stream(dev))


def topk_to_physical(topk_indices: torch.Tensor, block_table: torch.Tensor, block_size: int,
                     rows_per_table: int = 1, out: torch.Tensor | None = None) -> torch.Tensor:
    _require(topk_indices.dim() == 2 and topk_indices.dtype == torch.int32 and topk_indices.stride(1) == 1,
             "topk_indices must be int32 [rows, topk] with unit column stride")
    rows, k = topk_indices.shape
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    _require(bt.dim() == 2 and bt.stride(1) == 1, "block_table must be 2-D with unit column stride")
    _require(rows == bt.shape[0] * rows_per_table,
             f"rows {rows} != block_table rows {bt.shape[0]} x rows_per_table {rows_per_table}")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    dev = _check_cuda(topk_indices, bt)
    if out is None:
        out = torch.empty(rows, k, dtype=torch.int32, device=dev)
    _lib.call("dsa_topk_to_physical", topk_indices.data_ptr(), topk_indices.stride(0), bt.data_ptr(),
              bt.stride(0), bt.shape[1], rows, k, int(rows_per_table), int(block_size), out.data_ptr(),
              _stream(dev))
    return out


# --------------------------------------------------------------------------- sparse MLA
def mla_kv_geometry(k_cache: torch.Tensor) -> tuple[int, int]:
    """(block stride in bytes, rows per block) of an fp8 MLA cache view
    [num_blocks, block_size, (1,) 656] whose block stride may include the
    padding row (dlengine/runtime/context/cache/mla.py:164-182)."""
    _require(k_cache.dtype in (torch.uint8, torch.float8_e4m3fn), f"k_cache dtype {k_cache.dtype}")
    _require(k_cache.shape[-1] == MLA_ROW_BYTES and k_cache.stride(-1) == 1,
             f"k_cache rows must be {MLA_ROW_BYTES} contiguous bytes")
    _require(k_cache.dim() in (3, 4), "k_cache must be [blocks, block_size, (1,) 656]")
    if k_cache.dim() == 4:
        _require(k_cache.shape[2] == 1, "MLA cache has one KV head")
    _require(k_cache.stride(1) == MLA_ROW_BYTES, "rows inside a block must be 656 B apart")
    return k_cache.stride(0), k_cache.shape[1]


def sparse_mla_workspace_bytes(num_tokens: int, num_heads: int, num_splits: int) -> int:
    return int(_lib.load().dsa_sparse_mla_workspace_bytes(num_tokens, num_heads, num_splits))


def sparse_mla_num_splits(num_tokens: int, num_heads: int, topk: int, device=None) -> int:
    return int(_lib.load().dsa_sparse_mla_num_splits(num_tokens, num_heads, topk, num_cus(device)))


def sparse_mla_decode(q: torch.Tensor, k_cache: torch.Tensor, indices: torch.Tensor, sm_scale: float,
                      out: torch.Tensor | None = None, lse: torch.Tensor | None = None,
                      num_splits: int | None = None,
                      workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """q [T,H,576] bf16, indices [T,topk] int32 physical slots -> (o [T,H,512] bf16, lse [T,H] f32)."""
    _require(q.dim() == 3 and q.shape[2] == MLA_D_QK and q.dtype == torch.bfloat16 and q.stride(2) == 1,
             f"q must be bf16 [T, H, {MLA_D_QK}] with a contiguous last dim")
    T, H, _ = q.shape
    _require(indices.dim() == 2 and indices.shape[0] == T and indices.dtype == torch.int32
             and indices.stride(1) == 1, "indices must be int32 [T, topk] with unit column stride")
    topk = indices.shape[1]
    blk_stride, block_size = mla_kv_geometry(k_cache)
    dev = _check_cuda(q, k_cache, indices)
    if out is None:
        out = torch.empty(T, H, MLA_D_V, dtype=torch.bfloat16, device=dev)
    if lse is None:
        lse = torch.empty(T, H, dtype=torch.float32, device=dev)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H, MLA_D_V) and out.is_contiguous(),
             "out must be contiguous bf16 [T, H, 512]")
    _require(lse.dtype == torch.float32 and tuple(lse.shape) == (T, H) and lse.is_contiguous(),
             "lse must be contiguous f32 [T, H]")
    if num_splits is None:
        num_splits = sparse_mla_num_splits(T, H, topk, dev)
    need = sparse_mla_workspace_bytes(T, H, num_splits)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    ws_ptr = workspace.data_ptr() if (need and workspace is not None) else None
    ws_bytes = workspace.numel() * workspace.element_size() if (need and workspace is not None) else 0
    _lib.call("dsa_sparse_mla_decode", q.data_ptr(), q.stride(0), q.stride(1), _as_bytes(k_cache).data_ptr(),
              blk_stride, block_size, k_cache.shape[0], indices.data_ptr(), indices.stride(0), T, H, topk,
              float(sm_scale),
              out.data_ptr(), lse.data_ptr(), int(num_splits), ws_ptr, ws_bytes, _stream(dev))
    return out, lse


# --------------------------------------------------------------------------- cache writers
def _slots(slot_mapping: torch.Tensor, n: int) -> tuple[torch.Tensor, int]:
    _require(slot_mapping.dim() == 1 and slot_mapping.shape[0] >= n, "slot_mapping must be 1-D with >= n entries")
    _require(slot_mapping.dtype in (torch.int32, torch.int64), f"slot_mapping dtype {slot_mapping.dtype}")
    s = slot_mapping.contiguous()
    return s, int(s.dtype == torch.int64)


def mla_kv_store(kv: torch.Tensor, k_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Quantise kv [N, (1,) 576] bf16 into the fp8 MLA cache at slot_mapping (see dsa_mla_kv_store)."""
    kv2 = kv.reshape(kv.shape[0], -1)
    _require(kv2.shape[1] == MLA_D_QK and kv2.dtype == torch.bfloat16 and kv2.stride(1) == 1,
             f"kv must be bf16 [N, {MLA_D_QK}] with a contiguous last dim")
    blk_stride, block_size = mla_kv_geometry(k_cache)
    slots, is64 = _slots(slot_mapping, kv2.shape[0])
    dev = _check_cuda(kv2, k_cache, slots)
    _lib.call("dsa_mla_kv_store", kv2.data_ptr(), kv2.stride(0), slots.data_ptr(), is64, kv2.shape[0],
              _as_bytes(k_cache).data_ptr(), blk_stride, block_size, _stream(dev))


def indexer_k_store(key: torch.Tensor, cache: torch.Tensor, slot_mapping: torch.Tensor, page_size: int) -> None:
    """Quantise indexer keys [N, 128] bf16 into the split page layout (see dsa_indexer_k_store)."""
    _require(key.dim() == 2 and key.shape[1] == INDEXER_HEAD_DIM and key.dtype == torch.bfloat16
             and key.stride(1) == 1, "key must be bf16 [N, 128] with a contiguous last dim")
    _require(cache.dtype == torch.uint8 and cache.is_contiguous()
             and cache.numel() % (page_size * INDEXER_ROW_BYTES) == 0, "cache must be contiguous uint8 pages")
    slots, is64 = _slots(slot_mapping, key.shape[0])
    dev = _check_cuda(key, cache, slots)
    _lib.call("dsa_indexer_k_store", key.data_ptr(), key.stride(0), slots.data_ptr(), is64, key.shape[0],
              cache.data_ptr(), int(page_size), _stream(dev))


# --------------------------------------------------------------------------- indexer prologue
def _rope_cache(cos_sin_cache: torch.Tensor) -> torch.Tensor:
    cs = cos_sin_cache.reshape(cos_sin_cache.shape[0], -1)
    _require(cs.shape[1] == 64 and cs.dtype == torch.float32,
             f"cos_sin_cache must be float32 [max_pos, 64], got {tuple(cos_sin_cache.shape)} {cos_sin_cache.dtype}")
    return cs.contiguous()


def _positions(positions: torch.Tensor, n: int) -> tuple[torch.Tensor, int]:
    _require(positions.dim() == 1 and positions.shape[0] == n, f"positions must be 1-D of length {n}")
    _require(positions.dtype in (torch.int32, torch.int64), f"positions dtype {positions.dtype}")
    p = positions.contiguous()
    return p, int(p.dtype == torch.int64)


def indexer_q_prologue(query: torch.Tensor, gate_weight: torch.Tensor, weight_scale: float,
                       cos_sin_cache: torch.Tensor, positions: torch.Tensor, q_fp8: torch.Tensor,
                       weights_out: torch.Tensor, rope_interleaved: bool = True) -> None:
    """RoPE -> Hadamard-128 -> UE8M0 fp8 quant -> gate scaling of the indexer query
    (see dsa_indexer_q_prologue). query [T, H, 128] bf16 contiguous; gate_weight
    [T, H] bf16 (token stride free); q_fp8 [T, H, 128] float8_e4m3fn (or uint8);
    weights_out [T, H] (or [T, H, 1]) float32, contiguous."""
    _require(query.dim() == 3 and query.shape[-1] == INDEXER_HEAD_DIM and query.dtype == torch.bfloat16
             and query.is_contiguous(), "query must be contiguous bf16 [T, H, 128]", ValueError)
    t, h = query.shape[0], query.shape[1]
    _require(gate_weight.shape == (t, h) and gate_weight.dtype == torch.bfloat16 and gate_weight.stride(1) == 1,
             f"gate_weight must be bf16 [{t}, {h}] with a contiguous last dim", ValueError)
    _require(q_fp8.shape == query.shape and q_fp8.dtype in (torch.float8_e4m3fn, torch.uint8)
             and q_fp8.is_contiguous(), "q_fp8 must be contiguous fp8 [T, H, 128]", ValueError)
    _require(weights_out.numel() == t * h and weights_out.dtype == torch.float32 and weights_out.is_contiguous(),
             "weights_out must be contiguous float32 with T*H entries", ValueError)
    cs = _rope_cache(cos_sin_cache)
    pos, pos64 = _positions(positions, t)
    dev = _check_cuda(query, gate_weight, q_fp8, weights_out, cs, pos)
    _lib.call("dsa_indexer_q_prologue", query.data_ptr(), gate_weight.data_ptr(), gate_weight.stride(0),
              float(weight_scale), cs.data_ptr(), cs.shape[0], pos.data_ptr(), pos64, t, h, int(bool(rope_interleaved)),
              _as_bytes(q_fp8).data_ptr(), weights_out.data_ptr(), _stream(dev))


def indexer_k_transform_store(key: torch.Tensor, ln_weight: torch.Tensor, ln_bias: torch.Tensor, eps: float,
                              positions: torch.Tensor, cos_sin_cache: torch.Tensor, cache: torch.Tensor,
                              slot_mapping: torch.Tensor, page_size: int) -> None:
    """LayerNorm -> RoPE -> Hadamard-128 -> UE8M0 fp8 quant -> split-page store of
    indexer keys [T, 128] bf16 (see dsa_indexer_k_transform_store)."""
    _require(key.dim() == 2 and key.shape[1] == INDEXER_HEAD_DIM and key.dtype == torch.bfloat16
             and key.stride(1) == 1, "fused Indexer K path requires a bfloat16 [T, 128] key", ValueError)
    lw = ln_weight.to(torch.float32).contiguous()
    lb = ln_bias.to(torch.float32).contiguous()
    _require(lw.numel() == INDEXER_HEAD_DIM and lb.numel() == INDEXER_HEAD_DIM, "LayerNorm weight/bias must have 128 entries")
    _require(cache.dtype == torch.uint8 and cache.is_contiguous()
             and cache.numel() % (page_size * INDEXER_ROW_BYTES) == 0, "cache must be contiguous uint8 pages")
    cs = _rope_cache(cos_sin_cache)
    pos, pos64 = _positions(positions, key.shape[0])
    slots, is64 = _slots(slot_mapping, key.shape[0])
    dev = _check_cuda(key, lw, lb, cs, pos, slots, cache)
    _lib.call("dsa_indexer_k_transform_store", key.data_ptr(), key.stride(0), lw.data_ptr(), lb.data_ptr(),
              float(eps), cs.data_ptr(), cs.shape[0], pos.data_ptr(), pos64, slots.data_ptr(), is64, key.shape[0],
              cache.data_ptr(), int(page_size), _stream(dev))


# --------------------------------------------------------------------------- prefill indexer
def mqa_logits(q_fp8: torch.Tensor, kv_fp8: torch.Tensor, kv_scale: torch.Tensor, weights: torch.Tensor,
               ks: torch.Tensor, ke: torch.Tensor, out: torch.Tensor, clean_logits: bool = True) -> None:
    """Ragged fp8 MQA logits into out [M, >=N] f32 (see dsa_mqa_logits)."""
    _require(q_fp8.dim() == 3 and q_fp8.shape[1] == INDEXER_HEADS and q_fp8.shape[2] == INDEXER_HEAD_DIM
             and q_fp8.is_contiguous(), "q must be contiguous fp8 [M, 64, 128]", ValueError)
    m = q_fp8.shape[0]
    kv2 = kv_fp8.reshape(-1, INDEXER_HEAD_DIM)
    _require(kv2.is_contiguous(), "kv must be contiguous fp8 [N, 128]", ValueError)
    n = kv2.shape[0]
    sc = kv_scale.reshape(-1)
    _require(sc.numel() == n and sc.dtype == torch.float32 and sc.is_contiguous(),
             "kv scales must be contiguous f32 [N]", ValueError)
    _require(weights.shape == (m, INDEXER_HEADS) and weights.dtype == torch.float32 and weights.stride(1) == 1,
             "weights must be f32 [M, 64]", ValueError)
    for t in (ks, ke):
        _require(t.dim() == 1 and t.shape[0] == m and t.dtype == torch.int32 and t.is_contiguous(),
                 "k start/end must be contiguous int32 [M]", ValueError)
    _require(out.dim() == 2 and out.shape[0] == m and out.shape[1] >= n and out.dtype == torch.float32
             and out.stride(1) == 1, "out must be f32 [M, >=N]", ValueError)
    dev = _check_cuda(q_fp8, kv2, sc, weights, ks, ke, out)
    _lib.call("dsa_mqa_logits", _as_bytes(q_fp8).data_ptr(), _as_bytes(kv2).data_ptr(), sc.data_ptr(),
              weights.data_ptr(), weights.stride(0), ks.data_ptr(), ke.data_ptr(), m, n, INDEXER_HEADS,
              out.data_ptr(), out.stride(0), out.shape[1], int(bool(clean_logits)), _stream(dev))


def mqa_topk_workspace_bytes(num_rows: int, num_keys: int, top_k: int = 2048) -> int:
    return int(_lib.load().dsa_mqa_topk_workspace_bytes(int(num_rows), int(num_keys), int(top_k)))


def mqa_topk(q_fp8: torch.Tensor, kv_fp8: torch.Tensor, kv_scale: torch.Tensor, weights: torch.Tensor,
             ks: torch.Tensor, ke: torch.Tensor, max_len: int, out: torch.Tensor, top_k: int = 2048,
             workspace: torch.Tensor | None = None) -> None:
    """Ragged fp8 MQA logits + exact top-2048 without a logits buffer: out
    [M, 2048] int32 global key indices, -1 padded (see dsa_mqa_topk)."""
    if top_k != 2048:
        raise ValueError(f"ragged Indexer top_k must be 2048, got {top_k}")
    _require(q_fp8.dim() == 3 and q_fp8.shape[1] == INDEXER_HEADS and q_fp8.shape[2] == INDEXER_HEAD_DIM
             and q_fp8.is_contiguous(), "q must be contiguous fp8 [M, 64, 128]", ValueError)
    m = q_fp8.shape[0]
    kv2 = kv_fp8.reshape(-1, INDEXER_HEAD_DIM)
    _require(kv2.is_contiguous(), "kv must be contiguous fp8 [N, 128]", ValueError)
    n = kv2.shape[0]
    sc = kv_scale.reshape(-1)
    _require(sc.numel() == n and sc.dtype == torch.float32 and sc.is_contiguous(),
             "kv scales must be contiguous f32 [N]", ValueError)
    _require(weights.shape == (m, INDEXER_HEADS) and weights.dtype == torch.float32 and weights.stride(1) == 1,
             "weights must be f32 [M, 64]", ValueError)
    for t in (ks, ke):
        _require(t.dim() == 1 and t.shape[0] == m and t.dtype == torch.int32 and t.is_contiguous(),
                 "k start/end must be contiguous int32 [M]", ValueError)
    _require(out.dtype == torch.int32 and tuple(out.shape) == (m, top_k) and out.is_contiguous(),
             "out must be contiguous int32 [M, 2048]", ValueError)
    dev = _check_cuda(q_fp8, kv2, sc, weights, ks, ke, out)
    need = mqa_topk_workspace_bytes(m, n, top_k)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    _lib.call("dsa_mqa_topk", _as_bytes(q_fp8).data_ptr(), _as_bytes(kv2).data_ptr(), sc.data_ptr(),
              weights.data_ptr(), weights.stride(0), ks.data_ptr(), ke.data_ptr(), m, n, INDEXER_HEADS,
              int(max_len), int(top_k), out.data_ptr(), *_ws_args(workspace), _stream(dev))


def mla_prefill_kv(k_cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_q: torch.Tensor,
                   cu_seqlens_k: torch.Tensor, fresh: torch.Tensor, total_k: int, out: torch.Tensor) -> None:
    """Ragged bf16 keys [total_k, 576] of a prefill chunk: cached rows restored
    from the fp8 cache, fresh rows copied (see dsa_mla_prefill_kv)."""
    blk_stride, block_size = mla_kv_geometry(k_cache)
    _require(cu_seqlens_q.dtype == cu_seqlens_k.dtype and cu_seqlens_q.dtype in (torch.int32, torch.int64),
             "cu_seqlens_q/_k must share one dtype, int32 or int64", ValueError)
    _require(cu_seqlens_q.dim() == 1 and cu_seqlens_q.shape == cu_seqlens_k.shape and cu_seqlens_q.is_contiguous()
             and cu_seqlens_k.is_contiguous(), "cu_seqlens_q/_k must be contiguous [num_seqs + 1]", ValueError)
    num_seqs = cu_seqlens_q.numel() - 1
    _require(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == num_seqs
             and block_table.stride(1) == 1, "block_table must be int32 [num_seqs, M]", ValueError)
    _require(fresh.dtype == torch.bfloat16 and fresh.dim() == 2 and fresh.shape[1] == MLA_D_QK
             and fresh.stride(1) == 1, f"fresh must be bf16 [q, {MLA_D_QK}]", ValueError)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (total_k, MLA_D_QK) and out.stride(1) == 1,
             f"out must be bf16 [{total_k}, {MLA_D_QK}]", ValueError)
    dev = _check_cuda(k_cache, block_table, cu_seqlens_q, cu_seqlens_k, fresh, out)
    _lib.call("dsa_mla_prefill_kv", _as_bytes(k_cache).data_ptr(), blk_stride, block_size, k_cache.shape[0],
              block_table.data_ptr(), block_table.stride(0), block_table.shape[1], cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
              int(cu_seqlens_q.dtype == torch.int64), num_seqs, int(total_k), fresh.data_ptr(), fresh.stride(0),
              out.data_ptr(), out.stride(0), _stream(dev))


def prefill_windows(cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, num_queries: int, page_size: int,
                    ks: torch.Tensor, ke: torch.Tensor, status: torch.Tensor) -> None:
    """Per-query key windows [ks, ke) of a ragged prefill batch and the batch's
    status {fault bits, total keys, longest k length, most pages} (see
    dsa_prefill_windows), on the device."""
    _require(cu_seqlens_q.dtype == cu_seqlens_k.dtype and cu_seqlens_q.dtype in (torch.int32, torch.int64),
             "cu_seqlens_q/_k must share one dtype, int32 or int64", ValueError)
    _require(cu_seqlens_q.dim() == 1 and cu_seqlens_q.shape == cu_seqlens_k.shape and cu_seqlens_q.numel() >= 2
             and cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous(),
             "cu_seqlens_q/_k must be contiguous [num_seqs + 1], num_seqs >= 1", ValueError)
    for t in (ks, ke):
        _require(t.dtype == torch.int32 and tuple(t.shape) == (num_queries,) and t.is_contiguous(),
                 "ks/ke must be contiguous int32 [num_queries]", ValueError)
    _require(status.dtype == torch.int64 and status.numel() == 4 and status.is_contiguous(),
             "status must be contiguous int64 [4]", ValueError)
    dev = _check_cuda(cu_seqlens_q, cu_seqlens_k, ks, ke, status)
    _lib.call("dsa_prefill_windows", cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
              int(cu_seqlens_q.dtype == torch.int64), cu_seqlens_q.numel() - 1, int(num_queries), int(page_size),
              ks.data_ptr(), ke.data_ptr(), status.data_ptr(), _stream(dev))


def gather_indexer_cache(cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_k: torch.Tensor,
                         page_size: int, total_k: int, key_out: torch.Tensor, scale_out: torch.Tensor) -> None:
    """Paged indexer pages -> ragged keys [total_k, 128] and scale bytes [total_k, 4]
    (see dsa_gather_indexer_cache)."""
    _require(cu_seqlens_k.dtype in (torch.int32, torch.int64), "cu_seqlens_k must be int32 or int64", ValueError)
    _require(block_table.dtype == torch.int32, "block_table must be int32", ValueError)
    _require(key_out.shape == (total_k, INDEXER_HEAD_DIM) and key_out.dtype == torch.uint8
             and key_out.is_contiguous(), "key_out must be contiguous uint8 [total_k, 128]", ValueError)
    _require(scale_out.shape == (total_k, 4) and scale_out.dtype == torch.uint8 and scale_out.is_contiguous(),
             "scale_out must be contiguous uint8 [total_k, 4]", ValueError)
    dev = _check_cuda(cache, block_table, cu_seqlens_k, key_out, scale_out)
    _lib.call("dsa_gather_indexer_cache", cache.data_ptr(), cache.stride(0), int(page_size), INDEXER_HEAD_DIM,
              block_table.data_ptr(), block_table.stride(0), cu_seqlens_k.data_ptr(),
              int(cu_seqlens_k.dtype == torch.int64), block_table.shape[0], int(total_k), key_out.data_ptr(),
              scale_out.data_ptr(), _stream(dev))


def sparse_mla_prefill(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor, sm_scale: float,
                       out: torch.Tensor | None = None, max_logits: torch.Tensor | None = None,
                       lse: torch.Tensor | None = None):
    """Sparse MLA prefill (see dsa_sparse_mla_prefill): q [T, H, 576] bf16, kv
    [s_kv, 576] bf16 (row stride free), indices [T, topk] int32 into kv.
    Returns (out [T, H, 512] bf16, max_logits [T, H] f32, lse [T, H] f32)."""
    _require(q.dim() == 3 and q.shape[2] == MLA_D_QK and q.dtype == torch.bfloat16 and q.stride(2) == 1,
             f"q must be bf16 [T, H, 576] with a contiguous last dim, got {tuple(q.shape)} {q.dtype}", ValueError)
    kv2 = kv.reshape(kv.shape[0], -1) if kv.dim() == 3 else kv
    _require(kv2.dim() == 2 and kv2.shape[1] == MLA_D_QK and kv2.dtype == torch.bfloat16 and kv2.stride(1) == 1,
             f"kv must be bf16 [s_kv, 576] (or [s_kv, 1, 576]), got {tuple(kv.shape)} {kv.dtype}", ValueError)
    T, H, _ = q.shape
    _require(indices.dim() == 2 and indices.shape[0] == T and indices.dtype == torch.int32
             and indices.stride(1) == 1, "indices must be int32 [T, topk]", ValueError)
    topk = indices.shape[1]
    dev = _check_cuda(q, kv2, indices)
    if out is None:
        out = torch.empty(T, H, MLA_D_V, dtype=torch.bfloat16, device=dev)
    if max_logits is None:
        max_logits = torch.empty(T, H, dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty(T, H, dtype=torch.float32, device=dev)
    _require(out.shape == (T, H, MLA_D_V) and out.dtype == torch.bfloat16 and out.is_contiguous(),
             "out must be contiguous bf16 [T, H, 512]", ValueError)
    for t_, nm in ((max_logits, "max_logits"), (lse, "lse")):
        _require(t_.shape == (T, H) and t_.dtype == torch.float32 and t_.is_contiguous(),
                 f"{nm} must be contiguous f32 [T, H]", ValueError)
    _lib.call("dsa_sparse_mla_prefill", q.data_ptr(), q.stride(0), q.stride(1), kv2.data_ptr(), kv2.stride(0),
              kv2.shape[0], indices.data_ptr(), indices.stride(0), T, H, topk, float(sm_scale), out.data_ptr(),
              max_logits.data_ptr(), lse.data_ptr(), _stream(dev))
    return out, max_logits, lse


def sparse_mla_prefill_paged_workspace_bytes(num_tokens: int, topk: int) -> int:
    return int(_lib.load().dsa_sparse_mla_prefill_paged_workspace_bytes(num_tokens, topk))


def sparse_mla_prefill_paged(q: torch.Tensor, k_cache: torch.Tensor, block_table: torch.Tensor,
                             cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, fresh: torch.Tensor,
                             indices: torch.Tensor, sm_scale: float, total_k: int,
                             out: torch.Tensor | None = None, max_logits: torch.Tensor | None = None,
                             lse: torch.Tensor | None = None, workspace: torch.Tensor | None = None):
    """Sparse MLA prefill with the cached keys read from the paged fp8 cache and
    the fresh keys from bf16 rows (see dsa_sparse_mla_prefill_paged). indices
    [T, topk] int32 are positions in the ragged key order of total_k keys.
    Returns (out [T, H, 512] bf16, max_logits [T, H] f32, lse [T, H] f32)."""
    _require(q.dim() == 3 and q.shape[2] == MLA_D_QK and q.dtype == torch.bfloat16 and q.stride(2) == 1,
             f"q must be bf16 [T, H, 576] with a contiguous last dim, got {tuple(q.shape)} {q.dtype}", ValueError)
    blk_stride, block_size = mla_kv_geometry(k_cache)
    T, H, _ = q.shape
    _require(indices.dim() == 2 and indices.shape[0] == T and indices.dtype == torch.int32
             and indices.stride(1) == 1, "indices must be int32 [T, topk]", ValueError)
    _require(cu_seqlens_q.dtype == cu_seqlens_k.dtype and cu_seqlens_q.dtype in (torch.int32, torch.int64)
             and cu_seqlens_q.shape == cu_seqlens_k.shape and cu_seqlens_q.dim() == 1
             and cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous(),
             "cu_seqlens_q/_k must be contiguous int32 or int64 [num_seqs + 1] of one dtype", ValueError)
    num_seqs = cu_seqlens_q.numel() - 1
    _require(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == num_seqs
             and block_table.stride(1) == 1, "block_table must be int32 [num_seqs, M]", ValueError)
    f2 = fresh.reshape(fresh.shape[0], -1) if fresh.dim() == 3 else fresh
    _require(f2.dim() == 2 and f2.shape[1] == MLA_D_QK and f2.dtype == torch.bfloat16 and f2.stride(1) == 1,
             "fresh must be bf16 [total_q, 576]", ValueError)
    topk = indices.shape[1]
    dev = _check_cuda(q, k_cache, block_table, cu_seqlens_q, cu_seqlens_k, f2, indices)
    if out is None:
        out = torch.empty(T, H, MLA_D_V, dtype=torch.bfloat16, device=dev)
    if max_logits is None:
        max_logits = torch.empty(T, H, dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty(T, H, dtype=torch.float32, device=dev)
    _require(out.shape == (T, H, MLA_D_V) and out.dtype == torch.bfloat16 and out.is_contiguous(),
             "out must be contiguous bf16 [T, H, 512]", ValueError)
    for t_, nm in ((max_logits, "max_logits"), (lse, "lse")):
        _require(t_.shape == (T, H) and t_.dtype == torch.float32 and t_.is_contiguous(),
                 f"{nm} must be contiguous f32 [T, H]", ValueError)
    need = sparse_mla_prefill_paged_workspace_bytes(T, topk)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    _lib.call("dsa_sparse_mla_prefill_paged", q.data_ptr(), q.stride(0), q.stride(1), _as_bytes(k_cache).data_ptr(),
              blk_stride, block_size, k_cache.shape[0], block_table.data_ptr(), block_table.stride(0),
              block_table.shape[1], cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
              int(cu_seqlens_q.dtype == torch.int64), num_seqs,
              int(total_k), f2.data_ptr(), f2.stride(0), f2.shape[0], indices.data_ptr(), indices.stride(0), T, H,
              topk, float(sm_scale), out.data_ptr(), max_logits.data_ptr(), lse.data_ptr(), workspace.data_ptr(),
              workspace.numel(), _stream(dev))
    return out, max_logits, lse
