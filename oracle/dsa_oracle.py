"""CPU restatement of the reference DSA decode path, in numpy.

TEST INFRASTRUCTURE ONLY. Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker; nothing in
``nanoengine_amd`` imports it, and it is never what is measured or shipped.

Every function cites the reference file:line it follows (paths relative to the
reference repository root, package ``dlengine``). Numerics:

* fp8 is OCP ``float8_e4m3fn`` (bias 7, no infinities, 0x7f/0xff = NaN,
  max finite 448), stored as raw ``uint8`` bytes.
* bf16 is stored as raw ``uint16`` (the upper half of an IEEE f32).
* Accumulation is float64 unless stated, so the oracle sits closer to the exact
  value than any fp32 kernel; tolerances in the tests absorb the kernels'
  fp32 accumulation order.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "FP8_MAX", "assemble_prefill_kv", "D_NOPE", "D_ROPE", "D_QK", "MLA_ROW_BYTES", "MLA_TILE",
    "fp8_e4m3fn_decode", "fp8_e4m3fn_encode", "bf16_to_f32", "f32_to_bf16",
    "ue8m0_ceil", "quantize_rows_ue8m0", "pack_indexer_cache", "indexer_cache_token",
    "quantize_mla_rows", "unpack_mla_rows", "dequant_mla_rows",
    "expand_decode_context_lens", "indexer_logits", "indexer_logits_bruteforce",
    "fp8_dot_error_bound", "indexer_logit_error_bound", "MFMA_FP8_BITS", "F32_EPS",
    "topk_select", "topk_transform", "topk_transform_ragged",
    "topk_indices_to_physical", "sparse_mla_decode", "indexer_decode_topk",
    "rope_cos_sin_cache", "interleaved_to_half", "rope_neox", "hadamard128", "f32_tree_sum128",
    "indexer_q_prologue", "indexer_k_transform", "mqa_logits", "gather_indexer_cache",
    "prefill_ks_ke", "sparse_mla_prefill",
]

FP8_MAX = 448.0
D_NOPE = 512          # fp8_utils.py:13
D_ROPE = 64           # fp8_utils.py:14
D_QK = D_NOPE + D_ROPE
MLA_TILE = 128        # fp8_utils.py:16
MLA_ROW_BYTES = D_NOPE + (D_NOPE // MLA_TILE) * 4 + D_ROPE * 2   # 656, fp8_utils.py:21
INDEXER_HEAD_DIM = 128
INDEXER_ROW_BYTES = INDEXER_HEAD_DIM + 4                            # 132, lightning.py:411-413


# --------------------------------------------------------------------------- fp8 / bf16
def _build_e4m3fn_table() -> np.ndarray:
    """Decode table for all 256 e4m3fn codes, from the OCP bit layout."""
    tab = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            tab[code] = np.nan
        elif e == 0:
            tab[code] = s * m * 2.0 ** -9          # subnormal: m/8 * 2^(1-7)
        else:
            tab[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return tab


_E4M3_TABLE = _build_e4m3fn_table()
_E4M3_POS = _E4M3_TABLE[:127]                        # codes 0..126: 0 .. 448, increasing


def fp8_e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values."""
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def fp8_e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """float -> e4m3fn codes, round-to-nearest-even, NaN for |x| beyond the
    rounding range of 448 (the non-saturating cast ``tensor.to(float8_e4m3fn)``
    used at lightning.py:92-97 and fp8_utils.py:55)."""
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    # nearest representable magnitude among the 127 finite non-negative codes
    hi = np.searchsorted(_E4M3_POS, a, side="left").clip(0, 126)
    lo = (hi - 1).clip(0, 126)
    dhi = np.abs(_E4M3_POS[hi] - a)
    dlo = np.abs(a - _E4M3_POS[lo])
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    # the next step above 448 would be 480 (the NaN code): [448, 464] rounds
    # to 448 (464 is the tie, even code wins), beyond that is NaN
    over = a > 464.0
    code = np.where(over | np.isnan(a), 0x7F, code).astype(np.uint8)
    neg = (np.signbit(x)) & ~np.isnan(a)
    return (code | np.where(neg, 0x80, 0).astype(np.uint8)).astype(np.uint8)


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, 0x7FC0, rounded).astype(np.uint16)


def ue8m0_ceil(scale: np.ndarray) -> np.ndarray:
    """Round a positive scale up to a power of two (UE8M0): lightning.py:91-92,
    fp8_utils.py:27-29 ``2^ceil(log2(s))``, and the exponent-plus-carry form of
    ``cast_to_ue8m0`` (jit/sgl/include/sgl_kernel/deepseek_v4/fp8_utils.cuh:20-26).
    Exact: from the binary exponent, not a floating log2."""
    s = np.asarray(scale, dtype=np.float32)
    m, e = np.frexp(s.astype(np.float64))          # s = m * 2^e, m in [0.5, 1)
    k = np.where(m == 0.5, e - 1, e)               # exact power of two: 2^(e-1)
    return np.ldexp(np.float64(1.0), k).astype(np.float32)


def assemble_prefill_kv(cache_rows: np.ndarray, block_size: int, block_table: np.ndarray,
                        cu_seqlens_q: np.ndarray, cu_seqlens_k: np.ndarray, fresh: np.ndarray) -> np.ndarray:
    """The sparse prefill's ragged keys [total_k, 576] float32 (bf16 values).

    Restates deepseek_v2.py:1573-1604: ``_gather_cache_cached_only``
    (mla_utils.py:200-234: the first ``k_len - q_len`` tokens of each sequence,
    through its block table), ``restore_mla_fp8_cache_rows`` (fp8_utils.py:
    180-196, the 656-byte layout -> ``dequant_mla_rows``) and
    ``_interleave_cached_fresh`` (mla_utils.py:118-165: per sequence the cached
    rows, then the fresh ones). ``cache_rows`` is the cache as [blocks *
    block_size, 656] bytes; ``fresh`` [total_q, 576] holds bf16 values."""
    cq = np.asarray(cu_seqlens_q, dtype=np.int64)
    ck = np.asarray(cu_seqlens_k, dtype=np.int64)
    parts = []
    for b in range(len(cq) - 1):
        q_len, k_len = cq[b + 1] - cq[b], ck[b + 1] - ck[b]
        cached = k_len - q_len
        slots = [int(block_table[b, i // block_size]) * block_size + i % block_size for i in range(cached)]
        if cached:
            parts.append(dequant_mla_rows(cache_rows[np.asarray(slots)]))
        parts.append(np.asarray(fresh[cq[b]:cq[b + 1]], dtype=np.float32))
    return np.concatenate(parts) if parts else np.zeros((0, D_QK), np.float32)


# --------------------------------------------------------------------------- indexer formats
def quantize_rows_ue8m0(x: np.ndarray, min_amax: float = 1e-4):
    """Per-row (128-wide) fp8 quantisation with a UE8M0 scale.

    Follows ``_per_token_cast_to_fp8_ue8m0`` lightning.py:78-101 and the
    ``quant_fp8(..., round_ue8m0=True, min_absmax=1e-4)`` call at
    lightning.py:1327-1332: ``sf = 2^ceil(log2(max(amax,1e-4)/448))``,
    ``code = e4m3fn(x / sf)``. ``x`` is [..., 128] float32 (bf16 values).
    Returns (codes uint8 [...,128], scale float32 [...]).
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=-1)
    amax = np.maximum(amax, np.float32(min_amax))
    sf = ue8m0_ceil(amax / np.float32(FP8_MAX))
    # multiply by the reciprocal as lightning.py:95 does (exact: sf is 2^k)
    codes = fp8_e4m3fn_encode(x * (np.float32(1.0) / sf)[..., None])
    return codes, sf


def pack_indexer_cache(codes: np.ndarray, scales: np.ndarray, slots: np.ndarray,
                       num_pages: int, page_size: int = 64) -> np.ndarray:
    """Scatter per-token (fp8[128], f32 scale) into the split page layout
    ``[page_size*128 fp8][page_size*4 scale]`` (lightning.py:494-507,
    IndexerCache docstring :410-413). Returns uint8 [num_pages, page_size*132]."""
    buf = np.zeros((num_pages, page_size * INDEXER_ROW_BYTES), dtype=np.uint8)
    sc_bytes = np.asarray(scales, dtype=np.float32).reshape(-1, 1).view(np.uint8)
    for tok, slot in enumerate(np.asarray(slots).tolist()):
        page, off = divmod(int(slot), page_size)
        buf[page, off * 128:(off + 1) * 128] = codes[tok]
        base = page_size * 128 + off * 4
        buf[page, base:base + 4] = sc_bytes[tok]
    return buf


def indexer_cache_token(cache: np.ndarray, slot: int, page_size: int = 64):
    """Read one token back out of the split page layout -> (codes[128], scale)."""
    page, off = divmod(int(slot), page_size)
    codes = cache[page, off * 128:(off + 1) * 128]
    base = page_size * 128 + off * 4
    scale = cache[page, base:base + 4].copy().view(np.float32)[0]
    return codes, scale


# --------------------------------------------------------------------------- MLA row format
def quantize_mla_rows(kv: np.ndarray) -> np.ndarray:
    """[N,576] bf16-valued float32 -> [N,656] uint8 packed rows.

    ``quantize_nope_fp8`` fp8_utils.py:32-58 (per-128-tile
    ``scale = 2^ceil(log2(max(amax/448, 1e-12)))``, ``code = e4m3fn(v/scale)``)
    then ``pack_mla_fp8`` fp8_utils.py:80-108 (bytes [0,512) fp8, [512,528)
    4 x f32 scales, [528,656) 64 x bf16 rope).
    """
    kv = np.asarray(kv, dtype=np.float32)
    n = kv.shape[0]
    nope = kv[:, :D_NOPE].reshape(n, D_NOPE // MLA_TILE, MLA_TILE)
    amax = np.abs(nope).max(axis=-1)
    scales = np.exp2(np.ceil(np.log2(np.maximum(amax / np.float32(FP8_MAX),
                                                np.float32(1e-12))))).astype(np.float32)
    codes = fp8_e4m3fn_encode(nope / scales[..., None]).reshape(n, D_NOPE)
    out = np.empty((n, MLA_ROW_BYTES), dtype=np.uint8)
    out[:, :D_NOPE] = codes
    out[:, D_NOPE:D_NOPE + 16] = scales.view(np.uint8).reshape(n, 16)
    out[:, D_NOPE + 16:] = f32_to_bf16(kv[:, D_NOPE:]).view(np.uint8).reshape(n, 128)
    return out


def unpack_mla_rows(rows: np.ndarray):
    """``unpack_mla_fp8`` fp8_utils.py:111-134 -> (codes [N,512], scales [N,4], rope bf16 bits [N,64])."""
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    codes = rows[:, :D_NOPE]
    scales = rows[:, D_NOPE:D_NOPE + 16].copy().view(np.float32)
    rope = rows[:, D_NOPE + 16:].copy().view(np.uint16)
    return codes, scales, rope


def dequant_mla_rows(rows: np.ndarray) -> np.ndarray:
    """``dequantize_and_unpack_mla`` fp8_utils.py:153-177 -> [N,576] float32.
    fp8 * power-of-two scale is exact in bf16, so the reference's bf16 cast
    (fp8_utils.py:76) changes nothing for finite in-range values."""
    codes, scales, rope = unpack_mla_rows(rows)
    n = codes.shape[0]
    nope = fp8_e4m3fn_decode(codes).reshape(n, 4, MLA_TILE) * scales[..., None]
    out = np.empty((n, D_QK), dtype=np.float32)
    out[:, :D_NOPE] = bf16_to_f32(f32_to_bf16(nope.reshape(n, D_NOPE)))
    out[:, D_NOPE:] = bf16_to_f32(rope)
    return out


# --------------------------------------------------------------------------- indexer
def expand_decode_context_lens(context_lens: np.ndarray, next_n: int) -> np.ndarray:
    """``_expand_decode_context_lens`` lightning.py:350-378: per-query causal
    length ``ctx - (next_n-1-j)`` clamped to >= 1, shape [B, next_n] int32."""
    c = np.asarray(context_lens)
    if c.ndim == 1:
        c = c[:, None]
    if c.ndim != 2 or c.shape[1] not in (1, next_n):
        raise ValueError(
            "Indexer context_lens must have shape [batch], [batch, 1], or "
            f"[batch, next_n]; got {tuple(c.shape)} for next_n={next_n}")
    if c.shape[1] == next_n:
        return c.astype(np.int32)
    offs = np.arange(next_n - 1, -1, -1, dtype=np.int64)
    return np.maximum(c.astype(np.int64) - offs[None, :], 1).astype(np.int32)


def indexer_logits(q_fp8: np.ndarray, kv_cache: np.ndarray, weights: np.ndarray,
                   context_lens: np.ndarray, block_tables: np.ndarray,
                   max_context_len: int, page_size: int = 64) -> np.ndarray:
    """Paged fp8 lightning-indexer logits (the contract of
    ``deep_gemm.fp8_paged_mqa_logits`` as called at lightning.py:1395-1406).

    ``logits[b*n+j, t] = sum_h w[b*n+j,h] * relu(q[b,j,h,:] . k[t,:]) * s_k[t]``
    (lightning.py:116-131 ``_weighted_relu_mqa_scores``; tilelang
    fp8_index.py:81-92; ``w`` already folds q_scale, lightning.py:1252-1273).
    q_fp8 uint8 [B,n,H,128]; kv_cache uint8 [pages, page_size*132];
    weights f32 [B*n,H]; context_lens int [B,n]; block_tables int [B,M].
    Positions t >= context_lens[b,j] are set to -inf (the reference leaves them
    unspecified; the top-k never selects them).
    """
    B, n, H, D = q_fp8.shape
    cl = expand_decode_context_lens(context_lens, n)
    out = np.full((B * n, max_context_len), -np.inf, dtype=np.float32)
    qf = fp8_e4m3fn_decode(q_fp8).astype(np.float64)
    w = np.asarray(weights, dtype=np.float64).reshape(B, n, H)
    for b in range(B):
        L = int(cl[b].max())
        if L <= 0:
            continue
        npages = (L + page_size - 1) // page_size
        pages = np.asarray(block_tables[b, :npages], dtype=np.int64)
        blk = kv_cache[pages]                                   # [np, P*132]
        k = fp8_e4m3fn_decode(blk[:, :page_size * D].reshape(-1, D)).astype(np.float64)
        s = blk[:, page_size * D:].copy().view(np.float32).reshape(-1).astype(np.float64)
        k, s = k[:L], s[:L]
        for j in range(n):
            dots = np.einsum("hd,td->ht", qf[b, j], k)          # [H, L]
            lg = (np.maximum(dots, 0.0) * w[b, j][:, None]).sum(axis=0) * s
            Lj = int(cl[b, j])
            out[b * n + j, :Lj] = lg[:Lj].astype(np.float32)
    return out


def indexer_logits_bruteforce(q: np.ndarray, w: np.ndarray, k: np.ndarray,
                              s: np.ndarray) -> np.ndarray:
    """Scalar-loop form of the weighted-ReLU score for tiny inputs (an
    independent check of :func:`indexer_logits`): q [H,D], w [H], k [T,D], s [T]."""
    H, D = q.shape
    T = k.shape[0]
    out = []
    for t in range(T):
        acc = 0.0
        for h in range(H):
            dot = 0.0
            for d in range(D):
                dot += float(q[h, d]) * float(k[t, d])
            acc += float(w[h]) * max(dot, 0.0)
        out.append(acc * float(s[t]))
    return np.asarray(out, dtype=np.float64)


# Summation model of the gfx950 scaled fp8 MFMA (v_mfma_scale_f32_16x16x128 /
# 32x32x64_f8f6f4), which the HIP indexer uses for every q . k of 128 terms.
# The instruction does not add its products exactly: bits of a product far
# below the largest one are lost (the two-product probe ``fp8_mfma_sum`` of
# ``bench.py --micro`` keeps 2^p + 1.875 exactly up to p = 10, then 1.75,
# 1.5, 1.0, then nothing: a quantum of 2^-13 of the largest product's binade),
# while sums of same-sign products of similar size are exact. The bound used
# here assumes that each of the n products and each of the n - 1 additions of
# the reduction truncates toward zero at that quantum q = 2^(E - 13), E =
# floor(log2 max_i |p_i|):
#     B = sum_i (|p_i| - |trunc(p_i / q) * q|)  +  (n - 1) * q  (+ one f32 rounding).
# Over 2.56 million random dots with values spread over 16 binades
# (``mfma_sum_bound`` of ``bench.py --micro``), the error stayed at or below
# 0.41 B (16x16x128) and 0.70 B (32x32x64); on N(0,1)-quantised operands B is
# ~0.65% of |dot| and the errors are far smaller. The reference's kernel
# (DeepGEMM on Hopper) also sums fp8 products in a limited-precision
# accumulator. This bound is what a GPU logit is held to where the 1e-3
# relative tolerance has no scale (a head sum that cancels). Pinned by the GPU
# probes above and tests/test_gpu_indexer.py::test_logits_within_the_derived_mfma_bound.
MFMA_FP8_BITS = 13
F32_EPS = 2.0 ** -24


def fp8_dot_error_bound(qf: np.ndarray, kf: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Exact dots and their error bound B on the scaled fp8 MFMA.

    qf [H, D] and kf [T, D] decoded fp8 values (float64). Returns
    (dots [T, H], bound [T, H]); bound adds one f32 rounding of the dot."""
    P = kf[:, None, :] * qf[None, :, :]                       # [T, H, D], exact in float64
    dots = P.sum(-1)
    pm = np.abs(P).max(-1)
    E = np.floor(np.log2(np.where(pm > 0, pm, 1.0)))
    quantum = np.exp2(E - MFMA_FP8_BITS)
    R = (np.abs(P) - np.abs(np.trunc(P / quantum[..., None]) * quantum[..., None])).sum(-1)
    adders = np.maximum((P != 0).sum(-1) - 1, 0) * quantum
    return dots, np.where(pm > 0, R + adders, 0.0) + F32_EPS * np.abs(dots)


def indexer_logit_error_bound(q_codes: np.ndarray, weights: np.ndarray, k_codes: np.ndarray,
                              k_scale: np.ndarray) -> np.ndarray:
    """Largest error of a GPU indexer logit against the exact value, for one
    query token: q_codes uint8 [H, 128], weights f32 [H] (q scale folded in),
    k_codes uint8 [T, 128], k_scale f32 [T]. Returns float64 [T]:

        s_t * ( sum_h |w_h| * B_h(t)  +  (H + 1) * 2^-24 * sum_h |w_h| * relu(dot_h(t)) )

    with B_h(t) the dot's bound from :func:`fp8_dot_error_bound`. The first
    term carries each dot's MFMA error through relu (1-Lipschitz) and the head
    weights; the second bounds the f32 weighted sum of H terms
    and the final product with the key scale."""
    qf = fp8_e4m3fn_decode(q_codes).astype(np.float64)
    kf = fp8_e4m3fn_decode(k_codes).astype(np.float64)
    w = np.abs(np.asarray(weights, dtype=np.float64))
    dots, R = fp8_dot_error_bound(qf, kf)
    H = qf.shape[0]
    b = R @ w + (H + 1) * F32_EPS * (np.maximum(dots, 0.0) @ w)
    return b * np.abs(np.asarray(k_scale, dtype=np.float64))


# --------------------------------------------------------------------------- top-k
def _order_keys(x: np.ndarray) -> np.ndarray:
    """Monotone uint32 key of float32 (NaN mapped to -inf first)."""
    x = np.where(np.isnan(x), -np.inf, x).astype(np.float32)
    u = x.view(np.uint32)
    return np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)


def topk_select(row: np.ndarray, length: int, k: int) -> np.ndarray:
    """Exact top-k positions of ``row[:length]``.

    Set semantics follow ``torch.topk`` on the valid prefix
    (lightning.py:1480-1482; topk.cuh:249-287 treats positions >= seq_len as
    absent). The reference leaves the order of equal values unspecified; this
    restatement fixes it: among equal scores the lowest positions win, and NaN
    ranks as -inf. Returns the selected positions sorted ascending; when
    ``length <= k`` that is ``0..length-1`` (topk.cuh:58-81).
    """
    length = int(length)
    if length <= k:
        return np.arange(max(length, 0), dtype=np.int32)
    keys = _order_keys(np.asarray(row[:length], dtype=np.float32)).astype(np.int64)
    order = np.lexsort((np.arange(length), -keys))            # key desc, index asc
    return np.sort(order[:k]).astype(np.int32)


def topk_transform(scores: np.ndarray, seq_lens: np.ndarray, page_tables: np.ndarray,
                   page_size: int, top_k: int):
    """``topk_transform`` deepseek_v4.py:324-367 -> kernel topk.cuh:249-287.

    Per row: select the top ``top_k`` positions among ``[0, seq_len)``, write
    them as logical positions (``raw``) and as physical slots
    ``(page_table[p >> bits] << bits) | (p & mask)`` (topk.cuh:52-56); pad with
    -1. Returns (page_indices, raw_indices), both int32 [B, top_k]; positions
    are in ascending order.
    """
    if top_k not in (512, 2048):
        raise ValueError(f"top_k must be 512 or 2048, got {top_k}")
    if page_size <= 0 or page_size & (page_size - 1):
        raise ValueError("page_size must be power of 2")
    bits = page_size.bit_length() - 1
    B = scores.shape[0]
    page = np.full((B, top_k), -1, dtype=np.int32)
    raw = np.full((B, top_k), -1, dtype=np.int32)
    for b in range(B):
        sel = topk_select(scores[b], int(seq_lens[b]), top_k)
        raw[b, :sel.size] = sel
        pt = np.asarray(page_tables[b], dtype=np.int64)
        page[b, :sel.size] = ((pt[sel >> bits] << bits) | (sel & (page_size - 1))).astype(np.int32)
    return page, raw


def topk_transform_ragged(scores: np.ndarray, seq_lens: np.ndarray, row_starts: np.ndarray,
                          offsets: np.ndarray, top_k: int) -> np.ndarray:
    """``topk_transform_ragged`` deepseek_v4.py:370-388 -> topk.cuh:289-316:
    top-k over ``scores[b, row_start : row_start+len]`` plus ``offsets[b]``;
    ``len <= top_k`` emits ``i + offset`` for i < len, then -1. Exact here (the
    reference's bounded candidate buffer may differ by <= 5 entries)."""
    if top_k != 2048:
        raise ValueError(f"ragged Indexer top_k must be 2048, got {top_k}")
    B = scores.shape[0]
    out = np.full((B, top_k), -1, dtype=np.int32)
    for b in range(B):
        L, r0, off = int(seq_lens[b]), int(row_starts[b]), int(offsets[b])
        sel = topk_select(scores[b, r0:r0 + max(L, 0)], L, top_k)
        out[b, :sel.size] = sel + off
    return out


def topk_indices_to_physical(topk_indices: np.ndarray, block_table: np.ndarray,
                             block_size: int) -> np.ndarray:
    """``topk_indices_to_physical`` mla_utils.py:237-272:
    ``block_table[b, idx // bs] * bs + idx % bs``, -1 preserved."""
    t = np.asarray(topk_indices, dtype=np.int64)
    valid = t >= 0
    safe = np.where(valid, t, 0)
    blk = np.take_along_axis(np.asarray(block_table, dtype=np.int64), safe // block_size, axis=1)
    phys = blk * block_size + safe % block_size
    return np.where(valid, phys, -1).astype(np.int32)


def indexer_decode_topk(logits: np.ndarray, context_lens: np.ndarray, index_topk: int) -> np.ndarray:
    """The portable selection tail of ``Indexer.forward`` lightning.py:1468-1492:
    mask ``t >= ctx`` and non-finite/|x|>=1e30 to -inf, top-k, indices >= ctx
    -> -1, pad to ``index_topk`` with -1. Returns logical positions
    (ascending, ties to the lowest position) int32 [rows, index_topk]."""
    rows, max_ctx = logits.shape
    ctx = np.asarray(context_lens).reshape(-1)
    out = np.full((rows, index_topk), -1, dtype=np.int32)
    for r in range(rows):
        L = int(ctx[r])
        x = np.asarray(logits[r, :max_ctx], dtype=np.float32).copy()
        bad = ~np.isfinite(x) | (np.abs(x) >= 1e30)
        x[bad] = -np.inf
        sel = topk_select(x, min(L, max_ctx), index_topk)
        out[r, :sel.size] = sel
    return out


# --------------------------------------------------------------------------- sparse MLA
def sparse_mla_decode(q: np.ndarray, kv_rows: np.ndarray, indices: np.ndarray,
                      sm_scale: float, d_v: int = D_NOPE):
    """Absorbed sparse MLA decode over packed fp8 rows (the contract of
    ``flash_mla.flash_mla_with_kvcache(..., is_fp8_kvcache=True, indices=...)``
    flash_mla.py:76-99).

    q float32 [T,H,576] (bf16 values); kv_rows uint8 [num_slots,656] addressed
    by physical slot; indices int [T,K], -1 = skip (mla_utils.py:267-271).
    Per (t,h): ``s_i = scale * q . kv(idx_i)`` over valid i, ``o = softmax(s) @
    kv(idx)[:, :512]`` (test_mla_decode_head_padding.py:30-33), and the natural
    log LSE ``log sum_i exp(s_i)`` (the convention of
    ``merge_attention_states`` mla_utils.py:19-21). Rows dequantise as
    fp8_utils.py:153-177. A query with no valid index gives o = 0, lse = -inf.
    Returns (o float32 [T,H,d_v], lse float32 [T,H]).
    """
    q = np.asarray(q, dtype=np.float64)
    T, H, D = q.shape
    o = np.zeros((T, H, d_v), dtype=np.float32)
    lse = np.full((T, H), -np.inf, dtype=np.float32)
    for t in range(T):
        idx = np.asarray(indices[t]).astype(np.int64)
        idx = idx[idx >= 0]
        if idx.size == 0:
            continue
        kv = dequant_mla_rows(kv_rows[idx]).astype(np.float64)   # [n, 576]
        s = (q[t] @ kv[:, :D].T) * sm_scale                      # [H, n]
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        den = p.sum(axis=1, keepdims=True)
        o[t] = ((p / den) @ kv[:, :d_v]).astype(np.float32)
        lse[t] = (m[:, 0] + np.log(den[:, 0])).astype(np.float32)
    return o, lse


def sparse_mla_prefill(q: np.ndarray, kv: np.ndarray, indices: np.ndarray, sm_scale: float,
                       d_v: int = D_NOPE):
    """Sparse MLA prefill over ragged bf16 rows (the contract of
    ``flash_mla_sparse_fwd(q, kv, indices, sm_scale, d_v)`` as called at
    deepseek_v2.py:1644-1650; FlashMLA is third-party and not vendored).

    q float [T,H,576] and kv float [s_kv,576] (bf16 values); indices int [T,K]
    into kv, entries < 0 or >= s_kv skipped. Per (t,h): ``s_i = scale * q .
    kv[idx_i]``, ``o = softmax(s) @ kv[idx, :512]``, ``max_logits = max_i s_i``,
    ``lse = log sum_i exp(s_i)`` (natural log, as the decode path). A query with
    no valid index gives o = 0, max_logits = lse = -inf. Float64 math.
    Returns (o float32 [T,H,d_v], max_logits float32 [T,H], lse float32 [T,H]).
    """
    q = np.asarray(q, dtype=np.float64)
    kv = np.asarray(kv, dtype=np.float64)
    T, H, D = q.shape
    o = np.zeros((T, H, d_v), dtype=np.float32)
    mx = np.full((T, H), -np.inf, dtype=np.float32)
    lse = np.full((T, H), -np.inf, dtype=np.float32)
    for t in range(T):
        idx = np.asarray(indices[t]).astype(np.int64)
        idx = idx[(idx >= 0) & (idx < kv.shape[0])]
        if idx.size == 0:
            continue
        rows = kv[idx]
        s = (q[t] @ rows[:, :D].T) * sm_scale
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        den = p.sum(axis=1, keepdims=True)
        o[t] = ((p / den) @ rows[:, :d_v]).astype(np.float32)
        mx[t] = m[:, 0].astype(np.float32)
        lse[t] = (m[:, 0] + np.log(den[:, 0])).astype(np.float32)
    return o, mx, lse


# --------------------------------------------------------------------------- indexer prologue
# The reference leaves the f32 summation order of its Hadamard and LayerNorm
# unspecified (a butterfly in indexer_q.cuh:164-193, tl.sum in
# indexer_transform.py:177-181, 223-232). The functions below fix one order and
# compute in IEEE f32 without fused multiply-adds, so a kernel using the same
# order matches them bit for bit; the tests pin them against float64 library
# routines (scipy's Hadamard matrix, complex multiplication, LayerNorm).
_INV_SQRT128 = np.float32(0.0883883461356163)     # f32 nearest to 128^-0.5


def rope_cos_sin_cache(max_pos: int, rotary_dim: int = 64, base: float = 10000.0) -> np.ndarray:
    """[max_pos, rotary_dim] f32 = [cos | sin] of t * inv_freq (rotary_embedding.py:33-40)."""
    inv_freq = (1.0 / (np.float32(base) ** (np.arange(0, rotary_dim, 2, dtype=np.float32) / rotary_dim)))
    freqs = np.arange(max_pos, dtype=np.float32)[:, None] * inv_freq.astype(np.float32)[None, :]
    return np.concatenate([np.cos(freqs), np.sin(freqs)], axis=-1).astype(np.float32)


def interleaved_to_half(x: np.ndarray) -> np.ndarray:
    """[..., 2m] interleaved (re, im) pairs -> [re 0..m-1 | im 0..m-1] (lightning.py:110-113)."""
    x = np.asarray(x)
    return np.swapaxes(x.reshape(*x.shape[:-1], -1, 2), -1, -2).reshape(x.shape)


def rope_neox(x_half: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """NeoX rotation in f32 (rotary_embedding.py:10-18): x = [x1 | x2],
    y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin. cos/sin broadcast over x1."""
    x = np.asarray(x_half, dtype=np.float32)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return np.concatenate([y1, y2], axis=-1).astype(np.float32)


def hadamard128(x: np.ndarray) -> np.ndarray:
    """128-point Walsh-Hadamard transform times 128^-0.5 in f32: stages h = 1, 2,
    ..., 64, each (a, b) -> (a + b, a - b) (indexer_q.cuh:164-198)."""
    y = np.array(x, dtype=np.float32, copy=True)
    n = y.shape[-1]
    assert n == 128
    h = 1
    while h < n:
        v = y.reshape(*y.shape[:-1], n // (2 * h), 2, h)
        a = v[..., 0, :].copy()
        b = v[..., 1, :].copy()
        v[..., 0, :] = a + b
        v[..., 1, :] = a - b
        h *= 2
    return (y * _INV_SQRT128).astype(np.float32)


def f32_tree_sum128(x: np.ndarray) -> np.ndarray:
    """Sum over the last axis (128) in f32: element e = 8j + i, in-j tree over i
    ((i, i+4), (i, i+2), (i, i+1)), then a butterfly over j (xor 1, 2, 4, 8)."""
    v = np.asarray(x, dtype=np.float32).reshape(*np.shape(x)[:-1], 16, 8)
    v = v[..., :4] + v[..., 4:]
    v = v[..., :2] + v[..., 2:]
    s = (v[..., 0] + v[..., 1]).astype(np.float32)           # [..., 16]
    j = np.arange(16)
    for m in (1, 2, 4, 8):
        s = (s + s[..., j ^ m]).astype(np.float32)
    return s[..., 0]


def _quant_ue8m0_f32(x: np.ndarray):
    amax = np.maximum(np.abs(x).max(axis=-1), np.float32(1e-4)).astype(np.float32)
    sf = ue8m0_ceil((amax / np.float32(FP8_MAX)).astype(np.float32))
    codes = fp8_e4m3fn_encode(x * (np.float32(1.0) / sf)[..., None])
    return codes, sf


def indexer_q_prologue(q_bf16: np.ndarray, gate_bf16: np.ndarray, weight_scale: float, cos_sin: np.ndarray,
                       positions: np.ndarray, rope_interleaved: bool = True):
    """Indexer query prologue (indexer_q.cuh:57-225 as instantiated at
    jit/sgl/deepseek_v4.py:153-165, 290-322; unfused steps lightning.py:720-755,
    1327-1337 and their composition in tests/test_indexer_transform.py:72-116).

    q_bf16 [T, H, 128] uint16, gate_bf16 [T, H] uint16, cos_sin [P, 64] f32,
    positions [T]. Returns (codes uint8 [T, H, 128], weights f32 [T, H])."""
    x = bf16_to_f32(q_bf16).astype(np.float32)
    rope = x[..., :64]
    if rope_interleaved:
        rope = interleaved_to_half(rope)
    cs = np.asarray(cos_sin, dtype=np.float32)[np.asarray(positions, dtype=np.int64)]   # [T, 64]
    rot = rope_neox(rope, cs[:, None, :32], cs[:, None, 32:])
    x = np.concatenate([bf16_to_f32(f32_to_bf16(rot)), x[..., 64:]], axis=-1)
    y = bf16_to_f32(f32_to_bf16(hadamard128(x)))
    codes, sf = _quant_ue8m0_f32(y)
    g = bf16_to_f32(gate_bf16).astype(np.float32)
    weights = (g * np.float32(weight_scale)).astype(np.float32) * sf
    return codes, weights.astype(np.float32)


def indexer_k_transform(key_bf16: np.ndarray, ln_w: np.ndarray, ln_b: np.ndarray, eps: float,
                        cos_sin: np.ndarray, positions: np.ndarray):
    """Indexer key transform (indexer_transform.py:156-260): LayerNorm (biased
    variance, 1/sqrt(var + eps)) rounded to bf16, RoPE on the interleaved
    leading 64 dims rounded to bf16, Hadamard kept in f32, UE8M0 quantisation.

    key_bf16 [T, 128] uint16. Returns (codes uint8 [T, 128], scales f32 [T])."""
    x = bf16_to_f32(key_bf16).astype(np.float32)
    mean = (f32_tree_sum128(x) * np.float32(1.0 / 128.0)).astype(np.float32)
    c = (x - mean[:, None]).astype(np.float32)
    var = (f32_tree_sum128(c * c) * np.float32(1.0 / 128.0)).astype(np.float32)
    inv_std = (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)
    y = ((c * inv_std[:, None]).astype(np.float32) * np.asarray(ln_w, dtype=np.float32)).astype(np.float32)
    y = bf16_to_f32(f32_to_bf16(y + np.asarray(ln_b, dtype=np.float32)))
    cs = np.asarray(cos_sin, dtype=np.float32)[np.asarray(positions, dtype=np.int64)]
    rot = rope_neox(interleaved_to_half(y[:, :64]), cs[:, :32], cs[:, 32:])
    y = np.concatenate([bf16_to_f32(f32_to_bf16(rot)), y[:, 64:]], axis=-1)
    return _quant_ue8m0_f32(hadamard128(y))


# --------------------------------------------------------------------------- prefill indexer
def gather_indexer_cache(cache: np.ndarray, block_table: np.ndarray, cu_seqlens_k: np.ndarray,
                         page_size: int = 64, head_dim: int = 128):
    """Paged split-layout cache -> contiguous ragged (keys uint8 [total_k, 128],
    scales f32 [total_k]) (kernel/triton/generic/indexer_cache_gather.py:8-114):
    ragged token cu[b] + t is token t of sequence b, read through block_table[b]."""
    cu = np.asarray(cu_seqlens_k, dtype=np.int64)
    total = int(cu[-1])
    keys = np.zeros((total, head_dim), dtype=np.uint8)
    scales = np.zeros(total, dtype=np.float32)
    for b in range(len(cu) - 1):
        for t in range(int(cu[b + 1] - cu[b])):
            page = int(block_table[b, t // page_size])
            off = t % page_size
            keys[cu[b] + t] = cache[page, off * head_dim:(off + 1) * head_dim]
            base = page_size * head_dim + off * 4
            scales[cu[b] + t] = cache[page, base:base + 4].copy().view(np.float32)[0]
    return keys, scales


def prefill_ks_ke(cu_seqlens_q: np.ndarray, cu_seqlens_k: np.ndarray):
    """Per-query ragged key window [ks, ke) of a chunked prefill
    (lightning.py:1187-1209): query t of sequence b sees its cached prefix and
    the fresh keys up to itself, ks = cu_k[b], ke = ks + (k_len - q_len) + local + 1."""
    cq = np.asarray(cu_seqlens_q, dtype=np.int64)
    ck = np.asarray(cu_seqlens_k, dtype=np.int64)
    ks, ke = [], []
    for b in range(len(cq) - 1):
        qn, kn = cq[b + 1] - cq[b], ck[b + 1] - ck[b]
        for t in range(qn):
            ks.append(ck[b])
            ke.append(ck[b] + (kn - qn) + t + 1)
    return np.asarray(ks, dtype=np.int32), np.asarray(ke, dtype=np.int32)


def mqa_logits(q_fp8: np.ndarray, kv_fp8: np.ndarray, kv_scale: np.ndarray, weights: np.ndarray,
               ks: np.ndarray, ke: np.ndarray, clean_logits: bool = True) -> np.ndarray:
    """Ragged fp8 MQA logits, the contract of ``deep_gemm.fp8_mqa_logits`` as
    called at lightning.py:1212-1219 (third-party DeepGEMM, not vendored; the
    score is lightning.py:116-131 ``_weighted_relu_mqa_scores`` times the key
    scale):

    ``logits[i, j] = sum_h w[i,h] * relu(q[i,h,:] . kv[j,:]) * kv_scale[j]`` for
    ``ks[i] <= j < ke[i]``, -inf elsewhere (``clean_logits``; otherwise the
    entries outside are left at 0 here, the reference leaves them unspecified).
    q_fp8 uint8 [M, H, 128], kv_fp8 uint8 [N, 128], kv_scale f32 [N],
    weights f32 [M, H]. float64 accumulation; returns f32 [M, N]."""
    M, H, D = q_fp8.shape
    N = kv_fp8.shape[0]
    out = np.full((M, N), -np.inf if clean_logits else 0.0, dtype=np.float32)
    qf = fp8_e4m3fn_decode(q_fp8).astype(np.float64)
    kf = fp8_e4m3fn_decode(kv_fp8).astype(np.float64)
    sc = np.asarray(kv_scale, dtype=np.float64)
    w = np.asarray(weights, dtype=np.float64)
    for i in range(M):
        a, e = int(ks[i]), int(ke[i])
        if e <= a:
            continue
        dots = qf[i] @ kf[a:e].T                                # [H, e-a]
        out[i, a:e] = ((np.maximum(dots, 0.0) * w[i][:, None]).sum(axis=0) * sc[a:e]).astype(np.float32)
    return out
