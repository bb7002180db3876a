"""Sampled-row parity check of a full DSA decode step (test infrastructure only).

TEST INFRASTRUCTURE ONLY. Used by ``tests/test_gpu_full_shape.py``, ``tests/test_gpu_config4.py`` and by the
``cpu_baseline`` leg of ``bench.py`` to check the outputs of a GPU step at its
own shape (B=128 x 64K) on a handful of rows spread over the
batch. Nothing in ``nanoengine_amd`` imports it.

The bounds are the north-star tolerances:

* indexer logits: |gpu - oracle| <= 1e-3 * max(|oracle|, row RMS) on t < ctx,
  or, for a logit whose head sum cancels, within the scaled fp8 MFMA's derived
  error bound (``indexer_logit_error_bound``);
* top-k: the GPU's logical set equals the oracle's exact selection
  (``topk_transform``, topk.cuh:249-287) over the GPU's own logits, bit for bit;
  against the oracle's float64 logits the sets may differ only at ties within
  1e-3 of the k-th score;
* physical slots: bit-exact ``topk_indices_to_physical`` (mla_utils.py:237-272);
* MLA o within atol 2e-2 and natural-log LSE within 1e-3 (absolute), both
  against ``sparse_mla_decode`` over the GPU's own physical indices.
"""
from __future__ import annotations

import numpy as np

from . import dsa_oracle as O

LOGITS_RTOL = 1e-3
O_ATOL = 2e-2
LSE_ATOL = 1e-3


def spread_rows(batch: int, count: int) -> np.ndarray:
    """``count`` distinct row ids spread evenly over ``[0, batch)``, first and
    last included (so both ends of any contiguous work split are sampled)."""
    count = min(count, batch)
    return np.unique(np.round(np.linspace(0, batch - 1, count)).astype(np.int64))


def localize_pages(block_tables: np.ndarray, lens: np.ndarray, page_size: int = 64):
    """The pages the rows use, renumbered densely: returns (used page ids,
    block tables over the dense numbering). Pages past a row's length map to 0."""
    bt = np.asarray(block_tables, dtype=np.int64)
    npages = (np.asarray(lens, dtype=np.int64) + page_size - 1) // page_size
    mask = np.arange(bt.shape[1])[None, :] < npages[:, None]
    used = np.unique(bt[mask])
    local = np.zeros_like(bt)
    local[mask] = np.searchsorted(used, bt[mask])
    return used, local.astype(np.int32)


def check_logits(gpu: np.ndarray, exp: np.ndarray, ctx: np.ndarray, bound=None) -> dict:
    """Logits against the oracle over the valid prefix of every row.

    A logit passes when |gpu - oracle| <= 1e-3 * max(|oracle|, row RMS) (the
    north-star tolerance) or, where a head sum cancels and the relative
    tolerance has no scale, when the error is within the scaled fp8 MFMA's
    derived error bound ``bound(r, positions)`` (``indexer_logit_error_bound``
    in the oracle: each dot's truncation remainders at 2^-13 of its largest
    product, plus f32 rounding). Returns {max_rel_err, over_rtol,
    max_err_over_bound, ok}: ``max_rel_err`` over every logit, ``over_rtol``
    the logits beyond 1e-3, ``max_err_over_bound`` the largest error / bound
    among those (ok needs it <= 1; None when no logit needed the bound)."""
    worst, over, worst_b = 0.0, 0, None
    for r in range(exp.shape[0]):
        L = int(ctx[r])
        if L <= 0:
            continue
        g, e = gpu[r, :L].astype(np.float64), exp[r, :L].astype(np.float64)
        rms = np.sqrt(np.mean(e * e)) + 1e-30
        rel = np.abs(g - e) / np.maximum(np.abs(e), rms)
        worst = max(worst, float(rel.max()))
        bad = np.nonzero(~(rel <= LOGITS_RTOL))[0]
        if bad.size == 0:
            continue
        over += int(bad.size)
        if bound is None:
            worst_b = float("inf")
            continue
        b = bound(r, bad)
        ratio = np.where(np.isfinite(g[bad]), np.abs(g[bad] - e[bad]) / np.maximum(b, 1e-300), np.inf)
        worst_b = max(worst_b or 0.0, float(ratio.max()))
    return {"max_rel_err": worst, "over_rtol": over, "max_err_over_bound": worst_b,
            "ok": worst_b is None or worst_b <= 1.0}


def paged_logit_bound(q_idx, weights, idx_pages, bt_local, page_size: int = 64):
    """``bound(r, positions)`` for :func:`check_logits` over paged indexer
    keys: q_idx uint8 [S,1,H,128], weights [S,H], idx_pages [P, page*132],
    bt_local [S,M] (the rows' dense page numbering)."""
    D = q_idx.shape[-1]

    def bound(r, pos):
        pos = np.asarray(pos, dtype=np.int64)
        pages = np.asarray(bt_local[r], dtype=np.int64)[pos // page_size]
        off = pos % page_size
        codes = np.stack([idx_pages[p, o * D:(o + 1) * D] for p, o in zip(pages, off)])
        sc = np.array([idx_pages[p, page_size * D + 4 * o:page_size * D + 4 * o + 4].copy().view(np.float32)[0]
                       for p, o in zip(pages, off)], dtype=np.float32)
        return O.indexer_logit_error_bound(q_idx[r, 0], weights[r], codes, sc)
    return bound


def ragged_logit_bound(q_codes, weights, keys, key_scales):
    """``bound(r, positions)`` for :func:`check_logits` over ragged keys:
    q_codes uint8 [S,H,128], weights [S,H], keys uint8 [N,128], key_scales f32 [N]."""
    def bound(r, pos):
        pos = np.asarray(pos, dtype=np.int64)
        return O.indexer_logit_error_bound(q_codes[r], weights[r], keys[pos], key_scales[pos])
    return bound


def topk_tie_violations(logical: np.ndarray, exp_logits: np.ndarray, ctx: np.ndarray, k: int) -> int:
    """Positions in the symmetric difference between the GPU's selection and
    the exact selection over the oracle's logits whose oracle score is further
    than 1e-3 (relative to max(|k-th score|, row RMS)) from the k-th score."""
    bad = 0
    for r in range(logical.shape[0]):
        L = int(ctx[r])
        mine = set(int(x) for x in logical[r] if x >= 0)
        sel = O.topk_select(exp_logits[r], L, k)
        diff = mine.symmetric_difference(int(x) for x in sel)
        if not diff:
            continue
        row = exp_logits[r, :L].astype(np.float64)
        kth = np.sort(row)[::-1][min(k, L) - 1]
        tol = LOGITS_RTOL * max(abs(kth), float(np.sqrt(np.mean(row * row))))
        bad += sum(1 for p in diff if not (p < L and abs(row[p] - kth) <= tol))
    return bad


def check_step_rows(*, q_idx, idx_pages, weights, ctx, bt_local, bt_global, max_ctx,
                    gpu_logits, gpu_logical, gpu_physical, q_mla, kv_sel, gpu_o, gpu_lse,
                    sm_scale, topk, page_size=64, exp_logits=None) -> dict:
    """Checks S sampled rows of one decode step (next_n = 1).

    q_idx uint8 [S,1,64,128]; idx_pages uint8 [P, page*132] (the rows' pages,
    densely renumbered); weights f32 [S,64]; ctx int [S]; bt_local int [S,M]
    over the dense pages; bt_global int [S,M] (the real block tables, for the
    physical check); gpu_logits f32 [S,max_ctx] (the standalone logits
    operator); gpu_logical / gpu_physical int32 [S,topk]; q_mla f32 [S,H,576];
    kv_sel uint8 [S,topk,656] (the cache rows at gpu_physical, any bytes where
    it is -1); gpu_o f32 [S,H,512]; gpu_lse f32 [S,H]. ``exp_logits`` may pass
    oracle logits computed already. Returns a report dict whose ``ok`` is True
    when every bound holds."""
    ctx = np.asarray(ctx).reshape(-1)
    S = ctx.shape[0]
    if exp_logits is None:
        exp_logits = O.indexer_logits(q_idx, idx_pages, weights, ctx.reshape(S, 1), bt_local, max_ctx, page_size)
    rep = {"rows": S}
    lg = check_logits(gpu_logits, exp_logits, ctx, paged_logit_bound(q_idx, weights, idx_pages, bt_local, page_size))
    rep["logits_max_rel_err"] = lg["max_rel_err"]
    rep["logits_over_rtol"] = lg["over_rtol"]
    rep["logits_max_err_over_mfma_bound"] = lg["max_err_over_bound"]
    _, raw = O.topk_transform(gpu_logits, ctx, bt_global, page_size, topk)
    rep["topk_equal_on_gpu_logits"] = bool(np.array_equal(raw, gpu_logical))
    rep["topk_tie_violations"] = topk_tie_violations(gpu_logical, exp_logits, ctx, topk)
    phys = O.topk_indices_to_physical(gpu_logical, bt_global, page_size)
    rep["physical_equal"] = bool(np.array_equal(phys, gpu_physical))
    o_err, lse_err, lse_inf_ok = 0.0, 0.0, True
    for r in range(S):
        idx = np.where(gpu_physical[r] >= 0, np.arange(topk), -1)[None, :]
        eo, el = O.sparse_mla_decode(q_mla[r:r + 1], kv_sel[r], idx, sm_scale)
        o_err = max(o_err, float(np.abs(gpu_o[r] - eo[0]).max()))
        fin = np.isfinite(el[0])
        lse_inf_ok &= bool(np.array_equal(np.isfinite(gpu_lse[r]), fin))
        if fin.any():
            lse_err = max(lse_err, float(np.abs(gpu_lse[r][fin] - el[0][fin]).max()))
    rep["o_max_abs_err"] = o_err
    rep["lse_max_abs_err"] = lse_err
    rep["ok"] = bool(lg["ok"] and rep["topk_equal_on_gpu_logits"]
                     and rep["topk_tie_violations"] == 0 and rep["physical_equal"]
                     and o_err <= O_ATOL and lse_err <= LSE_ATOL and lse_inf_ok)
    return rep


def sample_from_device(rows, *, q_idx_fp8, weights, cache, lens, block_tables, q_mla, kv, logits,
                       logical, physical, o, lse, page_size=64, next_n=1) -> dict:
    """Copies what :func:`check_step_rows` needs for ``rows`` from the GPU
    step's tensors (torch, on the device) to host numpy: the rows' indexer
    pages (densely renumbered), their query, weights and tables, the GPU's
    logits, indices and outputs, and the MLA cache rows at the GPU's physical
    indices. ``kv`` is the [blocks, 64, 1, 656] cache view. Rows are query
    tokens: with ``next_n`` > 1 row r is draft position r % next_n of sequence
    r // next_n, and ``lens`` holds each query token's own causal length."""
    import torch

    dev = q_idx_fp8.device
    rt = torch.as_tensor(np.asarray(rows), dtype=torch.long, device=dev)
    ctx = np.asarray([int(lens[int(r)]) for r in rows], dtype=np.int32)
    bt_global = block_tables.index_select(0, rt // next_n).cpu().numpy()
    used, bt_local = localize_pages(bt_global, ctx, page_size)
    pages = cache.index_select(0, torch.as_tensor(used, dtype=torch.long, device=dev)).cpu().numpy()
    phys = physical.index_select(0, rt)
    safe = phys.clamp_min(0).long()
    kv_sel = kv[safe // page_size, safe % page_size, 0].cpu().numpy()
    return dict(q_idx=q_idx_fp8.index_select(0, rt).cpu().numpy().reshape(len(rows), 1, 64, 128),
                idx_pages=pages, weights=weights.index_select(0, rt).cpu().numpy(), ctx=ctx,
                bt_local=bt_local, bt_global=bt_global, max_ctx=block_tables.shape[1] * page_size,
                gpu_logits=logits.index_select(0, rt).cpu().numpy(),
                gpu_logical=logical.index_select(0, rt).cpu().numpy(), gpu_physical=phys.cpu().numpy(),
                q_mla=q_mla.index_select(0, rt).float().cpu().numpy(), kv_sel=kv_sel,
                gpu_o=o.index_select(0, rt).float().cpu().numpy(),
                gpu_lse=lse.index_select(0, rt).cpu().numpy())
