"""Prefill indexer on the GPU vs the oracle: ragged fp8 MQA logits (windows,
clean/unclean), the paged-to-ragged gather, and the prefill top-k driver.

Logit tolerance: |gpu - oracle| <= 1e-3 * max(|oracle|, row RMS) per element
(the indexer bound of the decode tests; fp8 products are exact in fp32, only
the accumulation order differs).
"""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import deep_gemm, ops

pytestmark = pytest.mark.gpu


def _inputs(rng, M, N, H=64):
    q = O.fp8_e4m3fn_encode(rng.standard_normal((M, H, 128)) * 40)
    kv = O.fp8_e4m3fn_encode(rng.standard_normal((N, 128)) * 40)
    sc = O.ue8m0_ceil(rng.uniform(1e-3, 1e-2, N).astype(np.float32))
    w = (rng.standard_normal((M, H)) * 64 ** -0.5 * 128 ** -0.5 * 1e-2).astype(np.float32)
    return q, kv, sc, w


def _run(cuda, q, kv, sc, w, ks, ke, clean, fill=None, ncols=None):
    M = q.shape[0]
    ncols = kv.shape[0] if ncols is None else ncols
    out = torch.full((M, ncols), float("nan") if fill is None else fill, dtype=torch.float32, device=cuda)
    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(cuda) if dt is None else \
        torch.from_numpy(np.ascontiguousarray(a)).to(dt).to(cuda)
    ops.mqa_logits(t(q).view(torch.float8_e4m3fn), t(kv).view(torch.float8_e4m3fn), t(sc), t(w),
                   t(ks, torch.int32), t(ke, torch.int32), out, clean)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check_windows(got, exp, ks, ke):
    for r in range(exp.shape[0]):
        a, e = int(ks[r]), int(ke[r])
        if e <= a:
            continue
        g, x = got[r, a:e].astype(np.float64), exp[r, a:e].astype(np.float64)
        rms = np.sqrt(np.mean(x * x)) + 1e-30
        err = np.abs(g - x) / np.maximum(np.abs(x), rms)
        assert err.max() <= 1e-3, (r, err.max())


@pytest.mark.parametrize("clean", [True, False])
def test_mqa_logits_multi_sequence_causal(cuda, clean):
    print(f"mqa_logits multi-seq clean={clean}", flush=True)
    rng = np.random.default_rng(1)
    cu_q, cu_k = np.array([0, 37, 100]), np.array([0, 700, 1500])
    ks, ke = O.prefill_ks_ke(cu_q, cu_k)
    q, kv, sc, w = _inputs(rng, 100, 1500)
    got = _run(cuda, q, kv, sc, w, ks, ke, clean)
    exp = O.mqa_logits(q, kv, sc, w, ks, ke, clean_logits=True)
    _check_windows(got, exp, ks, ke)
    cols = np.arange(1500)[None, :]
    outside = (cols < ks[:, None]) | (cols >= ke[:, None])
    if clean:
        assert np.all(np.isneginf(got[outside]))
    else:
        assert np.all(np.isnan(got[outside]))   # never written


def test_mqa_logits_ragged_edges(cuda):
    """Rows not a multiple of 16, keys not a multiple of 64, unaligned and empty windows."""
    rng = np.random.default_rng(2)
    M, N = 23, 1000
    q, kv, sc, w = _inputs(rng, M, N)
    ks = rng.integers(0, N, M).astype(np.int32)
    ke = np.minimum(ks + rng.integers(0, 400, M), N).astype(np.int32)
    ks[3], ke[3] = 999, 1000     # last key only
    ks[5], ke[5] = 10, 10        # empty
    ks[7], ke[7] = 0, N          # everything
    got = _run(cuda, q, kv, sc, w, ks, ke, True)
    exp = O.mqa_logits(q, kv, sc, w, ks, ke, clean_logits=True)
    _check_windows(got, exp, ks, ke)
    assert np.array_equal(np.isneginf(got), np.isneginf(exp))


def test_mqa_logits_long_single_sequence(cuda):
    """One sequence: a 256-token chunk over a 19.7K-key cached prefix (the
    config-4 shape, scaled down for the oracle)."""
    rng = np.random.default_rng(3)
    M, N = 256, 20000
    ks, ke = O.prefill_ks_ke(np.array([0, M]), np.array([0, N]))
    q, kv, sc, w = _inputs(rng, M, N)
    got = _run(cuda, q, kv, sc, w, ks, ke, False)
    exp = O.mqa_logits(q, kv, sc, w, ks, ke, clean_logits=True)
    _check_windows(got, exp, ks, ke)


def test_fp8_mqa_logits_entry_point(cuda):
    rng = np.random.default_rng(4)
    M, N = 40, 300
    q, kv, sc, w = _inputs(rng, M, N)
    ks, ke = O.prefill_ks_ke(np.array([0, M]), np.array([0, N]))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    got = deep_gemm.fp8_mqa_logits(t(q).view(torch.float8_e4m3fn), (t(kv).view(torch.float8_e4m3fn), t(sc)),
                                   t(w), t(ks), t(ke), clean_logits=True)
    exp = O.mqa_logits(q, kv, sc, w, ks, ke, clean_logits=True)
    got = got.cpu().numpy()
    _check_windows(got, exp, ks, ke)
    assert np.array_equal(np.isneginf(got), np.isneginf(exp))


def test_mqa_logits_within_the_derived_mfma_bound(cuda):
    """Queries whose head sums cancel over 48 wide-range fp8 keys (see
    test_gpu_indexer.py's cancelling rows) through the ragged prefill logits
    kernel (32x32x64 scaled fp8 MFMA): every logit within 1e-3 relative or
    within the derived MFMA bound (oracle ``indexer_logit_error_bound``)."""
    from oracle import step_check as SC
    from test_gpu_indexer import _wide_cancelling
    rng = np.random.default_rng(11)
    N, M, H = 48, 3, 64
    qs, ws = [], []
    k = None
    for _ in range(M):
        q, k_, w = _wide_cancelling(np.random.default_rng(rng.integers(1 << 30)), N, H)
        k = k_ if k is None else k
        # the keys are shared: re-project this query's weights on the first keys
        d = O.fp8_e4m3fn_decode(k).astype(np.float64) @ O.fp8_e4m3fn_decode(q).astype(np.float64).T
        R = np.maximum(d, 0.0)
        w = (w - np.linalg.pinv(R) @ (R @ w)).astype(np.float32)
        qs.append(q)
        ws.append(w)
    q, w = np.stack(qs), np.stack(ws)
    sc = np.full(N, 2.0 ** -6, np.float32)
    ks, ke = np.zeros(M, np.int32), np.full(M, N, np.int32)
    got = _run(cuda, q, k, sc, w, ks, ke, True)
    exp = O.mqa_logits(q, k, sc, w, ks, ke, clean_logits=True)
    rep = SC.check_logits(got, exp, ke, SC.ragged_logit_bound(q, w, k, sc))
    print(rep, flush=True)
    assert rep["over_rtol"] > 0, rep
    assert rep["ok"], rep
