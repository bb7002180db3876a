"""Fused ragged fp8 MQA logits + exact top-2048 (``ops.mqa_topk``,
``dsa_mqa_topk``) on the GPU.

The fused entry must return exactly what the two-step path returns:
``ops.mqa_logits`` into a buffer, then ``ops.topk_transform_ragged`` with
row_starts = offsets = ks (lightning.py:1212-1246). That path is itself
checked against the oracle (test_gpu_prefill.py, test_gpu_topk.py); here the
comparison is bit for bit, on:
  * random fp8 scores over ragged windows of every kind (empty, shorter than
    2048, exactly 2048, long, clamped by max_len);
  * inputs that defeat the sampled threshold, so every row goes through the
    host-ordered fix-up: hot keys on the sampled positions (the list comes up
    short) and all-equal scores (the list overflows), with more deferred rows
    than one fix-up chunk holds;
  * NaN keys and overflowing scores;
  * a small case against the oracle's logits and ragged top-k directly.
"""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import ops

pytestmark = pytest.mark.gpu


def _inputs(dev, m, n, seed, key_scale=None, weights=None):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(m, 64, 128, device=dev, generator=g) * 8).to(torch.float8_e4m3fn)
    kv = (torch.randn(n, 128, device=dev, generator=g) * 8).to(torch.float8_e4m3fn)
    sc = key_scale if key_scale is not None else \
        torch.exp2(torch.randint(-9, -5, (n,), device=dev, generator=g).float())
    w = weights if weights is not None else torch.randn(m, 64, device=dev, generator=g) * 0.01
    return q, kv, sc.contiguous(), w.contiguous()


def _two_step(q, kv, sc, w, ks, ke, max_len):
    m, n = q.shape[0], kv.shape[0]
    logits = torch.empty(m, n, dtype=torch.float32, device=q.device)
    ops.mqa_logits(q, kv, sc, w, ks, ke, logits, clean_logits=False)
    lens = (ke - ks).clamp(0, max_len).to(torch.int32).contiguous()
    out = torch.empty(m, 2048, dtype=torch.int32, device=q.device)
    ops.topk_transform_ragged(logits, lens, ks, ks, out, 2048)
    return out


def _fused(q, kv, sc, w, ks, ke, max_len):
    out = torch.full((q.shape[0], 2048), -7, dtype=torch.int32, device=q.device)
    ops.mqa_topk(q, kv, sc, w, ks, ke, max_len, out)
    return out


def _windows(dev, lens, n, seed):
    rng = np.random.default_rng(seed)
    ks = np.array([rng.integers(0, n - L + 1) for L in lens], dtype=np.int32)
    ke = ks + np.asarray(lens, dtype=np.int32)
    t = lambda a: torch.from_numpy(a).to(dev).contiguous()   # noqa: E731
    return t(ks), t(ke)


def test_fused_matches_two_step_random(cuda):
    print("mqa_topk random windows", flush=True)
    n = 40000
    lens = [0, 1, 100, 2047, 2048, 2049, 3000, 6000, 6200, 9000, 20000, 39999, 40000] * 3
    q, kv, sc, w = _inputs(cuda, len(lens), n, 1)
    ks, ke = _windows(cuda, lens, n, 2)
    for max_len in (n, 30000):
        exp = _two_step(q, kv, sc, w, ks, ke, max_len)
        got = _fused(q, kv, sc, w, ks, ke, max_len)
        torch.cuda.synchronize()
        assert torch.equal(got, exp), f"max_len {max_len}: rows differ " \
            f"{torch.nonzero((got != exp).any(1)).flatten().tolist()}"


def test_fused_matches_two_step_config4_rows(cuda):
    """Causal rows of one long sequence, as in a chunked prefill over a
    cached prefix (windows [0, prefix + i + 1))."""
    print("mqa_topk causal rows", flush=True)
    n, m = 70000, 96
    q, kv, sc, w = _inputs(cuda, m, n, 3)
    ke = torch.arange(n - m + 1, n + 1, dtype=torch.int32, device=cuda)
    ks = torch.zeros(m, dtype=torch.int32, device=cuda)
    exp = _two_step(q, kv, sc, w, ks, ke, n)
    got = _fused(q, kv, sc, w, ks, ke, n)
    torch.cuda.synchronize()
    assert torch.equal(got, exp)


def test_fix_up_hot_sampled_keys(cuda):
    """Keys 64j score far above the rest: the threshold from the sample sits
    among them, the list holds ~64 candidates < 2048, and every long row is
    redone through the fix-up."""
    print("mqa_topk fix-up (short lists)", flush=True)
    n = 50000
    lens = [40000, 45000, 2048, 3000, 50000, 10]
    sc = torch.full((n,), 2.0 ** -8, device=cuda)
    sc[::64] = 2.0 ** 6
    q, kv, _, w = _inputs(cuda, len(lens), n, 4, key_scale=sc)
    w = w.abs()  # positive weights: a hot key's score stays high
    ks, ke = _windows(cuda, lens, n, 5)
    exp = _two_step(q, kv, sc, w, ks, ke, n)
    got = _fused(q, kv, sc, w, ks, ke, n)
    torch.cuda.synchronize()
    assert torch.equal(got, exp)


def test_fix_up_ties_over_several_chunks(cuda):
    """Zero weights: every score is 0, every key ties with the threshold and
    each long list overflows. 2^20 keys make one fix-up chunk 64 rows, so the
    80 deferred rows take two chunks; ties resolve to the lowest positions."""
    print("mqa_topk fix-up (ties, two chunks)", flush=True)
    n = 1 << 20
    lens = [200000 + 37 * i for i in range(80)] + [5, 2048]
    m = len(lens)
    q, kv, sc, _ = _inputs(cuda, m, n, 6)
    w = torch.zeros(m, 64, device=cuda)
    ks, ke = _windows(cuda, lens, n, 7)
    got = _fused(q, kv, sc, w, ks, ke, 1 << 18)
    torch.cuda.synchronize()
    ks_h = ks.cpu()
    for r, L in enumerate(lens):
        k = min(L, 2048)
        exp = torch.full((2048,), -1, dtype=torch.int32)
        exp[:k] = torch.arange(k, dtype=torch.int32) + ks_h[r]
        assert torch.equal(got[r].cpu(), exp), f"row {r}"


def test_fused_against_oracle_small(cuda):
    print("mqa_topk vs oracle", flush=True)
    rng = np.random.default_rng(9)
    n, lens = 6000, [0, 700, 2048, 2500, 5999, 6000]
    m = len(lens)
    q = O.fp8_e4m3fn_encode(rng.standard_normal((m, 64, 128)) * 8)
    kv = O.fp8_e4m3fn_encode(rng.standard_normal((n, 128)) * 8)
    sc = O.ue8m0_ceil(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
    w = (rng.standard_normal((m, 64)) * 0.01).astype(np.float32)
    ks = np.array([rng.integers(0, n - L + 1) for L in lens], dtype=np.int32)
    ke = ks + np.asarray(lens, dtype=np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)   # noqa: E731
    got = _fused(t(q).view(torch.float8_e4m3fn), t(kv).view(torch.float8_e4m3fn), t(sc), t(w), t(ks), t(ke),
                 n).cpu().numpy()
    # the GPU's logits are within 1e-4 relative of the oracle's; compare the
    # selections on the oracle's own logits away from near-ties
    logits = O.mqa_logits(q, kv, sc, w, ks, ke, clean_logits=True)
    for r in range(m):
        row = logits[r, ks[r]:ke[r]].astype(np.float64)
        k = min(2048, len(row))
        sel = got[r][got[r] >= 0] - ks[r]
        assert len(sel) == k and len(set(sel.tolist())) == k and np.all(got[r][k:] == -1)
        if k < 2048:
            assert set(sel.tolist()) == set(range(len(row)))
            continue
        kth = np.sort(row)[::-1][k - 1]
        tol = 1e-4 * max(abs(kth), np.sqrt(np.mean(row * row)))
        assert set(np.nonzero(row > kth + tol)[0].tolist()) <= set(sel.tolist())
        assert set(sel.tolist()) <= set(np.nonzero(row >= kth - tol)[0].tolist())


def test_workspace_too_small_is_rejected(cuda):
    q, kv, sc, w = _inputs(cuda, 2, 5000, 8)
    ks = torch.zeros(2, dtype=torch.int32, device=cuda)
    ke = torch.full((2,), 5000, dtype=torch.int32, device=cuda)
    out = torch.empty(2, 2048, dtype=torch.int32, device=cuda)
    need = ops.mqa_topk_workspace_bytes(2, 5000)
    ws = torch.empty(need - 256, dtype=torch.uint8, device=cuda)
    with pytest.raises(RuntimeError, match="workspace"):
        ops.mqa_topk(q, kv, sc, w, ks, ke, 5000, out, workspace=ws)


def test_nan_and_overflowing_scores_match_two_step(cuda):
    """fp8 NaN codes in some keys (NaN logits rank lowest) and weights large
    enough that some logits overflow to +-inf: the fused entry still returns
    the two-step path's indices."""
    print("mqa_topk NaN / inf scores", flush=True)
    n = 20000
    lens = [15000, 9000, 3000, 20000]
    q, kv, sc, w = _inputs(cuda, len(lens), n, 10)
    raw = kv.view(torch.uint8).clone()
    g = torch.Generator(device=cuda).manual_seed(11)
    nan_keys = torch.randint(0, n, (500,), device=cuda, generator=g)
    raw[nan_keys, 5] = 0x7f                     # e4m3fn NaN
    kv = raw.view(torch.float8_e4m3fn)
    w = w.clone()
    w[1] *= 1e36                                # row 1: many logits overflow to +-inf
    ks, ke = _windows(cuda, lens, n, 12)
    exp = _two_step(q, kv, sc, w, ks, ke, n)
    got = _fused(q, kv, sc, w, ks, ke, n)
    torch.cuda.synchronize()
    assert torch.equal(got, exp)
