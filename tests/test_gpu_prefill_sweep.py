"""Randomised shapes through the paged sparse MLA prefill (cached keys read
from the fp8 cache, fresh keys as bf16 rows, one softmax), sampled tokens
against the CPU oracle over the oracle's own assembled keys.

Each case draws, from its own seed: 1-4 sequences with 0-3000 cached tokens
(page edges included) and 1-70 fresh tokens, 16-128 heads, top-k of 64 to
2048 (so that windows are shorter than, equal to or longer than k), causal
random selections with -1 entries and indices past the key count mixed in."""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import ops, synth

pytestmark = pytest.mark.gpu

CACHED = [0, 1, 63, 64, 65, 2047, 2048]


@pytest.mark.parametrize("case", range(12))
def test_random_paged_prefill_matches_oracle(cuda, case):
    rng = np.random.default_rng(500 + case)
    S = int(rng.integers(1, 5))
    H = int(rng.choice([16, 32, 64, 96, 128]))
    topk = int(rng.choice([64, 128, 512, 2048]))
    cached = np.array([int(rng.choice(CACHED)) if rng.random() < 0.5 else int(rng.integers(0, 3000))
                       for _ in range(S)])
    q_lens = rng.integers(1, 71, S)
    k_lens = q_lens + cached
    print(f"prefill sweep case {case}: S={S} H={H} topk={topk} cached={cached.tolist()} "
          f"q_lens={q_lens.tolist()}", flush=True)
    pages = (k_lens + 63) // 64
    num_blocks = int(pages.sum()) + 3
    perm = rng.permutation(num_blocks)
    bt = np.zeros((S, pages.max()), np.int32)
    at = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[at:at + p]
        at += p
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    T, total_k = int(cu_q[-1]), int(cu_k[-1])
    idx = np.full((T, topk), -1, np.int32)
    for b in range(S):
        for j in range(q_lens[b]):
            t = cu_q[b] + j
            win = cached[b] + j + 1
            n = min(topk, win)
            sel = rng.choice(win, size=n, replace=False) + cu_k[b]
            drop = rng.random(n) < 0.1
            sel[drop] = -1
            past = rng.random(n) < 0.02
            sel[past] = total_k + 7
            idx[t, :n] = sel
    kv = synth.make_mla_cache(num_blocks, seed=case, device=cuda)
    g = torch.Generator(device=cuda).manual_seed(case)
    fresh = torch.randn(T, 576, device=cuda, generator=g).to(torch.bfloat16)
    q = synth.make_mla_query(T, H, seed=case, device=cuda)
    t32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda, torch.int32)   # noqa: E731
    scale = 192 ** -0.5
    o, mx, lse = ops.sparse_mla_prefill_paged(q, kv, t32(bt), t32(cu_q), t32(cu_k), fresh, t32(idx), scale,
                                              total_k)
    torch.cuda.synchronize()
    rows = kv.contiguous().reshape(-1, 656).cpu().numpy()
    kv_or = O.assemble_prefill_kv(rows, 64, bt, cu_q, cu_k, fresh.float().cpu().numpy())
    # every sequence's first and last token, then random ones, at most 16
    sample = sorted(set([int(cu_q[b]) for b in range(S)] + [int(cu_q[b + 1]) - 1 for b in range(S)]
                        + rng.integers(0, T, 8).tolist()))[:16]
    oo, omx, olse = O.sparse_mla_prefill(q[sample].float().cpu().numpy(), kv_or, idx[sample], scale)
    err = np.abs(o[sample].float().cpu().numpy() - oo)
    print(f"max |o err| {err.max():.4f}", flush=True)
    assert np.all(np.isfinite(o[sample].float().cpu().numpy()))
    assert err.max() <= 2e-2
    ofin = np.isfinite(olse)
    assert np.array_equal(np.isfinite(lse[sample].cpu().numpy()), ofin)
    if ofin.any():
        assert np.abs(lse[sample].cpu().numpy()[ofin] - olse[ofin]).max() <= 1e-3
        assert np.abs(mx[sample].cpu().numpy()[ofin] - omx[ofin]).max() <= 1e-3
