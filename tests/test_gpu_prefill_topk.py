"""Prefill indexer selection on the GPU: the paged-to-ragged gather and the
chunked prefill top-k driver (lightning.py:1081-1250).

The gather is bit-exact (a byte copy). The driver is checked three ways, after
the reference's tests/test_indexer_prefill.py:
  * its orchestration (causal ragged windows, chunking, the topk path for
    top_k != 2048) with the logits replaced by a known function of the column;
  * the fused ragged top-2048 on long rows against torch.topk of the same
    logits (the reference tolerates 5 differences; this select is exact);
  * end to end on real fp8 pages against the oracle's gather and logits.
"""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import indexer as indexer_module
from nanoengine_amd import ops
from nanoengine_amd.indexer_cache_gather import gather_indexer_cache

pytestmark = pytest.mark.gpu


def test_gather_fragmented_partial_pages(cuda):
    """Two sequences of 70 and 65 tokens over fragmented pages (the case of
    tests/test_indexer_prefill.py:170-225): keys and scales land in ragged order."""
    print("gather fragmented pages", flush=True)
    page_size, head_dim, num_pages = 64, 128, 6
    cache = torch.empty(num_pages, page_size * (head_dim + 4), dtype=torch.uint8, device=cuda)
    for page in range(num_pages):
        cache[page, :page_size * head_dim] = ((torch.arange(page_size * head_dim, device=cuda) + page * 17)
                                              .remainder(251).to(torch.uint8))
        scales = torch.arange(page_size, dtype=torch.float32, device=cuda) + page * 100 + 0.25
        cache[page, page_size * head_dim:] = scales.view(torch.uint8)
    block_table = torch.tensor([[3, 1, 5], [4, 0, 2]], dtype=torch.int32, device=cuda)
    cu_k = torch.tensor([0, 70, 135], dtype=torch.int32, device=cuda)
    keys, scales = gather_indexer_cache(cache, block_table, cu_k, page_size=page_size, head_dim=head_dim,
                                        total_k=135, max_seqlen_k=70)
    torch.cuda.synchronize()

    def page_keys(p):
        return cache[p, :page_size * head_dim].view(page_size, head_dim)

    def page_scales(p):
        return cache[p, page_size * head_dim:].view(torch.float32)

    exp_keys = torch.cat([page_keys(3), page_keys(1)[:6], page_keys(4), page_keys(0)[:1]])
    exp_scales = torch.cat([page_scales(3), page_scales(1)[:6], page_scales(4), page_scales(0)[:1]])
    assert torch.equal(keys, exp_keys)
    assert torch.equal(scales.view(torch.float32).reshape(-1), exp_scales)
    # int64 cu_seqlens and the oracle's gather agree
    keys64, scales64 = gather_indexer_cache(cache, block_table, cu_k.long(), page_size=page_size,
                                            head_dim=head_dim)
    ok, os_ = O.gather_indexer_cache(cache.cpu().numpy(), block_table.cpu().numpy(), cu_k.cpu().numpy())
    assert np.array_equal(keys64.cpu().numpy(), ok)
    assert np.array_equal(scales64.view(torch.float32).reshape(-1).cpu().numpy(), os_)


def test_driver_multi_seq_causal_ranges_and_chunks(cuda, monkeypatch):
    """Windows [ks, ke) per query, chunks of query_chunk rows, top_k = 3 through
    torch.topk (descending): the case of tests/test_indexer_prefill.py:241-337."""
    print("prefill driver ranges", flush=True)
    gather_calls, seen = [], []
    real_gather = indexer_module.gather_indexer_cache

    def spy_gather(cache, page_table, cu_k, **kw):
        gather_calls.append((cu_k.clone(), kw))
        return real_gather(cache, page_table, cu_k, **kw)

    def fake_logits(q, keys, key_scales, weights, ks, ke, out, clean):
        assert clean is True
        seen.append((ks.tolist(), ke.tolist()))
        total_k = keys.shape[0]
        out.copy_(torch.arange(total_k, dtype=torch.float32, device=cuda).expand(q.shape[0], -1))
        cols = torch.arange(total_k, device=cuda).unsqueeze(0)
        out.masked_fill_((cols < ks[:, None]) | (cols >= ke[:, None]), -torch.inf)

    monkeypatch.setattr(indexer_module, "gather_indexer_cache", spy_gather)
    monkeypatch.setattr(indexer_module, "_score_chunk", fake_logits)
    cache = torch.zeros(6, 4 * 132, dtype=torch.uint8, device=cuda)
    q = torch.zeros(5, 64, 128, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    w = torch.ones(5, 64, dtype=torch.float32, device=cuda)
    cu_q = torch.tensor([0, 2, 5], dtype=torch.int32, device=cuda)
    cu_k = torch.tensor([0, 5, 10], dtype=torch.int32, device=cuda)
    bt = torch.tensor([[3, 1], [4, 0]], dtype=torch.int32, device=cuda)
    got = indexer_module.compute_prefill_topk_paged(q, w, cu_q, cu_k, bt, cache, page_size=4, index_topk=3,
                                                    query_chunk=2)
    expected = torch.tensor([[3, 2, 1], [4, 3, 2], [7, 6, 5], [8, 7, 6], [9, 8, 7]], dtype=torch.int32,
                            device=cuda)
    assert torch.equal(got, expected)
    assert seen == [([0, 0], [4, 5]), ([5, 5], [8, 9]), ([5], [10])]
    assert len(gather_calls) == 1 and gather_calls[0][1]["total_k"] == 10
    assert gather_calls[0][1]["max_seqlen_k"] == 5


def test_driver_validation(cuda):
    cache = torch.zeros(6, 4 * 132, dtype=torch.uint8, device=cuda)
    q = torch.zeros(5, 64, 128, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    w = torch.ones(5, 64, dtype=torch.float32, device=cuda)
    bt = torch.tensor([[3, 1], [4, 0]], dtype=torch.int32, device=cuda)
    cu_q = torch.tensor([0, 2, 5], dtype=torch.int32, device=cuda)
    with pytest.raises(RuntimeError, match="K length must cover every Q length"):
        indexer_module.compute_prefill_topk_paged(q, w, cu_q, torch.tensor([0, 1, 5], dtype=torch.int32,
                                                                            device=cuda), bt, cache, page_size=4)
    with pytest.raises(RuntimeError, match="block table is too short"):
        indexer_module.compute_prefill_topk_paged(q, w, cu_q, torch.tensor([0, 9, 18], dtype=torch.int32,
                                                                            device=cuda), bt, cache, page_size=4)
    with pytest.raises(ValueError, match="query_chunk must be positive"):
        indexer_module.compute_prefill_topk_paged(q, w, cu_q, cu_q, bt, cache, page_size=4, query_chunk=0)
    with pytest.raises(RuntimeError, match="must start at zero"):
        indexer_module.compute_prefill_topk_paged(q, w, torch.tensor([1, 2, 5], dtype=torch.int32, device=cuda),
                                                  cu_q + 1, bt, cache, page_size=4)
    with pytest.raises(RuntimeError, match="does not cover the packed queries: 4 vs 5"):
        indexer_module.compute_prefill_topk_paged(q, w, torch.tensor([0, 2, 4], dtype=torch.int32, device=cuda),
                                                  torch.tensor([0, 5, 9], dtype=torch.int32, device=cuda), bt,
                                                  cache, page_size=4)


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_prefill_windows_match_oracle(cuda, dtype):
    """The device-side windows equal the oracle's causal [ks, ke) on a ragged
    batch with empty sequences and prefix-free ones; the status carries the
    totals the gather sizes from."""
    print(f"prefill windows {dtype}", flush=True)
    rng = np.random.default_rng(3)
    q_lens = rng.integers(0, 300, 37)
    q_lens[[0, 5, 36]] = 0
    k_lens = q_lens + rng.integers(0, 5000, 37)
    k_lens[7] = q_lens[7]                       # no cached prefix
    cu_q = np.concatenate([[0], np.cumsum(q_lens)])
    cu_k = np.concatenate([[0], np.cumsum(k_lens)])
    nq = int(cu_q[-1])
    ks = torch.empty(nq, dtype=torch.int32, device=cuda)
    ke = torch.empty_like(ks)
    status = torch.empty(4, dtype=torch.int64, device=cuda)
    ops.prefill_windows(torch.from_numpy(cu_q).to(cuda, dtype), torch.from_numpy(cu_k).to(cuda, dtype), nq, 64,
                        ks, ke, status)
    eks, eke = O.prefill_ks_ke(cu_q, cu_k)
    assert np.array_equal(ks.cpu().numpy(), eks) and np.array_equal(ke.cpu().numpy(), eke)
    assert status.tolist() == [0, int(cu_k[-1]), int(k_lens.max()), int(((k_lens + 63) // 64).max())]


def test_driver_long_rows_fused_topk_is_exact(cuda, monkeypatch):
    """top_k = 2048 over 65537- and 65538-key windows, with the logits-buffer
    path: the ragged select (clean_logits=False) is exact against torch.topk."""
    print("prefill driver long rows", flush=True)
    seen = []

    def fake_logits(q, keys, key_scales, weights, ks, ke, out, clean):
        assert clean is False
        g = torch.Generator(device=cuda).manual_seed(7)
        out.copy_(torch.randn(q.shape[0], keys.shape[0], dtype=torch.float32, device=cuda, generator=g))
        seen.append(out.clone())

    monkeypatch.setattr(indexer_module, "_score_chunk", fake_logits)
    monkeypatch.setattr(indexer_module, "PREFILL_FUSED_TOPK", False)
    cache = torch.zeros(1, 64 * 132, dtype=torch.uint8, device=cuda)
    q = torch.zeros(2, 64, 128, dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
    w = torch.ones(2, 64, dtype=torch.float32, device=cuda)
    cu_q = torch.tensor([0, 2], dtype=torch.int32, device=cuda)
    cu_k = torch.tensor([0, 65538], dtype=torch.int32, device=cuda)
    bt = torch.zeros((1, 1025), dtype=torch.int32, device=cuda)
    got = indexer_module.compute_prefill_topk_paged(q, w, cu_q, cu_k, bt, cache, page_size=64, index_topk=2048,
                                                    query_chunk=2)
    assert got.shape == (2, 2048)
    for row, length in enumerate((65537, 65538)):
        exp = set(torch.topk(seen[0][row, :length], 2048).indices.cpu().tolist())
        assert set(got[row].cpu().tolist()) == exp


def test_driver_end_to_end_against_oracle(cuda):
    """Real fp8 pages: two sequences with cached prefixes and fresh queries,
    the real logits kernel, top-2048 sets equal to torch.topk of the oracle's
    float64 logits except at near-ties (|score gap| <= 1e-3 relative)."""
    print("prefill driver end to end", flush=True)
    rng = np.random.default_rng(11)
    page_size, k_lens, q_lens = 64, [3000, 2200], [40, 24]
    pages = [(L + page_size - 1) // page_size for L in k_lens]
    perm = rng.permutation(sum(pages))
    bt = np.zeros((2, max(pages)), dtype=np.int32)
    bt[0, :pages[0]] = perm[:pages[0]]
    bt[1, :pages[1]] = perm[pages[0]:]
    keys = O.fp8_e4m3fn_encode(rng.standard_normal((sum(k_lens), 128)) * 40)
    scales = O.ue8m0_ceil(rng.uniform(1e-3, 1e-2, sum(k_lens)).astype(np.float32))
    cache = np.zeros((sum(pages), page_size * 132), dtype=np.uint8)
    cu_k = np.array([0, k_lens[0], sum(k_lens)])
    for b in range(2):
        for i in range(k_lens[b]):
            p, off = bt[b, i // page_size], i % page_size
            cache[p, off * 128:(off + 1) * 128] = keys[cu_k[b] + i]
            cache[p, page_size * 128 + off * 4:page_size * 128 + off * 4 + 4] = \
                np.frombuffer(scales[cu_k[b] + i].tobytes(), dtype=np.uint8)
    nq = sum(q_lens)
    q = O.fp8_e4m3fn_encode(rng.standard_normal((nq, 64, 128)) * 40)
    w = (rng.standard_normal((nq, 64)) * 64 ** -0.5 * 128 ** -0.5 * 1e-2).astype(np.float32)
    cu_q = np.array([0, q_lens[0], nq])
    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(cuda if dt is None else cuda)
    got = indexer_module.compute_prefill_topk_paged(
        t(q).view(torch.float8_e4m3fn), t(w), t(cu_q.astype(np.int32)), t(cu_k.astype(np.int32)), t(bt),
        t(cache), page_size=page_size, index_topk=2048).cpu().numpy()
    ks, ke = O.prefill_ks_ke(cu_q, cu_k)
    g_keys, g_scales = O.gather_indexer_cache(cache, bt, cu_k)
    exp_logits = O.mqa_logits(q, g_keys, g_scales, w, ks, ke, clean_logits=True)
    for r in range(nq):
        row = exp_logits[r, ks[r]:ke[r]].astype(np.float64)
        n = min(2048, len(row))
        sel = got[r][got[r] >= 0] - ks[r]
        assert len(sel) == n and len(set(sel.tolist())) == n
        assert np.all(got[r][n:] == -1)
        if n < 2048:
            assert set(sel.tolist()) == set(range(len(row)))
            continue
        kth = np.sort(row)[::-1][n - 1]
        tol = 1e-3 * max(abs(kth), np.sqrt(np.mean(row * row)))
        exp_set = set(np.nonzero(row > kth + tol)[0].tolist())     # certainly selected
        assert exp_set <= set(sel.tolist())
        assert np.all(row[sel] >= kth - tol)                        # nothing far below the boundary
