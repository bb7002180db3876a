"""Pins the oracle's prefill-indexer pieces on the CPU: the ragged key windows,
the paged-to-ragged cache gather and the ragged MQA logits.

Known answers come from the reference's tests/test_indexer_prefill.py (the
windows of :258-335, the fragmented-page gather of :168-225, the weighted-ReLU
counterexample of :68-80); the logits are checked against the scalar brute
force and against the paged decode oracle on the same keys.
"""
import numpy as np

import oracle as O


def test_prefill_windows_match_reference_known_answer():
    # tests/test_indexer_prefill.py:317-334: cu_q [0,2,5], cu_k [0,5,10]
    ks, ke = O.prefill_ks_ke(np.array([0, 2, 5]), np.array([0, 5, 10]))
    assert ks.tolist() == [0, 0, 5, 5, 5]
    assert ke.tolist() == [4, 5, 8, 9, 10]


def test_gather_matches_reference_fragmented_pages():
    # tests/test_indexer_prefill.py:168-225
    page_size, head_dim, num_pages = 64, 128, 6
    cache = np.zeros((num_pages, page_size * (head_dim + 4)), dtype=np.uint8)
    for page in range(num_pages):
        cache[page, :page_size * head_dim] = ((np.arange(page_size * head_dim) + page * 17) % 251).astype(np.uint8)
        sc = (np.arange(page_size, dtype=np.float32) + page * 100 + 0.25).astype(np.float32)
        cache[page, page_size * head_dim:] = sc.view(np.uint8)
    bt = np.array([[3, 1, 5], [4, 0, 2]])
    keys, scales = O.gather_indexer_cache(cache, bt, np.array([0, 70, 135]))

    def page_keys(p):
        return cache[p, :page_size * head_dim].reshape(page_size, head_dim)

    def page_scales(p):
        return cache[p, page_size * head_dim:].copy().view(np.float32)

    exp_k = np.concatenate([page_keys(3), page_keys(1)[:6], page_keys(4), page_keys(0)[:1]])
    exp_s = np.concatenate([page_scales(3), page_scales(1)[:6], page_scales(4), page_scales(0)[:1]])
    assert np.array_equal(keys, exp_k)
    assert np.array_equal(scales, exp_s)


def _codes(rng, shape, scale=1.0):
    return O.fp8_e4m3fn_encode(rng.standard_normal(shape) * scale)


def test_mqa_logits_matches_bruteforce_and_windows():
    rng = np.random.default_rng(0)
    M, H, N = 5, 3, 9
    q = _codes(rng, (M, H, 128))
    kv = _codes(rng, (N, 128))
    sc = rng.uniform(0.5, 2.0, N).astype(np.float32)
    w = rng.standard_normal((M, H)).astype(np.float32)
    ks = np.array([0, 0, 2, 4, 3], np.int32)
    ke = np.array([4, 5, 9, 7, 3], np.int32)
    got = O.mqa_logits(q, kv, sc, w, ks, ke)
    qf, kf = O.fp8_e4m3fn_decode(q), O.fp8_e4m3fn_decode(kv)
    for i in range(M):
        bf = O.indexer_logits_bruteforce(qf[i], w[i], kf, sc)
        for j in range(N):
            if ks[i] <= j < ke[i]:
                np.testing.assert_allclose(got[i, j], bf[j], rtol=1e-6, atol=1e-6)
            else:
                assert got[i, j] == -np.inf
    assert np.all(np.isneginf(got[4]))       # empty window


def test_mqa_logits_relu_before_head_sum():
    # tests/test_indexer_prefill.py:68-80: folding the weights into one query picks the wrong key
    q = np.zeros((1, 2, 128), np.float32)
    q[0, 0, 0], q[0, 1, 0] = 2.0, -1.0
    k = np.zeros((2, 128), np.float32)
    k[0, 0], k[1, 0] = 10.0, -1.0
    w = np.array([[1.0, 3.0]], np.float32)
    got = O.mqa_logits(O.fp8_e4m3fn_encode(q), O.fp8_e4m3fn_encode(k), np.ones(2, np.float32), w,
                       np.array([0]), np.array([2]))
    assert got[0].tolist() == [20.0, 3.0]
    folded = (w[0] @ q[0]) @ k.T
    assert np.argmax(folded) == 1 and np.argmax(got[0]) == 0


def test_mqa_logits_equals_paged_decode_logits():
    """A prefill row whose window is a whole sequence equals the decode logits of
    the paged oracle over the same keys."""
    rng = np.random.default_rng(1)
    L, H = 150, 64
    keys = _codes(rng, (L, 128))
    scales = O.ue8m0_ceil(rng.uniform(1e-3, 1e-1, L).astype(np.float32))
    pages = rng.permutation(4)
    slots = (pages[np.arange(L) // 64] * 64 + np.arange(L) % 64)
    cache = O.pack_indexer_cache(keys, scales, slots, 4)
    q = _codes(rng, (1, 1, H, 128))
    w = rng.standard_normal((1, H)).astype(np.float32)
    dec = O.indexer_logits(q, cache, w, np.array([[L]]), pages[None, :], L)
    g_keys, g_scales = O.gather_indexer_cache(cache, pages[None, :], np.array([0, L]))
    assert np.array_equal(g_keys, keys) and np.array_equal(g_scales, scales)
    pre = O.mqa_logits(q[0], g_keys, g_scales, w, np.array([0]), np.array([L]))
    np.testing.assert_allclose(pre, dec, rtol=1e-6)


def test_assemble_prefill_kv_known_answer():
    """Two sequences over a 2-row-block cache: sequence 0 has 2 cached keys
    (slots 2, 3 through block_table [1, 0]) and 1 fresh; sequence 1 is all
    fresh. Row values are small integers, exact through fp8 and bf16."""
    slots = 4
    src = np.zeros((slots, 576), np.float32)
    for s in range(slots):
        src[s, :512] = s + 1
        src[s, 512:] = -(s + 1)
    cache = O.quantize_mla_rows(src)
    fresh = np.stack([np.full(576, 100.0 + j, np.float32) for j in range(3)])
    got = O.assemble_prefill_kv(cache, 2, np.array([[1, 0], [0, 1]]), np.array([0, 1, 3]), np.array([0, 3, 5]),
                                fresh)
    exp = np.stack([src[2], src[3], fresh[0], fresh[1], fresh[2]])
    assert np.array_equal(got, exp)
    # no cached prefix anywhere: the fresh rows unchanged
    assert np.array_equal(O.assemble_prefill_kv(cache, 2, np.zeros((1, 1), int), np.array([0, 3]),
                                                np.array([0, 3]), fresh), fresh)
