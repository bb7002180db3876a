"""Pins the numpy oracle (CPU only).

Each check is chosen so that a plausible mistake in the oracle fails it:
known-answer vectors from the reference's own tests, library routines that
compute the same thing independently (torch's fp8 cast and decode, torch.topk,
einsum/softmax/logsumexp), closed forms and invariants, and brute force on tiny
inputs.
"""
import numpy as np
import pytest
import torch

import oracle as O


# ----------------------------------------------------------------- fp8 / bf16
def test_e4m3fn_decode_matches_torch_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = O.fp8_e4m3fn_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])


def test_e4m3fn_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * np.float32(40),
                        rng.standard_normal(1000).astype(np.float32) * np.float32(1e-3),
                        np.array([0, -0.0, 448, -448, 449, 463.9, 464, 464.5, 1e-9, 2 ** -9, 1.5 * 2 ** -9,
                                  2 ** -10, 0.0009765625 * 1.5], np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.fp8_e4m3fn_encode(x), ref)


def test_bf16_round_trip_and_rne():
    x = np.array([1.0, 1.00390625, 1.005859375, -3.14159, 65504.0, 1e-30], np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), ref)
    assert np.array_equal(O.bf16_to_f32(ref), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ----------------------------------------------------------------- quantisation
def test_ue8m0_row_quant_known_answers():
    # amax 448 -> scale 1; amax 449 -> scale 2; zero row -> clamp 1e-4 -> 2^-22
    rows = np.zeros((3, 128), np.float32)
    rows[0, 5] = 448.0
    rows[1, 7] = -449.0
    codes, sf = O.quantize_rows_ue8m0(rows)
    assert sf.tolist() == [1.0, 2.0, 2.0 ** -22]
    assert O.fp8_e4m3fn_decode(codes[0])[5] == 448.0
    assert O.fp8_e4m3fn_decode(codes[1])[7] == -224.0 and np.all(codes[2] == 0)


def test_ue8m0_row_quant_properties():
    rng = np.random.default_rng(1)
    x = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((500, 128)).astype(np.float32)
                                    * rng.uniform(1e-3, 1e3, (500, 1)).astype(np.float32)))
    codes, sf = O.quantize_rows_ue8m0(x)
    amax = np.abs(x).max(1)
    assert np.all(np.log2(sf) == np.round(np.log2(sf)))            # powers of two
    assert np.all(sf >= amax / 448) and np.all(sf / 2 < amax / 448)  # the smallest such
    deq = O.fp8_e4m3fn_decode(codes) * sf[:, None]
    assert np.all(np.abs(deq - x) <= np.abs(x) * 2 ** -4 + sf[:, None] * 2 ** -10)


def test_mla_row_pack_layout_and_accuracy():
    # tests/test_store_fp8.py:49-56: rope bit-exact, nope rel err < 0.06;
    # tests/test_cache_fp8.py: 656-byte rows
    rng = np.random.default_rng(2)
    kv = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((64, 576)).astype(np.float32)))
    rows = O.quantize_mla_rows(kv)
    assert rows.shape == (64, 656)
    codes, scales, rope = O.unpack_mla_rows(rows)
    assert np.array_equal(rope, O.f32_to_bf16(kv[:, 512:]))
    assert np.all(np.log2(scales) == np.round(np.log2(scales)))
    deq = O.dequant_mla_rows(rows)
    err = np.abs(deq[:, :512] - kv[:, :512]).max(1) / np.abs(kv[:, :512]).max(1)
    assert np.all(err < 0.06)
    assert np.array_equal(deq[:, 512:], kv[:, 512:])
    # byte offsets: scales at [512, 528) as 4 little-endian f32
    assert np.array_equal(rows[:, 512:528].copy().view(np.float32), scales)


def test_indexer_cache_split_page_layout():
    # tests/test_indexer_fp8_kernels.py:39-74: fp8 block first, scales after
    rng = np.random.default_rng(3)
    k = rng.standard_normal((3, 128)).astype(np.float32)
    codes, sf = O.quantize_rows_ue8m0(k)
    cache = O.pack_indexer_cache(codes, sf, np.array([5, 70, 130]), num_pages=3)
    flat = cache.reshape(-1)
    for tok, slot in enumerate([5, 70, 130]):
        page, off = divmod(slot, 64)
        base = page * 64 * 132
        assert np.array_equal(flat[base + off * 128: base + off * 128 + 128], codes[tok])
        assert flat[base + 64 * 128 + off * 4: base + 64 * 128 + off * 4 + 4].view(np.float32)[0] == sf[tok]
        c2, s2 = O.indexer_cache_token(cache, slot)
        assert np.array_equal(c2, codes[tok]) and s2 == sf[tok]


# ----------------------------------------------------------------- indexer
def test_expand_decode_context_lens_known_answers():
    # tests/test_shared_indexer.py:162-181
    assert O.expand_decode_context_lens(np.array([4098, 513]), 2).tolist() == [[4097, 4098], [512, 513]]
    assert O.expand_decode_context_lens(np.array([1]), 8).tolist() == [[1] * 8]
    with pytest.raises(ValueError):
        O.expand_decode_context_lens(np.zeros((2, 3)), 2)


def test_weighted_relu_counterexample_to_folding():
    # tests/test_indexer_prefill.py:68-80: relu before the head sum
    q = np.array([[2.0], [-1.0]])
    w = np.array([1.0, 3.0])
    k = np.array([[10.0], [-1.0]])
    s = np.ones(2)
    correct = O.indexer_logits_bruteforce(q, w, k, s)
    folded = (w @ q) @ k.T
    assert int(np.argmax(correct)) == 0 and int(np.argmax(folded)) == 1


def test_indexer_logits_vs_bruteforce_paged():
    rng = np.random.default_rng(4)
    lens = [70, 129]
    P = 64
    pages = [(L + P - 1) // P for L in lens]
    total = sum(pages)
    perm = rng.permutation(total)
    bt = np.zeros((2, max(pages)), np.int32)
    bt[0, :pages[0]] = perm[:pages[0]]
    bt[1, :pages[1]] = perm[pages[0]:]
    q = rng.standard_normal((2, 1, 4, 128)).astype(np.float32)
    qc = np.stack([O.quantize_rows_ue8m0(q[b, 0])[0] for b in range(2)])[:, None]
    k = rng.standard_normal((total * P, 128)).astype(np.float32)
    kc, ks = O.quantize_rows_ue8m0(k)
    cache = O.pack_indexer_cache(kc, ks, np.arange(total * P), total)
    w = rng.standard_normal((2, 4)).astype(np.float32)
    # the oracle takes 64 heads in production; the formula is head-count agnostic
    got = O.indexer_logits(qc, cache, w, np.array(lens).reshape(2, 1), bt, bt.shape[1] * P)
    for b, L in enumerate(lens):
        slots = [bt[b, t // P] * P + t % P for t in range(L)]
        kk = O.fp8_e4m3fn_decode(kc[slots])
        ref = O.indexer_logits_bruteforce(O.fp8_e4m3fn_decode(qc[b, 0]), w[b], kk, ks[slots])
        np.testing.assert_allclose(got[b, :L], ref, rtol=2e-6, atol=1e-6)
        assert np.all(np.isneginf(got[b, L:]))


def test_indexer_logits_scale_commutes_with_relu():
    # w folds q_scale (lightning.py:1269-1271): relu(s x) = s relu(x) for s > 0
    rng = np.random.default_rng(5)
    qc = rng.integers(0, 120, (1, 1, 64, 128)).astype(np.uint8)
    k = rng.standard_normal((64, 128)).astype(np.float32)
    kc, ks = O.quantize_rows_ue8m0(k)
    cache = O.pack_indexer_cache(kc, ks, np.arange(64), 1)
    w = rng.standard_normal((1, 64)).astype(np.float32)
    bt = np.zeros((1, 1), np.int32)
    a = O.indexer_logits(qc, cache, w * 4.0, np.array([[64]]), bt, 64)
    b = O.indexer_logits(qc, cache, w, np.array([[64]]), bt, 64)
    np.testing.assert_allclose(a, 4.0 * b, rtol=1e-6)


# ----------------------------------------------------------------- top-k
def test_topk_select_matches_torch_topk_sets():
    rng = np.random.default_rng(6)
    for L in [3000, 16384, 70000]:
        x = rng.standard_normal(L).astype(np.float32)
        got = O.topk_select(x, L, 2048)
        ref = torch.topk(torch.from_numpy(x), 2048).indices.numpy()
        assert np.array_equal(np.sort(ref), got)


def test_topk_select_ties_short_rows_and_nan():
    assert np.array_equal(O.topk_select(np.zeros(5000, np.float32), 5000, 2048), np.arange(2048))
    assert np.array_equal(O.topk_select(np.zeros(100, np.float32), 100, 2048), np.arange(100))
    x = np.full(4000, np.nan, np.float32)
    x[3000:] = -np.inf
    x[:10] = 1.0
    sel = O.topk_select(x, 4000, 512)
    assert set(range(10)) <= set(sel.tolist())
    # NaN ranks as -inf: among the rest, the lowest positions win
    assert np.array_equal(sel, np.arange(512))


def test_topk_transform_known_answers_and_padding():
    scores = np.zeros((2, 256), np.float32)
    scores[0, [3, 100, 200]] = [5, 4, 3]
    pt = np.array([[7, 2, 9, 4], [1, 1, 1, 1]], np.int32)
    page, raw = O.topk_transform(scores, np.array([256, 40]), pt, 64, 512)
    assert raw[0, :256].tolist() == list(range(256)) and np.all(raw[0, 256:] == -1)
    assert page[0, 3] == 7 * 64 + 3 and page[0, 100] == 2 * 64 + 36 and page[0, 200] == 4 * 64 + 8
    assert raw[1, :40].tolist() == list(range(40)) and np.all(page[1, 40:] == -1)
    with pytest.raises(ValueError, match="512 or 2048"):
        O.topk_transform(scores, np.array([1, 1]), pt, 64, 100)
    with pytest.raises(ValueError, match="power of 2"):
        O.topk_transform(scores, np.array([1, 1]), pt, 48, 512)


def test_topk_transform_ragged_offsets():
    rng = np.random.default_rng(7)
    s = rng.standard_normal((2, 5000)).astype(np.float32)
    out = O.topk_transform_ragged(s, np.array([17, 4096]), np.array([9, 123]), np.array([0, 17]), 2048)
    assert out[0, :17].tolist() == list(range(17)) and np.all(out[0, 17:] == -1)
    ref = torch.topk(torch.from_numpy(s[1, 123:123 + 4096]), 2048).indices.numpy() + 17
    assert np.array_equal(np.sort(ref), out[1])


def test_topk_indices_to_physical_known_answers():
    # tests/test_sparse_decode.py:98-161
    f = O.topk_indices_to_physical
    assert f(np.array([[0, 65, 192, 130]]), np.array([[5, 10, 2, 8]]), 64).tolist() == [[320, 641, 512, 130]]
    assert f(np.array([[10, -1, 70, -1]]), np.array([[3, 7]]), 64).tolist() == [[3 * 64 + 10, -1, 7 * 64 + 6, -1]]
    assert f(np.array([[0, 64], [63, 127]]), np.array([[1, 2], [5, 6]]), 64).tolist() == [[64, 128], [383, 447]]


def test_indexer_decode_topk_masks_and_pads():
    # lightning.py:1468-1492 semantics: positions >= ctx never chosen, |x|>=1e30 is -inf, pad -1
    logits = np.zeros((2, 3000), np.float32)
    logits[0, 2500:] = 100.0   # beyond ctx 2500
    logits[1, :5] = 1e31       # garbage-sized values -> -inf
    out = O.indexer_decode_topk(logits, np.array([2500, 3000]), 2048)
    assert out[0].max() < 2500 and np.all(out[0] >= 0)
    assert not set(range(5)) & set(out[1].tolist())
    out = O.indexer_decode_topk(np.zeros((1, 3000), np.float32), np.array([100]), 2048)
    assert out[0, :100].tolist() == list(range(100)) and np.all(out[0, 100:] == -1)


# ----------------------------------------------------------------- sparse MLA
def test_sparse_mla_matches_torch_softmax_reference():
    # tests/test_mla_decode_head_padding.py:30-33 dense math on the selected rows
    rng = np.random.default_rng(8)
    kv = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((300, 576)).astype(np.float32)))
    rows = O.quantize_mla_rows(kv)
    q = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((3, 8, 576)).astype(np.float32)))
    idx = np.stack([rng.permutation(300)[:128] for _ in range(3)]).astype(np.int32)
    idx[1, ::3] = -1
    scale = 192 ** -0.5
    o, lse = O.sparse_mla_decode(q, rows, idx, scale)
    deq = torch.from_numpy(O.dequant_mla_rows(rows)).double()
    for t in range(3):
        sel = deq[torch.from_numpy(idx[t][idx[t] >= 0]).long()]
        s = torch.from_numpy(q[t]).double() @ sel.T * scale
        ref = torch.softmax(s, -1) @ sel[:, :512]
        np.testing.assert_allclose(o[t], ref.numpy(), atol=1e-6, rtol=1e-5)
        np.testing.assert_allclose(lse[t], torch.logsumexp(s, -1).numpy(), atol=1e-5, rtol=0)


def test_sparse_mla_invalid_rows_and_merge_rule():
    rng = np.random.default_rng(9)
    kv = rng.standard_normal((128, 576)).astype(np.float32)
    rows = O.quantize_mla_rows(kv)
    q = rng.standard_normal((1, 4, 576)).astype(np.float32)
    idx = np.arange(128, dtype=np.int32)[None]
    o, lse = O.sparse_mla_decode(q, rows, idx, 0.1)
    # splitting the index list and merging by LSE (mla_utils.py:12-23) gives the same result
    o1, l1 = O.sparse_mla_decode(q, rows, idx[:, :50], 0.1)
    o2, l2 = O.sparse_mla_decode(q, rows, idx[:, 50:], 0.1)
    m = np.logaddexp(l1, l2)
    merged = o1 * np.exp(l1 - m)[..., None] + o2 * np.exp(l2 - m)[..., None]
    np.testing.assert_allclose(merged, o, atol=1e-5)
    np.testing.assert_allclose(m, lse, atol=1e-5)
    # no valid index: o = 0, lse = -inf
    o0, l0 = O.sparse_mla_decode(q, rows, np.full((1, 64), -1, np.int32), 0.1)
    assert np.all(o0 == 0) and np.all(np.isneginf(l0))


def test_sparse_mla_prefill_matches_torch_and_decode_oracle():
    """The bf16-row prefill oracle against (a) torch softmax / logsumexp / max on
    the gathered rows, (b) the fp8 decode oracle on the same rows dequantised
    (fp8 times a power-of-two scale is exact in bf16), (c) the split-and-merge
    rule, and the skip rules (negative and out-of-range indices)."""
    rng = np.random.default_rng(12)
    kv = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((300, 576)).astype(np.float32)))
    rows8 = O.quantize_mla_rows(kv)
    kv_deq = O.dequant_mla_rows(rows8)
    q = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((3, 8, 576)).astype(np.float32)))
    idx = np.stack([rng.permutation(300)[:128] for _ in range(3)]).astype(np.int32)
    idx[1, ::3] = -1
    idx[2, ::5] = 300 + 7          # past s_kv: skipped
    scale = 192 ** -0.5
    o, mx, lse = O.sparse_mla_prefill(q, kv_deq, idx, scale)
    for t in range(3):
        sel = torch.from_numpy(kv_deq[idx[t][(idx[t] >= 0) & (idx[t] < 300)]]).double()
        s = torch.from_numpy(q[t]).double() @ sel.T * scale
        np.testing.assert_allclose(o[t], (torch.softmax(s, -1) @ sel[:, :512]).numpy(), atol=1e-6, rtol=1e-5)
        np.testing.assert_allclose(lse[t], torch.logsumexp(s, -1).numpy(), atol=1e-5, rtol=0)
        np.testing.assert_allclose(mx[t], s.max(-1).values.numpy(), atol=1e-5, rtol=0)
    idx_dec = np.where(idx >= 300, -1, idx)
    od, ld = O.sparse_mla_decode(q, rows8, idx_dec, scale)
    np.testing.assert_allclose(o, od, atol=1e-6)
    np.testing.assert_allclose(lse, ld, atol=1e-6)
    o1, _, l1 = O.sparse_mla_prefill(q, kv_deq, idx[:, :40], scale)
    o2, _, l2 = O.sparse_mla_prefill(q, kv_deq, idx[:, 40:], scale)
    m = np.logaddexp(l1, l2)
    np.testing.assert_allclose(o1 * np.exp(l1 - m)[..., None] + o2 * np.exp(l2 - m)[..., None], o, atol=1e-5)
    o0, m0, l0 = O.sparse_mla_prefill(q, kv_deq, np.full((3, 32), -1, np.int32), scale)
    assert np.all(o0 == 0) and np.all(np.isneginf(l0)) and np.all(np.isneginf(m0))


def test_step_check_catches_wrong_outputs():
    """The sampled-row step checker passes the oracle's own outputs and fails
    each plausible mistake: a shifted physical slot, a swapped selected
    position, a perturbed logit, a perturbed o."""
    from oracle import step_check as SC
    rng = np.random.default_rng(3)
    S, L, P, H, K = 2, 1200, 64, 4, 512
    npg = (L + P - 1) // P
    bt = rng.permutation(3 * npg)[:S * npg].reshape(S, npg).astype(np.int32)
    used, btl = SC.localize_pages(bt, np.full(S, L), P)
    assert np.array_equal(used[btl], bt)
    codes = rng.integers(0, 0x7e, size=(used.size, P * 128), dtype=np.uint8)
    scales = np.full((used.size, P), 0.5, np.float32).view(np.uint8)
    pages = np.concatenate([codes, scales], axis=1)
    q = rng.integers(0, 0x7e, size=(S, 1, 64, 128), dtype=np.uint8)
    w = rng.standard_normal((S, 64)).astype(np.float32) * 0.01
    ctx = np.full(S, L, np.int32)
    logits = O.indexer_logits(q, pages, w, ctx.reshape(S, 1), btl, npg * P, P)
    phys, raw = O.topk_transform(logits, ctx, bt, P, K)
    qm = rng.standard_normal((S, H, 576)).astype(np.float32)
    kv_sel = O.quantize_mla_rows(rng.standard_normal((S * K, 576)).astype(np.float32)).reshape(S, K, 656)
    o = np.zeros((S, H, 512), np.float32)
    lse = np.zeros((S, H), np.float32)
    for r in range(S):
        eo, el = O.sparse_mla_decode(qm[r:r + 1], kv_sel[r], np.arange(K)[None], 0.1)
        o[r], lse[r] = eo[0], el[0]
    base = dict(q_idx=q, idx_pages=pages, weights=w, ctx=ctx, bt_local=btl, bt_global=bt, max_ctx=npg * P,
                gpu_logits=logits.copy(), gpu_logical=raw.copy(), gpu_physical=phys.copy(), q_mla=qm,
                kv_sel=kv_sel, gpu_o=o.copy(), gpu_lse=lse.copy(), sm_scale=0.1, topk=K, page_size=P)
    assert SC.check_step_rows(**base)["ok"]
    bad = dict(base, gpu_physical=phys + 1)
    assert not SC.check_step_rows(**bad)["ok"]
    unsel = np.setdiff1d(np.arange(L), raw[0])[0]
    lg2 = raw.copy()
    lg2[0, 0] = unsel
    lg2[0] = np.sort(lg2[0])
    assert not SC.check_step_rows(**dict(base, gpu_logical=lg2))["ok"]
    lgt = logits.copy()
    lgt[1, 5] *= 1.1
    assert not SC.check_step_rows(**dict(base, gpu_logits=lgt))["ok"]
    o2 = o.copy()
    o2[1, 2, 3] += 0.05
    assert not SC.check_step_rows(**dict(base, gpu_o=o2))["ok"]


def _cancelling_row(seed):
    """A query token, 8 keys and head weights whose weighted head sums all
    cancel: w lies in the null space of relu(q_h . k_t) [8 x 64], so every
    logit sum_h w_h relu(q_h . k_t) is ~0 and the row has no RMS scale."""
    rng = np.random.default_rng(seed)
    q = O.fp8_e4m3fn_encode(np.clip(rng.standard_normal((64, 128)) * 60, -440, 440))
    k = O.fp8_e4m3fn_encode(np.clip(rng.standard_normal((8, 128)) * 60, -440, 440))
    s = np.full(8, 2.0 ** -10, np.float32)
    qf, kf = O.fp8_e4m3fn_decode(q).astype(np.float64), O.fp8_e4m3fn_decode(k).astype(np.float64)
    d = kf @ qf.T                                              # [8, 64]
    R = np.maximum(d, 0.0)
    w = rng.standard_normal(64) * 64 ** -0.5 * 2.0 ** -9
    w = w - np.linalg.pinv(R) @ (R @ w)                        # project onto the null space of R
    return q, k, s, w.astype(np.float32), qf, kf, d


def test_mfma_logit_bound_accepts_truncated_sums_and_rejects_wrong_head_sums():
    """The derived bound of the scaled fp8 MFMA (indexer_logit_error_bound) on
    a row whose head sums all cancel, where 1e-3 relative has no scale:
    * the exact logits are ~0 and the bound is a small share (< 5%) of the
      logit's magnitude sum sum_h |w_h| relu(q_h . k) s, so it is not vacuous;
    * sums whose products are truncated toward zero at 2^-13 of the largest
      product (the behaviour the GPU probe measures) pass check_logits;
    * a wrong head sum fails it: one head dropped, |w| for w, no ReLU, the
      weights shifted by one head, the key scale left out."""
    from oracle import step_check as SC
    for seed in range(3):
        q, k, s, w, qf, kf, d = _cancelling_row(seed)
        wd = w.astype(np.float64)
        exact = (np.maximum(d, 0.0) @ wd) * s
        mag = (np.maximum(d, 0.0) @ np.abs(wd)) * s
        assert np.all(np.abs(exact) < 1e-6 * mag)
        B = O.indexer_logit_error_bound(q, w, k, s)
        assert np.all(B > 0) and np.all(B < 5e-2 * mag), (B / mag)
        # products truncated toward zero at 2^(E-13): within the bound
        P = kf[:, None, :] * qf[None, :, :]
        quantum = np.exp2(np.floor(np.log2(np.abs(P).max(-1))) - 13)[..., None]
        dt = (np.trunc(P / quantum) * quantum).sum(-1)
        trunc_logit = ((np.maximum(dt, 0.0) @ wd) * s)[None, :]
        ctx = np.array([8])
        bound = SC.ragged_logit_bound(q[None], w[None], k, s)
        rep = SC.check_logits(trunc_logit.astype(np.float32), exact[None].astype(np.float32), ctx, bound)
        assert rep["ok"] and rep["over_rtol"] == 8, rep
        hot = int(np.argmax(np.abs(wd) * np.maximum(d, 0.0).sum(0)))   # a head that contributes
        wrong = {
            "dropped head": (np.maximum(np.delete(d, hot, axis=1), 0.0) @ np.delete(wd, hot)) * s,
            "abs weights": (np.maximum(d, 0.0) @ np.abs(wd)) * s,
            "no relu": (d @ wd) * s,
            "shifted weights": (np.maximum(d, 0.0) @ np.roll(wd, 1)) * s,
        }
        for name, val in wrong.items():
            rep = SC.check_logits(val[None].astype(np.float32), exact[None].astype(np.float32), ctx, bound)
            assert not rep["ok"], (name, rep)


def test_mfma_dot_bound_two_product_probe():
    """fp8_dot_error_bound on the two-product probe 2^p + 1.875 (one output of
    the scaled MFMA): the GPU keeps 1.875 exactly to p = 10, then 1.75, 1.5,
    1.0, then nothing (bench.py --micro, fp8_mfma_sum); the bound's remainder
    term equals each observed loss exactly (the bound adds one quantum for
    the one addition and one f32 rounding)."""
    kept = {11: 1.75, 12: 1.5, 13: 1.0, 14: 0.0, 15: 0.0, 16: 0.0}
    for p in range(17):
        a = min(p, 8)
        q = np.zeros((1, 128)); k = np.zeros((1, 128))
        q[0, 0], k[0, 0] = 2.0 ** a, 2.0 ** (p - a)
        q[0, 1], k[0, 1] = 1.875, 1.0
        dots, bnd = O.fp8_dot_error_bound(q, k)
        lost = 1.875 - kept.get(p, 1.875)
        assert dots[0, 0] == 2.0 ** p + 1.875
        quantum = 2.0 ** (p - O.MFMA_FP8_BITS)
        assert bnd[0, 0] - O.F32_EPS * dots[0, 0] - quantum == pytest.approx(lost, abs=1e-12), p
