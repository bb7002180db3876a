"""fp8 paged indexer logits on the GPU vs the CPU oracle.

Tolerance: |gpu - oracle| <= 1e-3 * max(|oracle|, row RMS) per element (the
north-star bound "indexer logits within 1e-3 relative"; fp8 products are exact
in fp32, so the only difference is the fp32 accumulation order).
"""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import deep_gemm, indexer as nidx, synth

pytestmark = pytest.mark.gpu


def _oracle_logits(inp: synth.IndexerInputs, max_ctx: int):
    B = inp.context_lens.shape[0]
    n = inp.next_n
    q = inp.q_fp8.cpu().numpy().reshape(B, n, 64, 128)
    ctx = O.expand_decode_context_lens(inp.context_lens.cpu().numpy(), n)
    return O.indexer_logits(q, inp.cache.cpu().numpy(), inp.weights.cpu().numpy(), ctx,
                            inp.block_tables.cpu().numpy(), max_ctx), ctx


def _assert_close_rows(got, exp, ctx):
    for r in range(exp.shape[0]):
        L = int(ctx.reshape(-1)[r])
        g, e = got[r, :L].astype(np.float64), exp[r, :L].astype(np.float64)
        rms = np.sqrt(np.mean(e * e)) + 1e-30
        err = np.abs(g - e) / np.maximum(np.abs(e), rms)
        assert err.max() <= 1e-3, (r, err.max())


@pytest.mark.parametrize("next_n", [1, 2])
def test_config0_logits_match_oracle(cuda, next_n):
    lens = [1024, 2048, 3000, 4096]
    inp = synth.make_indexer_inputs(lens, next_n=next_n, seed=0, device=cuda)
    B = len(lens)
    max_ctx = inp.block_tables.shape[1] * 64
    ctx = nidx._expand_decode_context_lens(inp.context_lens, next_n)
    q4 = inp.q_fp8.view(torch.float8_e4m3fn).view(B, next_n, 64, 128)
    kv = inp.cache.view(inp.cache.shape[0], 64, 1, 132)
    meta = deep_gemm.get_paged_mqa_logits_metadata(ctx, 64, deep_gemm.get_num_sms())
    got = deep_gemm.fp8_paged_mqa_logits(q4, kv, inp.weights, ctx, inp.block_tables, meta, max_ctx,
                                         clean_logits=True)
    torch.cuda.synchronize()
    exp, ectx = _oracle_logits(inp, max_ctx)
    got = got.cpu().numpy()
    _assert_close_rows(got, exp, ectx)
    # clean_logits: everything past the context is -inf
    for r in range(B * next_n):
        assert np.all(np.isneginf(got[r, int(ectx.reshape(-1)[r]):]))
    # schedule = exclusive prefix sum of page counts
    pages = [(L + 63) // 64 for L in lens]
    assert meta.cpu().tolist() == [0] + list(np.cumsum(pages))


def test_wide_mtp_next_n_uses_per_position_launches(cuda):
    lens = [700, 1500]
    inp = synth.make_indexer_inputs(lens, next_n=3, seed=4, device=cuda)
    max_ctx = inp.block_tables.shape[1] * 64
    ctx = nidx._expand_decode_context_lens(inp.context_lens, 3)
    q4 = inp.q_fp8.view(torch.float8_e4m3fn).view(2, 3, 64, 128)
    got = deep_gemm.fp8_paged_mqa_logits(q4, inp.cache, inp.weights, ctx, inp.block_tables, None, max_ctx)
    torch.cuda.synchronize()
    exp, ectx = _oracle_logits(inp, max_ctx)
    _assert_close_rows(got.cpu().numpy(), exp, ectx)


def test_golden_config0_fixture(cuda):
    g = np.load(__file__.replace("test_gpu_indexer.py", "golden/config0_indexer.npz"))
    B, n = g["q_fp8"].shape[:2]
    q = torch.from_numpy(g["q_fp8"]).to(cuda).view(torch.float8_e4m3fn)
    got = deep_gemm.fp8_paged_mqa_logits(q, torch.from_numpy(g["cache"]).to(cuda),
                                         torch.from_numpy(g["weights"]).to(cuda),
                                         torch.from_numpy(g["context_lens"]).to(cuda).view(B, n),
                                         torch.from_numpy(g["block_tables"]).to(cuda), None,
                                         int(g["logits"].shape[1]))
    torch.cuda.synchronize()
    _assert_close_rows(got.cpu().numpy(), g["logits"], g["context_lens"])


@pytest.mark.parametrize("translate", [False, True])
def test_indexer_decode_topk_end_to_end(cuda, translate):
    lens = [64, 256, 3000, 20000]
    inp = synth.make_indexer_inputs(lens, next_n=1, seed=2, device=cuda)
    res = nidx.indexer_decode_topk(inp.q_fp8.view(torch.float8_e4m3fn), inp.weights, inp.cache,
                                   inp.context_lens, inp.block_tables, 2048, translate_topk=translate,
                                   topk_page_size=64)
    torch.cuda.synchronize()
    logical = res[0] if translate else res
    max_ctx = inp.block_tables.shape[1] * 64
    exp_logits, ectx = _oracle_logits(inp, max_ctx)
    exp = O.indexer_decode_topk(exp_logits, ectx, 2048)
    got = logical.cpu().numpy()
    for r in range(len(lens)):
        L = lens[r]
        if L <= 2048:
            assert np.array_equal(got[r], exp[r])
        else:
            # equal sets up to ties within the logits tolerance at the k-th value
            g = set(got[r][got[r] >= 0].tolist())
            e = set(exp[r][exp[r] >= 0].tolist())
            assert len(g) == 2048
            kth = np.sort(exp_logits[r, :L])[::-1][2047]
            for p in g ^ e:
                assert abs(exp_logits[r, p] - kth) <= 1e-3 * max(abs(kth), 1e-6), (r, p)
    if translate:
        phys = res[1].cpu().numpy()
        bt = inp.block_tables.cpu().numpy()
        assert np.array_equal(phys, O.topk_indices_to_physical(got, bt, 64))


def test_golden_config0_topk_transform(cuda):
    g = np.load(__file__.replace("test_gpu_indexer.py", "golden/config0_indexer.npz"))
    logits = torch.from_numpy(np.where(np.isfinite(g["logits"]), g["logits"], 0).astype(np.float32)).to(cuda)
    lens = torch.from_numpy(g["context_lens"].reshape(-1)).to(cuda)
    bt = torch.from_numpy(g["block_tables"]).to(cuda)
    out = torch.empty(4, 2048, dtype=torch.int32, device=cuda)
    raw = torch.empty_like(out)
    from nanoengine_amd import deepseek_v4
    deepseek_v4.topk_transform(logits, lens, bt, out, 64, 2048, raw)
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), g["topk_raw"])
    assert np.array_equal(out.cpu().numpy(), g["topk_page"])


def _wide_cancelling(rng, n_tok, H=64):
    """fp8 query and keys spread over ~16 binades (so the scaled fp8 MFMA
    drops low bits of most dots) and head weights in the null space of
    relu(q_h . k_t), so that every logit's head sum cancels to ~0."""
    q = O.fp8_e4m3fn_encode(np.clip(rng.standard_normal((H, 128)) * np.exp2(rng.integers(-8, 8, (H, 128))), -448, 448))
    k = O.fp8_e4m3fn_encode(np.clip(rng.standard_normal((n_tok, 128)) * np.exp2(rng.integers(-8, 8, (n_tok, 128))),
                                    -448, 448))
    d = O.fp8_e4m3fn_decode(k).astype(np.float64) @ O.fp8_e4m3fn_decode(q).astype(np.float64).T
    R = np.maximum(d, 0.0)
    w = rng.standard_normal(H) * 2.0 ** -12
    w = (w - np.linalg.pinv(R) @ (R @ w)).astype(np.float32)
    return q, k, w


def test_logits_within_the_derived_mfma_bound(cuda):
    """Rows of 2 and 40 tokens whose head sums cancel (the short-row case a
    randomised step sweep hit: a logit ~0 has no relative-error scale), with
    wide-range fp8 values, through the paged decode logits kernel. Every
    logit must lie within 1e-3 relative or within the scaled fp8 MFMA's
    derived bound (oracle ``indexer_logit_error_bound``: truncation remainders
    at 2^-13 of each dot's largest product, plus f32 rounding); here most
    logits need the bound, and none may exceed it."""
    from oracle import step_check as SC
    rng = np.random.default_rng(7)
    lens = [2, 40]
    B, H = len(lens), 64
    qs, ws, codes, scales, slots = [], [], [], [], []
    for b, L in enumerate(lens):
        q, k, w = _wide_cancelling(rng, L, H)
        qs.append(q)
        ws.append(w)
        codes.append(k)
        scales.append(np.full(L, 2.0 ** -7, np.float32))
        slots.append(64 * b + np.arange(L))
    cache = O.pack_indexer_cache(np.concatenate(codes), np.concatenate(scales), np.concatenate(slots), B)
    bt = np.arange(B, dtype=np.int32).reshape(B, 1)
    q4 = torch.from_numpy(np.stack(qs)).to(cuda).view(torch.float8_e4m3fn).view(B, 1, H, 128)
    got = ops_logits(cuda, q4, cache, np.stack(ws), lens, bt)
    exp = O.indexer_logits(np.stack(qs).reshape(B, 1, H, 128), cache, np.stack(ws), np.array(lens).reshape(B, 1),
                           bt, 64)

    def bound(r, pos):
        return O.indexer_logit_error_bound(qs[r], ws[r], codes[r][pos], scales[r][pos])
    rep = SC.check_logits(got, exp, np.array(lens), bound)
    print(rep, flush=True)
    assert rep["over_rtol"] > 0, rep        # the relative tolerance does not apply here
    assert rep["ok"], rep


def ops_logits(cuda, q4, cache, w, lens, bt):
    from nanoengine_amd import ops
    B = q4.shape[0]
    out = ops.indexer_logits(q4, torch.from_numpy(cache).to(cuda), torch.from_numpy(w).to(cuda),
                             torch.tensor(lens, dtype=torch.int32, device=cuda).view(B, 1),
                             torch.from_numpy(bt).to(cuda), 64)
    torch.cuda.synchronize()
    return out.cpu().numpy()
