"""Sparse MLA decode on the GPU vs the CPU oracle.

Tolerances (north star): o within bf16 atol 2e-2, LSE within 1e-3 (absolute,
natural log). The rows' fp8 values times their power-of-two tile scales are
exact in bf16, so the score products are exact and only their f32 summation
rounds. The remaining differences are the bf16 rounding of P and the fp32
accumulation order.
"""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import flash_mla, ops, synth

pytestmark = pytest.mark.gpu


def _case(T, H, K, num_blocks, seed, invalid_frac=0.0, device="cuda"):
    kv = synth.make_mla_cache(num_blocks, seed=seed, device=device)
    q = synth.make_mla_query(T, H, seed=seed, device=device)
    g = torch.Generator(device="cpu").manual_seed(seed)
    idx = torch.stack([torch.randperm(num_blocks * 64, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    if invalid_frac:
        idx[torch.rand(T, K, generator=g) < invalid_frac] = -1
    return q, kv, idx.to(device)


def _oracle(q, kv, idx, scale):
    rows = kv.reshape(-1, 656).cpu().numpy() if kv.is_contiguous() else \
        kv.contiguous().reshape(-1, 656).cpu().numpy()
    qf = q.float().cpu().numpy()
    return O.sparse_mla_decode(qf, rows, idx.cpu().numpy(), scale)


def _check(o, lse, eo, elv, lse_atol=1e-3):
    o = o.float().cpu().numpy()
    lse = lse.cpu().numpy()
    assert np.abs(o - eo).max() <= 2e-2
    fin = np.isfinite(elv)
    assert np.array_equal(np.isfinite(lse), fin)
    assert np.abs(lse[fin] - elv[fin]).max() <= lse_atol


@pytest.mark.parametrize("T,H,K,splits", [(2, 128, 2048, 1), (3, 128, 512, 4), (4, 64, 256, 2), (2, 16, 128, 1)])
def test_matches_oracle(cuda, T, H, K, splits):
    q, kv, idx = _case(T, H, K, num_blocks=80, seed=T * 1000 + K)
    scale = 192 ** -0.5
    # oracle addresses slots as block*64+row in a dense [blocks*64, 656] view
    o, lse = ops.sparse_mla_decode(q, kv, idx, scale, num_splits=splits)
    torch.cuda.synchronize()
    eo, elv = _oracle(q, kv, idx, scale)
    _check(o, lse, eo, elv)


@pytest.mark.parametrize("splits", [1, 2])
def test_large_score_jumps_redo_blocks(cuda, splits):
    """A softmax scale of 1 spreads the scores over hundreds of log2 units:
    later blocks overshoot the running maximum by more than 2^64, so the lazy
    rescale of O and l (which waits for a rise of 2^8) runs on many blocks with
    large factors, and the online softmax must still match the oracle."""
    T, H, K = 3, 128, 2048
    q, kv, idx = _case(T, H, K, num_blocks=80, seed=17)
    scale = 1.0
    print(f"mla large jumps splits={splits}", flush=True)
    o, lse = ops.sparse_mla_decode(q, kv, idx, scale, num_splits=splits)
    torch.cuda.synchronize()
    eo, elv = _oracle(q, kv, idx, scale)
    # precondition: some head's block maximum (list order, 64-key blocks within
    # each split) exceeds the running maximum of the earlier blocks by > 64 (log2)
    rows = kv.reshape(-1, 656).cpu().numpy()
    deq = O.dequant_mla_rows(rows)
    sel = deq[idx.cpu().numpy()]                                        # [T, K, 576]
    sc = np.einsum("thd,tkd->thk", q.float().cpu().numpy().astype(np.float64), sel.astype(np.float64))
    sc *= scale / np.log(2.0)
    blk = sc.reshape(T, H, splits, K // splits // 64, 64).max(axis=-1)   # [T, H, splits, blocks]
    run = np.maximum.accumulate(blk, axis=-1)
    assert np.any(blk[..., 1:] - run[..., :-1] > 64.0)
    # the scores' rounding error grows with the softmax scale: the LSE bound is
    # the north-star 1e-3 scaled from 192**-0.5 to 1
    _check(o, lse, eo, elv, lse_atol=1e-3 / 192 ** -0.5)


def test_key_half_far_below_the_other(cuda):
    """Each 64-key block holds the token's best keys in its first 32 slots and
    its worst in the last 32 (ordered by head 0's score, softmax scale 1), so
    the second key half's reference falls more than 2^30 below the first's:
    P.V scales that half by 2^-30 instead of its true, smaller factor (which
    keeps the bf16 exponent arithmetic normal) and the output must still match
    the oracle."""
    T, H, K = 2, 128, 2048
    q, kv, idx = _case(T, H, K, num_blocks=80, seed=23)
    scale = 1.0
    rows = kv.reshape(-1, 656).cpu().numpy()
    deq = O.dequant_mla_rows(rows).astype(np.float64)
    qf = q.float().cpu().numpy().astype(np.float64)
    ih = idx.cpu().numpy()
    for t in range(T):
        order = np.argsort(-(deq[ih[t]] @ qf[t, 0]))          # best first, by head 0
        best, worst = ih[t][order[:K // 2]], ih[t][order[K // 2:]][::-1]
        ih[t] = np.stack([best.reshape(-1, 32), worst.reshape(-1, 32)], 1).reshape(-1)
    idx = torch.from_numpy(ih).to(cuda)
    # precondition: for head 0, some block's second-half reference (running
    # maximum, log2 units) is more than 30 below the first half's
    sc = np.einsum("td,tkd->tk", qf[:, 0], deq[ih]) * scale / np.log(2.0)
    halves = sc.reshape(T, K // 64, 2, 32).max(-1)
    run = np.maximum.accumulate(halves, axis=1)
    assert np.any(run[:, :, 0] - run[:, :, 1] > 30.0)
    print("mla key halves far apart", flush=True)
    o, lse = ops.sparse_mla_decode(q, kv, idx, scale, num_splits=1)
    torch.cuda.synchronize()
    eo, elv = _oracle(q, kv, idx, scale)
    _check(o, lse, eo, elv, lse_atol=1e-3 / 192 ** -0.5)


def test_invalid_indices_and_empty_rows(cuda):
    q, kv, idx = _case(3, 128, 1024, num_blocks=40, seed=3, invalid_frac=0.3)
    idx[1] = -1                         # a query with no valid index: o = 0, lse = -inf
    idx[2, 64:] = -1                    # only the first block valid
    scale = 192 ** -0.5
    for splits in (1, 4):
        o, lse = ops.sparse_mla_decode(q, kv, idx, scale, num_splits=splits)
        torch.cuda.synchronize()
        eo, elv = _oracle(q, kv, idx, scale)
        _check(o, lse, eo, elv)
        assert torch.all(o[1] == 0) and torch.all(torch.isneginf(lse[1]))


def test_slots_past_the_cache_are_skipped(cuda):
    """A slot whose block lies past the cache (a stale index) is skipped like -1
    rather than read out of bounds."""
    q, kv, idx = _case(2, 128, 512, num_blocks=40, seed=5)
    bad = idx.clone()
    g = torch.Generator(device="cpu").manual_seed(5)
    past = torch.rand(bad.shape, generator=g) < 0.25
    bad[past.to(bad.device)] = 40 * 64 + 7          # block 40 of a 40-block cache
    ref = idx.clone()
    ref[past.to(ref.device)] = -1
    scale = 192 ** -0.5
    for splits in (1, 2):
        o, lse = ops.sparse_mla_decode(q, kv, bad, scale, num_splits=splits)
        eo, el = ops.sparse_mla_decode(q, kv, ref, scale, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(o, eo) and torch.equal(lse, el)


def test_split_counts_agree(cuda):
    q, kv, idx = _case(2, 128, 2048, num_blocks=64, seed=8)
    outs = [ops.sparse_mla_decode(q, kv, idx, 0.07, num_splits=s) for s in (1, 2, 8, 32)]
    torch.cuda.synchronize()
    base_o, base_l = outs[0]
    for o, l in outs[1:]:
        assert (o.float() - base_o.float()).abs().max().item() <= 1e-2
        assert (l - base_l).abs().max().item() <= 1e-4


def test_flash_mla_signature_and_dense_reference(cuda):
    # the reference's dense einsum check (tests/test_mla_decode_head_padding.py:30-33)
    B, n, H, K = 2, 2, 128, 512
    q, kv, idx = _case(B * n, H, K, num_blocks=32, seed=21)
    sched, _ = flash_mla.get_mla_metadata()
    o, lse = flash_mla.flash_mla_with_kvcache(q.view(B, n, H, 576), kv, None, None, 512, sched, None,
                                              192 ** -0.5, False, is_fp8_kvcache=True,
                                              indices=idx.view(B, n, K))
    torch.cuda.synchronize()
    assert o.shape == (B, n, H, 512) and lse.shape == (B, H, n)
    rows = torch.from_numpy(O.dequant_mla_rows(kv.contiguous().reshape(-1, 656).cpu().numpy()))
    sel = rows[idx.cpu().long()]                                     # [T, K, 576]
    scores = torch.einsum("thd,tkd->thk", q.float().cpu(), sel) * 192 ** -0.5
    ref = torch.einsum("thk,tkv->thv", scores.softmax(-1), sel[..., :512])
    diff = o.reshape(B * n, H, 512).float().cpu() - ref
    assert diff.norm() / ref.norm() < 0.006
    torch.testing.assert_close(lse.permute(0, 2, 1).reshape(B * n, H).cpu(), torch.logsumexp(scores, -1),
                               atol=1e-3, rtol=0)


def test_graph_capture_replays_match_eager(cuda):
    q, kv, idx = _case(4, 128, 2048, num_blocks=64, seed=5)
    out = torch.empty(4, 128, 512, dtype=torch.bfloat16, device=cuda)
    lse = torch.empty(4, 128, dtype=torch.float32, device=cuda)
    splits = 4
    ws = torch.empty(ops.sparse_mla_workspace_bytes(4, 128, splits), dtype=torch.uint8, device=cuda)
    ops.sparse_mla_decode(q, kv, idx, 0.1, out=out, lse=lse, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    eager_o, eager_l = out.clone(), lse.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.sparse_mla_decode(q, kv, idx, 0.1, out=out, lse=lse, num_splits=splits, workspace=ws)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_o) and torch.equal(lse, eager_l)


def test_schedule_keeps_workspaces_for_captured_graphs(cuda):
    """One schedule captured in HIP graphs at two batch sizes (both split the
    key list, so both use the workspace), then an eager call at a third size
    and other allocations; both graphs must still replay to their eager
    results (a freed workspace would be reused by the allocator)."""
    H, K, scale = 128, 2048, 192 ** -0.5
    sched, _ = flash_mla.get_mla_metadata()
    cases = {}
    for T in (2, 5):
        q, kv, idx = _case(T, H, K, num_blocks=80, seed=40 + T)
        assert ops.sparse_mla_num_splits(T, H, K, cuda) > 1
        args = (q.view(T, 1, H, 576), kv, None, None, 512, sched, None, scale)
        eager = [t.clone() for t in flash_mla.flash_mla_with_kvcache(*args, is_fp8_kvcache=True,
                                                                        indices=idx.view(T, 1, K))]
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            flash_mla.flash_mla_with_kvcache(*args, is_fp8_kvcache=True, indices=idx.view(T, 1, K))
            with torch.cuda.graph(g, stream=s):
                outs = flash_mla.flash_mla_with_kvcache(*args, is_fp8_kvcache=True, indices=idx.view(T, 1, K))
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        # the graph does not keep its inputs alive: hold them for the replays
        cases[T] = (g, outs, eager, (q, kv, idx))
    q3, kv3, idx3 = _case(3, H, K, num_blocks=80, seed=49)
    flash_mla.flash_mla_with_kvcache(q3.view(3, 1, H, 576), kv3, None, None, 512, sched, None, scale,
                                     is_fp8_kvcache=True, indices=idx3.view(3, 1, K))
    junk = [torch.full((1 << 20,), 7, dtype=torch.uint8, device=cuda) for _ in range(8)]
    torch.cuda.synchronize()
    for _ in range(2):
        for T, (g, outs, eager, _) in cases.items():
            for t in outs:
                t.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for a, b in zip(outs, eager):
                assert torch.equal(a, b), T
    del junk


def _query_error_bound_case(seed):
    """Queries whose 64-dim nope chunks each span ~24 binades (one anchor value
    and the rest spread down to 2^-24 of it, random signs), one valid key per
    query, so LSE = sm_scale * q.k with nothing else in it."""
    T, H, K = 4, 128, 64
    g = torch.Generator(device="cpu").manual_seed(seed)
    mag = torch.exp2(-24 * torch.rand(T, H, 512, generator=g))
    anchor = torch.exp2(torch.randint(-3, 7, (T, H, 8, 1), generator=g).float())
    nope = (mag.view(T, H, 8, 64) * anchor).view(T, H, 512)
    nope[..., ::64] = anchor[..., 0]                      # an exact power of two at each chunk's maximum
    nope *= torch.where(torch.rand(T, H, 512, generator=g) < 0.5, -1.0, 1.0)
    rope = torch.randn(T, H, 64, generator=g)
    q = torch.cat([nope, rope], -1).to(torch.bfloat16)
    kv = synth.make_mla_cache(4, seed=seed)
    idx = torch.full((T, K), -1, dtype=torch.int32)
    idx[:, 0] = torch.randperm(4 * 64, generator=g)[:T].to(torch.int32)
    return q, kv, idx


def test_qk_score_error_bound(cuda):
    """Bound on the score error of the QK product.

    The key's fp8 codes times their power-of-two tile scale are exact in bf16,
    the query enters as the caller's bf16, and the bf16 MFMA forms exact
    products summed in f32, so |s - s_exact| stays within f32 accumulation
    error: 2^-18 sum_d |q_d k_d| is a safe bound for 576 terms (plus f32
    rounding of the result). The query chunks span ~24 binades each, so any
    quantisation of the query to fp8 (one e4m3 term with a per-64-dim scale)
    breaks the bound by orders of magnitude; the scores are read from the LSE
    of a single valid key."""
    print("mla qk score bound", flush=True)
    q, kv, idx = _query_error_bound_case(seed=41)
    sm_scale = 1.0
    o, lse = ops.sparse_mla_decode(q.to(cuda), kv, idx.to(cuda), sm_scale)
    torch.cuda.synchronize()
    rows = O.dequant_mla_rows(kv.contiguous().reshape(-1, 656).cpu().numpy()).astype(np.float64)
    k = rows[idx[:, 0].numpy()]                                         # [T, 576]
    qf = q.float().numpy().astype(np.float64)                            # [T, H, 576]
    exact = np.einsum("thd,td->th", qf, k)
    got = lse.cpu().numpy().astype(np.float64) / sm_scale
    accum = np.einsum("thd,td->th", np.abs(qf), np.abs(k))
    bound = 2.0 ** -18 * accum + 2.0 ** -22 * np.abs(exact)
    err = np.abs(got - exact)
    assert np.all(err <= bound), f"worst err/bound {np.max(err / bound):.3g}"
    # the data defeats an fp8 query: one e4m3 term per value, scale 2^(ceil(log2 amax) - 8) per chunk
    x = qf[..., :512].reshape(*qf.shape[:2], 8, 64)
    s_hi = np.exp2(np.ceil(np.log2(np.abs(x).max(-1))) - 8)[..., None]
    hi = O.fp8_e4m3fn_decode(O.fp8_e4m3fn_encode(x / s_hi)) * s_hi
    err_hi = np.abs(np.einsum("thcd,tcd->th", hi - x, k[:, :512].reshape(-1, 8, 64)))
    assert np.median(err_hi / bound) > 100
