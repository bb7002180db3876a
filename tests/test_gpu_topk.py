"""Top-k selection + page translation on the GPU vs the CPU oracle and torch.topk.

Cases follow the reference's tests/test_topk_transform.py (set equality with
torch.topk, -1 padding for short rows, ragged rows with offsets, all-equal
scores staying unique and in range) plus exactness at 64K+ contexts, where the
reference's fused kernel is not used.
"""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import deepseek_v4, ops

pytestmark = pytest.mark.gpu


def _run(scores, lens, page_tables, page_size, top_k):
    """Both selection routes (sampled candidate list, and the full multi-pass
    select used without a workspace) must give the same exact answer."""
    B = scores.shape[0]
    res = []
    for ws in (None, False):
        out = torch.full((B, top_k), 7, dtype=torch.int32, device=scores.device)
        raw = torch.full_like(out, 7)
        ops.topk_transform(scores, lens, page_tables, out, page_size, top_k, raw, workspace=ws)
        torch.cuda.synchronize()
        res.append((out.cpu().numpy(), raw.cpu().numpy()))
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1])
    return res[0]


@pytest.mark.parametrize("top_k", [512, 2048])
def test_matches_torch_topk_reference_case(cuda, top_k):
    # tests/test_topk_transform.py:10-65 of the reference, same shapes and seed
    torch.manual_seed(0)
    page_size, max_ctx = 64, 16384
    lens = torch.tensor([min(64, top_k), max_ctx], dtype=torch.int32, device=cuda)
    scores = torch.randn(2, max_ctx, dtype=torch.float32, device=cuda)
    pt = torch.arange(max_ctx // page_size, dtype=torch.int32, device=cuda).repeat(2, 1)
    out, raw = _run(scores, lens, pt, page_size, top_k)
    for row in range(2):
        L = int(lens[row])
        k = min(L, top_k)
        exp_raw = torch.topk(scores[row, :L], k).indices.cpu()
        exp = (pt[row].cpu()[exp_raw // page_size] * page_size + exp_raw % page_size).numpy()
        assert np.array_equal(np.sort(out[row, :k]), np.sort(exp))
        assert np.array_equal(np.sort(raw[row, :k]), np.sort(exp_raw.numpy()))
        assert (out[row, k:] == -1).all() and (raw[row, k:] == -1).all()


@pytest.mark.parametrize("lens", [[1024, 2048, 3000, 4096], [65536, 70000, 2049, 131072]])
@pytest.mark.parametrize("page_size", [64, 16])
def test_exact_vs_oracle_permuted_tables(cuda, lens, page_size):
    rng = np.random.default_rng(sum(lens) + page_size)
    B, width = len(lens), max(lens)
    scores = rng.standard_normal((B, width)).astype(np.float32)
    pages = (width + page_size - 1) // page_size
    pt = np.stack([rng.permutation(pages * B)[:pages] for _ in range(B)]).astype(np.int32)
    out, raw = _run(torch.from_numpy(scores).to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda),
                    torch.from_numpy(pt).to(cuda), page_size, 2048)
    e_page, e_raw = O.topk_transform(scores, np.array(lens), pt, page_size, 2048)
    assert np.array_equal(raw, e_raw)
    assert np.array_equal(out, e_page)


def test_ties_and_duplicates_are_exact(cuda):
    # heavy ties force the position digits: lowest positions win among equals
    rng = np.random.default_rng(5)
    L = 65536
    rows = [np.zeros(L, np.float32),                                   # all equal
            rng.integers(0, 4, L).astype(np.float32),                  # 4 distinct values
            np.repeat(rng.standard_normal(L // 64).astype(np.float32), 64),  # runs of 64 equal
            np.where(rng.random(L) < 0.5, np.float32(1.0), np.float32(-np.inf))]
    scores = np.stack(rows)
    lens = np.full(len(rows), L, np.int32)
    pt = np.tile(np.arange(L // 64, dtype=np.int32), (len(rows), 1))
    out, raw = _run(torch.from_numpy(scores).to(cuda), torch.from_numpy(lens).to(cuda),
                    torch.from_numpy(pt).to(cuda), 64, 2048)
    e_page, e_raw = O.topk_transform(scores, lens, pt, 64, 2048)
    assert np.array_equal(raw, e_raw)
    assert np.array_equal(out, e_page)
    assert np.array_equal(raw[0], np.arange(2048))


def test_nan_ranks_lowest_and_specials(cuda):
    rng = np.random.default_rng(9)
    L = 10000
    x = rng.standard_normal(L).astype(np.float32)
    x[rng.choice(L, 3000, replace=False)] = np.nan
    x[:5] = np.inf
    x[5:10] = -0.0
    x[10:15] = 0.0
    x[15:20] = np.float32(1e38)
    scores = x[None, :]
    pt = np.arange((L + 63) // 64, dtype=np.int32)[None, :]
    out, raw = _run(torch.from_numpy(scores).to(cuda), torch.tensor([L], dtype=torch.int32, device=cuda),
                    torch.from_numpy(pt).to(cuda), 64, 2048)
    e_page, e_raw = O.topk_transform(scores, np.array([L]), pt, 64, 2048)
    assert np.array_equal(raw, e_raw)


def test_short_rows_emit_positions_in_order(cuda):
    lens = [0, 1, 63, 2048]
    width = 4096
    scores = torch.randn(4, width, device=cuda)
    pt = torch.arange(width // 64, dtype=torch.int32, device=cuda).flip(0).repeat(4, 1).contiguous()
    out, raw = _run(scores, torch.tensor(lens, dtype=torch.int32, device=cuda), pt, 64, 2048)
    e_page, e_raw = O.topk_transform(scores.cpu().numpy(), np.array(lens), pt.cpu().numpy(), 64, 2048)
    assert np.array_equal(raw, e_raw) and np.array_equal(out, e_page)


def test_ragged_long_multiseq_ranges_exact(cuda):
    # reference tests/test_topk_transform.py:68-98 (there: <= 5 differences allowed)
    torch.manual_seed(7)
    width = 70_000
    lens = torch.tensor([17, 4096, 65_536], dtype=torch.int32, device=cuda)
    starts = torch.tensor([9, 123, 1000], dtype=torch.int32, device=cuda)
    offs = torch.tensor([0, 17, 4113], dtype=torch.int32, device=cuda)
    scores = torch.randn(3, width, dtype=torch.float32, device=cuda)
    out = torch.empty(3, 2048, dtype=torch.int32, device=cuda)
    deepseek_v4.topk_transform_ragged(scores, lens, starts, offs, out, 2048)
    torch.cuda.synchronize()
    exp = O.topk_transform_ragged(scores.cpu().numpy(), lens.cpu().numpy(), starts.cpu().numpy(),
                                  offs.cpu().numpy(), 2048)
    assert np.array_equal(out.cpu().numpy(), exp)
    assert torch.equal(out[0, :17].sort().values.cpu(), torch.arange(17, dtype=torch.int32))
    for row in (1, 2):
        L, s, o = int(lens[row]), int(starts[row]), int(offs[row])
        ref = set(torch.topk(scores[row, s:s + L], 2048).indices.cpu().tolist())
        assert ref == set((out[row] - o).cpu().tolist())


def test_ragged_ties_unique_and_in_range(cuda):
    # reference tests/test_topk_transform.py:101-121
    length, start, off = 65_536, 321, 777
    scores = torch.zeros(1, 70_000, dtype=torch.float32, device=cuda)
    out = torch.empty(1, 2048, dtype=torch.int32, device=cuda)
    deepseek_v4.topk_transform_ragged(scores, torch.tensor([length], dtype=torch.int32, device=cuda),
                                      torch.tensor([start], dtype=torch.int32, device=cuda),
                                      torch.tensor([off], dtype=torch.int32, device=cuda), out, 2048)
    torch.cuda.synchronize()
    sel = out[0].cpu()
    assert int(sel.min()) >= off and int(sel.max()) < off + length
    assert torch.unique(sel).numel() == 2048
    assert torch.equal(sel, torch.arange(off, off + 2048, dtype=torch.int32))


def test_raw_positions_without_translation(cuda):
    rng = np.random.default_rng(3)
    scores = rng.standard_normal((3, 9000)).astype(np.float32)
    lens = np.array([9000, 5000, 100], np.int32)
    out = torch.empty(3, 512, dtype=torch.int32, device=cuda)
    ops.topk_transform_raw(torch.from_numpy(scores).to(cuda), torch.from_numpy(lens).to(cuda), out, 512)
    torch.cuda.synchronize()
    for b in range(3):
        exp = np.full(512, -1, np.int32)
        sel = O.topk_select(scores[b], int(lens[b]), 512)
        exp[:sel.size] = sel
        assert np.array_equal(out[b].cpu().numpy(), exp)


def test_rejects_bad_arguments(cuda):
    s = torch.randn(2, 128, device=cuda)
    lens = torch.tensor([128, 128], dtype=torch.int32, device=cuda)
    pt = torch.zeros(2, 2, dtype=torch.int32, device=cuda)
    out = torch.empty(2, 512, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="top_k must be 512 or 2048"):
        deepseek_v4.topk_transform(s, lens, pt, out, 64, 1000)
    with pytest.raises(RuntimeError, match="power of 2"):
        deepseek_v4.topk_transform(s, lens, pt, out, 48, 512)
    with pytest.raises(ValueError, match="ragged Indexer top_k must be 2048"):
        deepseek_v4.topk_transform_ragged(s, lens, lens, lens, out, 512)


def test_sample_blind_spots_fall_back_exactly(cuda):
    """Rows of up to 64K positions take the one-launch path, whose threshold comes
    from a 1/8 sample of the row. Scores that put the whole top-k where the sample
    does not look (positions 1 mod 4), or that make every position a candidate
    (a constant row), must still give the exact answer through the fallback."""
    L = 65536
    rng = np.random.default_rng(7)
    base = rng.standard_normal(L).astype(np.float32)
    blind = base.copy()
    blind[1::4] += 100.0                 # 16384 large scores, none sampled
    const = np.full(L, 0.5, np.float32)  # every position ties
    ramp = np.arange(L, dtype=np.float32)  # scores rise with position
    scores = np.stack([blind, const, ramp, base])
    lens = np.array([L, L, L, 40000], np.int32)
    pt = np.stack([np.random.default_rng(i).permutation(L // 64).astype(np.int32) for i in range(4)])
    out, raw = _run(torch.from_numpy(scores).to(cuda), torch.from_numpy(lens).to(cuda),
                    torch.from_numpy(pt).to(cuda), 64, 2048)
    e_page, e_raw = O.topk_transform(scores, lens, pt, 64, 2048)
    assert np.array_equal(raw, e_raw)
    assert np.array_equal(out, e_page)


@pytest.mark.parametrize("width,k", [(9000, 2048), (70000, 2048), (9000, 512), (3000, 100)])
@pytest.mark.parametrize("with_ws", [True, False])
def test_indexer_select_masks_extreme_logits(cuda, width, k, with_ws):
    """The indexer's portable selection tail (lightning.py:1468-1492): +inf,
    NaN, |x| >= 1e30 rank as -inf; positions past the context are never
    selected; compared with the oracle's indexer_decode_topk. Rows: more
    extreme values than non-selected room (so -inf ties are selected), a row
    shorter than k, and ordinary rows. k=100 takes the torch route."""
    from nanoengine_amd import indexer as nidx
    rng = np.random.default_rng(width + k)
    R = 4
    logits = rng.standard_normal((R, width)).astype(np.float32)
    for r in range(R):
        hot = rng.choice(width, size=width // 3, replace=False)
        vals = np.array([np.inf, -np.inf, np.nan, 1e31, -1e31, 3e38, 1e30], np.float32)
        logits[r, hot] = vals[rng.integers(0, vals.size, hot.size)]
    logits[2, : width // 2] = np.inf      # the whole first half masked
    ctx = np.array([width, width - 37, width // 2 + 5, min(k - 1, width)], np.int32)
    if not with_ws and k not in (512, 2048):
        pytest.skip("the torch route takes no workspace")
    out = torch.empty(R, k, dtype=torch.int32, device=cuda)
    lg = torch.from_numpy(logits).to(cuda)
    cl = torch.from_numpy(ctx).to(cuda)
    if k in (512, 2048):
        ops.indexer_select(lg, cl, out, k, workspace=None if with_ws else False)
    else:
        nidx._select_other_k(lg, cl, k, out)
    torch.cuda.synchronize()
    exp = O.indexer_decode_topk(logits, ctx, k)
    assert np.array_equal(out.cpu().numpy(), exp)
