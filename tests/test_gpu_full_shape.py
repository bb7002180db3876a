"""The decode step at the BASELINE shapes, checked against the CPU oracle.

Config 2 at its own shape: the fused decode step over B=128 sequences of 64K
context (top-2048, 128 MLA heads), exactly as bench.py builds
it, with 12 rows spread over the batch (and therefore over the persistent
filter's contiguous per-wave page ranges and the XCDs) checked against the CPU
oracle: logits within 1e-3 relative, logical top-2048 bit-exact against the
exact selection over the GPU logits (and tie-only differences against the
oracle's float64 logits), physical slots bit-exact, MLA o within atol 2e-2 and
LSE within 1e-3.

Config 0 (B=4, 1K-4K tokens) runs the same step with every row checked, for
seeds 0, 1 and 2; configs 1 and 3 are checked at their own shapes too."""
import numpy as np
import pytest
import torch

from oracle import step_check as SC
from nanoengine_amd import ops, synth
from nanoengine_amd.pipeline import DsaDecodeStep

pytestmark = pytest.mark.gpu


def test_config2_full_step_sampled_rows_match_oracle(cuda):
    B, L, H, K, seed = 128, 65536, 128, 2048, 0
    print(f"config2 B={B} L={L} H={H} K={K} seed={seed}", flush=True)
    lens = [L] * B
    inp = synth.make_indexer_inputs(lens, next_n=1, seed=seed, device=cuda)
    kv = synth.make_mla_cache(int(inp.block_tables.max().item()) + 1, seed=seed, device=cuda)
    q_mla = synth.make_mla_query(B, H, seed=seed, device=cuda)
    max_ctx = inp.block_tables.shape[1] * 64
    step = DsaDecodeStep(B, 1, max_ctx, num_heads=H, index_topk=K, device=cuda)
    seq = step.expand_lens(inp.context_lens)
    o, lse, logical, physical = step(inp.q_fp8, inp.weights, inp.cache, seq, inp.block_tables, inp.block_tables,
                                     q_mla, kv, 192 ** -0.5)
    logits = ops.indexer_logits(inp.q_fp8.view(B, 1, 64, 128), inp.cache, inp.weights, seq.view(B, 1),
                                inp.block_tables, max_ctx)
    torch.cuda.synchronize()
    rows = SC.spread_rows(B, 12)
    data = SC.sample_from_device(rows, q_idx_fp8=inp.q_fp8, weights=inp.weights, cache=inp.cache, lens=lens,
                                 block_tables=inp.block_tables, q_mla=q_mla, kv=kv, logits=logits,
                                 logical=logical, physical=physical, o=o, lse=lse)
    rep = SC.check_step_rows(**data, sm_scale=192 ** -0.5, topk=K)
    print(rep, flush=True)
    assert rep["ok"], rep
    # every row of the batch selected exactly K distinct in-range positions
    lg = logical.cpu().numpy()
    assert np.all((lg >= 0) & (lg < L))
    assert np.all(np.diff(lg, axis=1) > 0)


def test_config3_mtp_step_sampled_rows_match_oracle(cuda):
    """BASELINE config 3 at its own shape: MTP verify with next_n = 2 over 64
    sequences of lognormal length (median 16K, clipped to 2K-128K), built as
    bench.py --config 3 builds it. Each query token has its own causal length
    (ctx - 1 for the first draft position); 12 query rows spread over the batch
    are checked against the oracle to the same bounds as config 2."""
    B, n, H, K, seed = 64, 2, 128, 2048, 0
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in np.clip(np.exp(rng.normal(np.log(16384), 1.0, B)), 2048, 131072)]
    print(f"config3 B={B} n={n} H={H} K={K} seed={seed} max_len={max(lens)}", flush=True)
    inp = synth.make_indexer_inputs(lens, next_n=n, seed=seed, device=cuda)
    kv = synth.make_mla_cache(int(inp.block_tables.max().item()) + 1, seed=seed, device=cuda)
    q_mla = synth.make_mla_query(B * n, H, seed=seed, device=cuda)
    max_ctx = inp.block_tables.shape[1] * 64
    step = DsaDecodeStep(B, n, max_ctx, num_heads=H, index_topk=K, device=cuda)
    seq = step.expand_lens(inp.context_lens)
    pt = inp.block_tables.repeat_interleave(n, dim=0).contiguous()
    o, lse, logical, physical = step(inp.q_fp8, inp.weights, inp.cache, seq, inp.block_tables, pt, q_mla, kv,
                                     192 ** -0.5)
    logits = ops.indexer_logits(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, seq.view(B, n),
                                inp.block_tables, max_ctx)
    torch.cuda.synchronize()
    rows = SC.spread_rows(B * n, 12)
    qlens = seq.cpu().numpy()
    data = SC.sample_from_device(rows, q_idx_fp8=inp.q_fp8, weights=inp.weights, cache=inp.cache, lens=qlens,
                                 block_tables=inp.block_tables, q_mla=q_mla, kv=kv, logits=logits,
                                 logical=logical, physical=physical, o=o, lse=lse, next_n=n)
    rep = SC.check_step_rows(**data, sm_scale=192 ** -0.5, topk=K)
    print(rep, flush=True)
    assert rep["ok"], rep
    # the first draft position sees one key fewer than the second
    assert np.all(qlens.reshape(B, n)[:, 0] == qlens.reshape(B, n)[:, 1] - 1)


def test_config1_mla_alone_sampled_tokens_match_oracle(cuda):
    """BASELINE config 1 at its own shape: sparse MLA decode alone, B=32 x 32K
    context, 128 heads, top-2048 random positions through random block tables,
    with the split count the library picks (key splits + LSE combine). Eight
    tokens are checked against the oracle (o atol 2e-2, LSE 1e-3)."""
    import oracle as O
    from nanoengine_amd import mla_utils
    B, L, H, K, seed = 32, 32768, 128, 2048, 0
    print(f"config1 B={B} L={L} H={H} K={K} seed={seed}", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(seed)
    bt, num_pages = synth.make_block_tables([L] * B, gen, cuda)
    kv = synth.make_mla_cache(num_pages, seed=seed, device=cuda)
    q = synth.make_mla_query(B, H, seed=seed, device=cuda)
    pos = synth.random_topk_positions([L] * B, K, seed=seed, device=cuda)
    idx = mla_utils.topk_indices_to_physical(pos, bt, 64)
    splits = ops.sparse_mla_num_splits(B, H, K, cuda)
    assert splits > 1
    o, lse = ops.sparse_mla_decode(q, kv, idx, 192 ** -0.5, num_splits=splits)
    torch.cuda.synchronize()
    rows = SC.spread_rows(B, 8)
    for r in rows.tolist():
        sel = idx[r].long()
        kv_sel = kv[sel // 64, sel % 64, 0].cpu().numpy()
        eo, el = O.sparse_mla_decode(q[r:r + 1].float().cpu().numpy(), kv_sel, np.arange(K)[None, :],
                                     192 ** -0.5)
        assert np.abs(o[r].float().cpu().numpy() - eo[0]).max() <= 2e-2
        assert np.abs(lse[r].cpu().numpy() - el[0]).max() <= 1e-3


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config0_full_step_every_row_matches_oracle(cuda, seed):
    """BASELINE config 0 through the fused decode step: B=4 sequences of 1024,
    2048, 3000 and 4096 tokens (two rows at or below 2048 keep every position,
    two go through the exact top-2048), 128 MLA heads, seeds 0, 1 and 2 as the
    measurement plan asks. Every row is checked against the oracle to the same
    bounds as config 2."""
    B, H, K = 4, 128, 2048
    lens = [1024, 2048, 3000, 4096]
    print(f"config0 B={B} lens={lens} H={H} K={K} seed={seed}", flush=True)
    inp = synth.make_indexer_inputs(lens, next_n=1, seed=seed, device=cuda)
    kv = synth.make_mla_cache(int(inp.block_tables.max().item()) + 1, seed=seed, device=cuda)
    q_mla = synth.make_mla_query(B, H, seed=seed, device=cuda)
    max_ctx = inp.block_tables.shape[1] * 64
    step = DsaDecodeStep(B, 1, max_ctx, num_heads=H, index_topk=K, device=cuda)
    seq = step.expand_lens(inp.context_lens)
    o, lse, logical, physical = step(inp.q_fp8, inp.weights, inp.cache, seq, inp.block_tables, inp.block_tables,
                                     q_mla, kv, 192 ** -0.5)
    logits = ops.indexer_logits(inp.q_fp8.view(B, 1, 64, 128), inp.cache, inp.weights, seq.view(B, 1),
                                inp.block_tables, max_ctx)
    torch.cuda.synchronize()
    rows = np.arange(B)
    data = SC.sample_from_device(rows, q_idx_fp8=inp.q_fp8, weights=inp.weights, cache=inp.cache, lens=lens,
                                 block_tables=inp.block_tables, q_mla=q_mla, kv=kv, logits=logits,
                                 logical=logical, physical=physical, o=o, lse=lse)
    rep = SC.check_step_rows(**data, sm_scale=192 ** -0.5, topk=K)
    print(rep, flush=True)
    assert rep["ok"], rep
    lg = logical.cpu().numpy()
    for r, L in enumerate(lens):
        if L <= K:
            # a row no longer than k keeps every position, in order, then -1
            assert np.array_equal(lg[r, :L], np.arange(L)) and np.all(lg[r, L:] == -1)
        else:
            assert np.all((lg[r] >= 0) & (lg[r] < L)) and len(np.unique(lg[r])) == K
