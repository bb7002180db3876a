"""Fused indexer + top-k (dsa_indexer_topk) on the GPU.

The fused call must select exactly what topk_transform selects over the
logits of indexer_logits on the same inputs (same logits bit for bit, so the
comparison is exact), for plain decode, MTP rows (next_n = 2), short rows and
both top-k sizes, and also when the page sample misleads the threshold and the
list select has to redo a row from its full logits."""
import numpy as np
import pytest
import torch

from nanoengine_amd import ops, synth

pytestmark = pytest.mark.gpu


def _inputs(lens, n, seed):
    inp = synth.make_indexer_inputs(lens, next_n=n, seed=seed, device="cuda")
    ctx = inp.context_lens.to(torch.int32)
    if n == 1:
        cl = ctx.view(-1, 1)
    else:  # causal lengths of the draft tokens: L - (n-1-j)
        offs = torch.arange(n - 1, -1, -1, dtype=torch.int32, device="cuda")
        cl = (ctx[:, None] - offs).clamp_min(1).contiguous()
    max_ctx = inp.block_tables.shape[1] * 64
    return inp, cl, max_ctx


def _unfused(inp, cl, max_ctx, k, n):
    B = cl.shape[0]
    logits = ops.indexer_logits(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, cl, inp.block_tables,
                                max_ctx)
    pt = inp.block_tables.repeat_interleave(n, dim=0).contiguous()
    phys = torch.empty(B * n, k, dtype=torch.int32, device="cuda")
    logi = torch.empty_like(phys)
    ops.topk_transform(logits, cl.reshape(-1).contiguous(), pt, phys, 64, k, logi)
    torch.cuda.synchronize()
    return phys.cpu().numpy(), logi.cpu().numpy()


def _fused(inp, cl, max_ctx, k, n):
    B = cl.shape[0]
    phys = torch.full((B * n, k), 7, dtype=torch.int32, device="cuda")
    logi = torch.full_like(phys, 7)
    ops.indexer_topk(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, cl, inp.block_tables, max_ctx, k,
                     phys, logi)
    torch.cuda.synchronize()
    return phys.cpu().numpy(), logi.cpu().numpy()


@pytest.mark.parametrize("lens,n,k", [
    ([1024, 2048, 3000, 4096], 1, 2048),
    ([65536, 40000, 100, 5000], 1, 2048),
    ([20000, 70000, 3000], 2, 2048),              # MTP verify rows
    ([9000, 5000, 300], 1, 512),
    ([262144, 3000], 1, 2048),                    # the longest row: its page table does not fit in LDS
])
def test_fused_matches_indexer_then_topk(cuda, lens, n, k):
    inp, cl, max_ctx = _inputs(lens, n, seed=sum(lens) + n + k)
    e_phys, e_logi = _unfused(inp, cl, max_ctx, k, n)
    g_phys, g_logi = _fused(inp, cl, max_ctx, k, n)
    assert np.array_equal(g_logi, e_logi)
    assert np.array_equal(g_phys, e_phys)


def test_misleading_sample_takes_the_repair_path(cuda):
    """Row 0: the sampled pages (every 32nd) score 16x higher, so the threshold
    lands above almost every other token and the list is too short. Row 1: the
    sampled pages score 16x lower, so nearly every token passes and the list
    overflows. Both rows must come out exact through the in-place repair."""
    lens = [65536, 65536, 30000]
    inp, cl, max_ctx = _inputs(lens, 1, seed=5)
    scales = inp.cache[:, 64 * 128:].view(torch.float32)  # [pages, 64] per-token key scales
    bt = inp.block_tables.cpu().numpy()
    for row, factor in ((0, 16.0), (1, 1.0 / 16.0)):
        pages = torch.from_numpy(bt[row, 0:1024:32].astype(np.int64)).to("cuda")
        scales[pages] *= factor
    e_phys, e_logi = _unfused(inp, cl, max_ctx, 2048, 1)
    g_phys, g_logi = _fused(inp, cl, max_ctx, 2048, 1)
    assert np.array_equal(g_logi, e_logi)
    assert np.array_equal(g_phys, e_phys)


def test_workspace_and_argument_checks(cuda):
    assert ops.indexer_topk_workspace_bytes(128, 1, 65536) > 128 * 65536 * 4
    inp, cl, max_ctx = _inputs([3000], 1, seed=1)
    out = torch.empty(1, 2048, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        ops.indexer_topk(inp.q_fp8.view(1, 1, 64, 128), inp.cache, inp.weights, cl, inp.block_tables, max_ctx,
                         1000, torch.empty(1, 1000, dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError, match="workspace"):
        ops.indexer_topk(inp.q_fp8.view(1, 1, 64, 128), inp.cache, inp.weights, cl, inp.block_tables, max_ctx,
                         2048, out, workspace=torch.empty(16, dtype=torch.uint8, device="cuda"))


def test_fused_batch_at_the_persistent_limit(cuda):
    """4096 entries, the largest batch the persistent filter pass takes: its
    LDS page prefix is at its largest (two workgroups per CU), and every
    wave's page range crosses several batch entries; the selection is still
    exactly topk_transform over indexer_logits."""
    B, L, k = 4096, 2100, 2048
    print(f"fused batch at the persistent limit B={B} L={L}", flush=True)
    inp, cl, max_ctx = _inputs([L - (i % 64) for i in range(B)], 1, seed=4096)
    e_phys, e_logi = _unfused(inp, cl, max_ctx, k, 1)
    g_phys, g_logi = _fused(inp, cl, max_ctx, k, 1)
    assert np.array_equal(g_logi, e_logi)
    assert np.array_equal(g_phys, e_phys)


def test_fused_large_batch_takes_the_per_workgroup_filter(cuda):
    """Batches above 4096 entries do not fit the persistent filter pass's LDS
    page prefix (two workgroups per CU) and take the one-workgroup-per-24-pages
    filter instead; the
    selection is still exactly topk_transform over indexer_logits."""
    B, L, k = 8200, 2100, 2048
    print(f"fused large batch B={B} L={L}", flush=True)
    inp, cl, max_ctx = _inputs([L] * B, 1, seed=8200)
    e_phys, e_logi = _unfused(inp, cl, max_ctx, k, 1)
    g_phys, g_logi = _fused(inp, cl, max_ctx, k, 1)
    assert np.array_equal(g_logi, e_logi)
    assert np.array_equal(g_phys, e_phys)


def test_fused_max_context_below_some_rows(cuda):
    """max_context_len = 6000 (not a page multiple) with rows of 7000 and 9000
    tokens: every stage clamps a row to max_context_len, as the unfused
    operators do (the logits stop at max_context_len)."""
    print("fused max_context below rows", flush=True)
    inp, cl, _ = _inputs([7000, 5000, 9000, 2500], 1, seed=6000)
    max_ctx, k = 6000, 2048
    e_phys, e_logi = _unfused(inp, cl, max_ctx, k, 1)
    g_phys, g_logi = _fused(inp, cl, max_ctx, k, 1)
    assert np.array_equal(g_logi, e_logi)
    assert np.array_equal(g_phys, e_phys)
