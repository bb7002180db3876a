"""Randomised shapes through the whole decode step, every row against the
CPU oracle (``oracle/step_check.py``: logits, exact top-k, physical slots,
MLA o and LSE).

Each case draws, from its own seed: 1-9 sequences, next_n 1 or 2, 16-128 MLA
heads, top-512 or top-2048, the fused or the two-operator indexer, and
lengths either on the edges the kernels branch on (1, 2, one page +-1, k +-1,
4096 +-1) or uniform up to 24K tokens."""
import numpy as np
import pytest
import torch

from oracle import step_check as SC
from nanoengine_amd import ops, synth
from nanoengine_amd.pipeline import DsaDecodeStep

pytestmark = pytest.mark.gpu

EDGES = [1, 2, 63, 64, 65, 511, 512, 513, 2047, 2048, 2049, 4095, 4096, 4097]


@pytest.mark.parametrize("case", range(24))
def test_random_step_every_row_matches_oracle(cuda, case):
    rng = np.random.default_rng(1000 + case)
    B = int(rng.integers(1, 10))
    n = int(rng.choice([1, 2]))
    H = int(rng.choice([16, 32, 64, 96, 128]))
    K = int(rng.choice([512, 2048]))
    fused = bool(rng.random() < 0.7)
    lens = [int(rng.choice(EDGES)) if rng.random() < 0.5 else int(rng.integers(n, 24000)) for _ in range(B)]
    lens = [max(L, n) for L in lens]
    print(f"step sweep case {case}: B={B} n={n} H={H} K={K} fused={fused} lens={lens}", flush=True)
    inp = synth.make_indexer_inputs(lens, next_n=n, seed=case, device=cuda)
    kv = synth.make_mla_cache(int(inp.block_tables.max().item()) + 1, seed=case, device=cuda)
    q_mla = synth.make_mla_query(B * n, H, seed=case, device=cuda)
    max_ctx = inp.block_tables.shape[1] * 64
    step = DsaDecodeStep(B, n, max_ctx, num_heads=H, index_topk=K, device=cuda, fused=fused)
    seq = step.expand_lens(inp.context_lens)
    pt = inp.block_tables.repeat_interleave(n, dim=0).contiguous()
    o, lse, logical, physical = step(inp.q_fp8, inp.weights, inp.cache, seq, inp.block_tables, pt, q_mla, kv,
                                     192 ** -0.5)
    logits = ops.indexer_logits(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, seq.view(B, n),
                                inp.block_tables, max_ctx)
    torch.cuda.synchronize()
    data = SC.sample_from_device(np.arange(B * n), q_idx_fp8=inp.q_fp8, weights=inp.weights, cache=inp.cache,
                                 lens=seq.cpu().numpy(), block_tables=inp.block_tables, q_mla=q_mla, kv=kv,
                                 logits=logits, logical=logical, physical=physical, o=o, lse=lse, next_n=n)
    rep = SC.check_step_rows(**data, sm_scale=192 ** -0.5, topk=K)
    print(rep, flush=True)
    assert rep["ok"], rep
