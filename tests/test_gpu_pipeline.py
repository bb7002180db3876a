"""The whole decode step (DsaDecodeStep) on the GPU.

- The fused step (indexer + top-k without logits) and the two-operator step
  give bit-identical indices and therefore bit-identical attention outputs.
- The fused step captured in a HIP graph replays to the eager result, replay
  after replay, with other eager work in between (the lists and flags are reset
  by the kernels themselves, not by memsets).
- MTP verify rows (next_n = 2, BASELINE config 3 shape at reduced batch) run
  through the same step."""
import numpy as np
import pytest
import torch

from nanoengine_amd import synth
from nanoengine_amd.pipeline import DsaDecodeStep

pytestmark = pytest.mark.gpu


def _step_inputs(lens, n, H, seed):
    inp = synth.make_indexer_inputs(lens, next_n=n, seed=seed, device="cuda")
    num_blocks = int(inp.block_tables.max().item()) + 1
    kv = synth.make_mla_cache(num_blocks, seed=seed, device="cuda")
    B = len(lens)
    q = synth.make_mla_query(B * n, H, seed=seed, device="cuda")
    max_ctx = inp.block_tables.shape[1] * 64
    return inp, kv, q, max_ctx


def _run(step, inp, kv, q, n):
    seq = step.expand_lens(inp.context_lens)
    pt = inp.block_tables.repeat_interleave(n, dim=0).contiguous()
    return step(inp.q_fp8, inp.weights, inp.cache, seq, inp.block_tables, pt, q, kv, 192 ** -0.5)


@pytest.mark.parametrize("lens,n", [([4096, 70000, 1500, 30000], 1), ([20000, 3000, 65536], 2)])
def test_fused_step_equals_two_operator_step(cuda, lens, n):
    H = 64
    inp, kv, q, max_ctx = _step_inputs(lens, n, H, seed=len(lens) + n)
    B = len(lens)
    outs = []
    for fused in (True, False):
        step = DsaDecodeStep(B, n, max_ctx, num_heads=H, device=cuda, fused=fused)
        o, lse, logical, physical = _run(step, inp, kv, q, n)
        torch.cuda.synchronize()
        outs.append([t.clone() for t in (o, lse, logical, physical)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_graph_capture_of_the_fused_step(cuda):
    lens, n, H = [9000, 65536, 2048, 40000], 1, 128
    inp, kv, q, max_ctx = _step_inputs(lens, n, H, seed=11)
    step = DsaDecodeStep(len(lens), n, max_ctx, num_heads=H, device=cuda)
    eager = [t.clone() for t in _run(step, inp, kv, q, n)]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _run(step, inp, kv, q, n)  # warm-up on the capture stream
        with torch.cuda.graph(g, stream=s):
            outs = _run(step, inp, kv, q, n)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for _ in range(3):
        for t in outs:
            t.zero_()
        step.fused_workspace[:64].fill_(0xAB)  # stale list headers must not matter
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b)
