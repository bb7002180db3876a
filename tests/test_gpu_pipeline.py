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


def test_shared_layer_reuses_the_published_topk(cuda):
    """A full layer publishes its (logical, physical) pair; the next shared
    layer runs no indexer (its indexer inputs are None) and attends over
    exactly those slots: its output is bit-identical to sparse MLA over the
    published physical indices with the shared layer's own query and cache."""
    from nanoengine_amd import ops
    from nanoengine_amd.state import IndexerTopKState
    lens, n, H = [5000, 65536, 1200, 30000], 1, 128
    inp, kv, q, max_ctx = _step_inputs(lens, n, H, seed=23)
    step = DsaDecodeStep(len(lens), n, max_ctx, num_heads=H, device=cuda)
    state = IndexerTopKState()
    seq = step.expand_lens(inp.context_lens)
    pt = inp.block_tables.repeat_interleave(n, dim=0).contiguous()
    _, _, logical, physical = step(inp.q_fp8, inp.weights, inp.cache, seq, inp.block_tables, pt, q, kv,
                                   192 ** -0.5, layer_idx=2, indexer_state=state)
    published = (logical.clone(), physical.clone())
    assert state.source_layer == 2 and state.logical_indices is logical
    kv3 = synth.make_mla_cache(kv.shape[0], seed=99, device="cuda")
    q3 = synth.make_mla_query(len(lens) * n, H, seed=99, device="cuda")
    o, lse, l3, p3 = step(None, None, None, None, None, None, q3, kv3, 192 ** -0.5, layer_idx=3,
                          indexer_state=state, shared=True)
    o, lse = o.clone(), lse.clone()
    eo, else_ = ops.sparse_mla_decode(q3, kv3, published[1], 192 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(l3, published[0]) and torch.equal(p3, published[1])
    assert torch.equal(o, eo) and torch.equal(lse, else_)
    # a shared layer with nothing published, or at another batch shape, is refused
    with pytest.raises(RuntimeError, match="no TopK"):
        step(None, None, None, None, None, None, q3, kv3, 0.1, layer_idx=3, indexer_state=IndexerTopKState(),
             shared=True)
    small = IndexerTopKState()
    small.publish(2, published[0][:2], published[1][:2])
    with pytest.raises(RuntimeError, match="stale TopK shape"):
        step(None, None, None, None, None, None, q3, kv3, 0.1, layer_idx=3, indexer_state=small, shared=True)
