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


def test_full_shared_full_layers_keep_each_output(cuda):
    """Layers 0 (full), 1 (shared) and 2 (full) of one step. Layers 0 and 2
    run through step object A with their own out=/lse= tensors; layer 1
    runs through a second object B over A's published pair. After layer 2,
    every layer's output still equals sparse MLA over the selection it used
    (layer 0's pair for layers 0 and 1, layer 2's own for layer 2), and the
    state has moved on to layer 2's pair."""
    from nanoengine_amd import ops
    from nanoengine_amd.state import IndexerTopKState
    lens, n, H = [3000, 20000, 700, 9000], 1, 128
    inp, kv, q, max_ctx = _step_inputs(lens, n, H, seed=31)
    B = len(lens)
    A = DsaDecodeStep(B, n, max_ctx, num_heads=H, device=cuda)
    Bs = DsaDecodeStep(B, n, max_ctx, num_heads=H, device=cuda)
    state = IndexerTopKState()
    seq = A.expand_lens(inp.context_lens)
    layers = []
    for i in range(3):
        layers.append((synth.make_mla_query(B * n, H, seed=100 + i, device="cuda"),
                       synth.make_mla_cache(kv.shape[0], seed=100 + i, device="cuda")))
    outs = [(torch.empty(B * n, H, 512, dtype=torch.bfloat16, device=cuda),
             torch.empty(B * n, H, dtype=torch.float32, device=cuda)) for _ in range(3)]
    # layer 2's indexer sees another query, so it selects differently
    q_idx2 = synth.make_indexer_inputs(lens, next_n=n, seed=32, device=cuda).q_fp8
    _, _, lg0, ph0 = A(inp.q_fp8, inp.weights, inp.cache, seq, inp.block_tables, inp.block_tables, *layers[0],
                       192 ** -0.5, layer_idx=0, indexer_state=state, out=outs[0][0], lse=outs[0][1])
    sel0 = ph0.clone()
    o1, l1, _, ph1 = Bs(None, None, None, None, None, None, *layers[1], 192 ** -0.5, layer_idx=1,
                        indexer_state=state, shared=True, out=outs[1][0], lse=outs[1][1])
    assert o1 is outs[1][0] and l1 is outs[1][1] and ph1 is ph0
    A(q_idx2, inp.weights, inp.cache, seq, inp.block_tables, inp.block_tables, *layers[2], 192 ** -0.5,
      layer_idx=2, indexer_state=state, out=outs[2][0], lse=outs[2][1])
    sel2 = A.physical.clone()
    torch.cuda.synchronize()
    assert not torch.equal(sel0, sel2), "layer 2 should select other slots"
    assert state.source_layer == 2 and state.physical_indices is A.physical
    for i, sel in ((0, sel0), (1, sel0), (2, sel2)):
        eo, el = ops.sparse_mla_decode(layers[i][0], layers[i][1], sel, 192 ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(outs[i][0], eo) and torch.equal(outs[i][1], el), f"layer {i}"
