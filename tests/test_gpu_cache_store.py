"""fp8 cache writers on the GPU vs the oracle (bit-exact), and the MLA backend
end to end: store through forward(), then sparse decode through the
reference-shaped backend call."""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import indexer, mla_backend, ops

pytestmark = pytest.mark.gpu


def _bf16(rng, shape, scale=1.0):
    return torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_mla_kv_store_bit_exact(cuda, slot_dtype):
    rng = np.random.default_rng(11)
    kv = _bf16(rng, (40, 1, 576))
    kv[3] *= 1e-3
    kv[4] *= 300.0
    slots = torch.tensor(list(range(0, 60, 3)) + [-1] + list(range(64, 64 + 19 * 7, 7)), dtype=slot_dtype)
    assert slots.numel() == 40
    padded = torch.zeros(3, 65, 1, 656, dtype=torch.uint8, device=cuda)
    cache = padded[:, :64]
    ops.mla_kv_store(kv.to(cuda), cache, slots.to(cuda))
    torch.cuda.synchronize()
    exp = O.quantize_mla_rows(kv.float().reshape(40, 576).numpy())
    flat = cache.contiguous().reshape(-1, 656).cpu().numpy()
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            assert np.array_equal(flat[s], exp[i]), i
    assert torch.all(padded[:, 64] == 0)   # the padding row is never written
    assert int((flat != 0).any(1).sum()) == 39


def test_indexer_k_store_bit_exact(cuda):
    rng = np.random.default_rng(12)
    keys = _bf16(rng, (70, 128))
    keys[0] = 0
    slots = torch.tensor(rng.permutation(3 * 64)[:70], dtype=torch.int32)
    cache = indexer.IndexerCache(1, 3, 64, 128, device=cuda)
    cache.store_key_fp8(0, keys.to(cuda), slots.to(cuda))
    torch.cuda.synchronize()
    codes, sf = O.quantize_rows_ue8m0(keys.float().numpy())
    exp = O.pack_indexer_cache(codes, sf, slots.numpy(), 3)
    assert np.array_equal(cache.get_buffer(0).cpu().numpy(), exp)


def test_backend_forward_stores_and_decodes(cuda):
    rng = np.random.default_rng(13)
    B, H, K, blocks = 3, 128, 256, 8
    layer = mla_backend.create_mla(hardware_backend="mi355x", num_heads=H, head_dim=576, scale=192 ** -0.5,
                                   num_kv_heads=1, v_head_dim=512, nsa_index_topk=K)
    layer.k_cache = torch.zeros(blocks, 65, 1, 656, dtype=torch.uint8, device=cuda)[:, :64]
    # history rows, then the new tokens through forward()
    hist = _bf16(rng, (blocks * 64, 576)).to(cuda)
    ops.mla_kv_store(hist, layer.k_cache, torch.arange(blocks * 64, dtype=torch.int32, device=cuda))
    new_k = _bf16(rng, (B, 1, 576)).to(cuda)
    slots = torch.tensor([5, 70, 300], dtype=torch.int32, device=cuda)
    mla_backend.set_batch_context(is_prefill=False, slot_mapping=slots, num_tokens_per_seq=1)
    try:
        q = _bf16(rng, (B, H, 576)).to(cuda)
        idx = torch.stack([torch.randperm(blocks * 64)[:K] for _ in range(B)]).to(torch.int32).to(cuda)
        idx[:, 0] = slots
        o = layer(q, new_k, None, sparse_indices=idx)
        torch.cuda.synchronize()
        rows = layer.k_cache.contiguous().reshape(-1, 656).cpu().numpy()
        assert np.array_equal(rows[slots.cpu().numpy()], O.quantize_mla_rows(new_k.float().reshape(B, 576).cpu().numpy()))
        eo, _ = O.sparse_mla_decode(q.float().cpu().numpy(), rows, idx.cpu().numpy(), 192 ** -0.5)
        assert o.shape == (B, H, 512)
        assert np.abs(o.float().cpu().numpy() - eo).max() <= 2e-2
        # no indices (graph-capture warm-up): all -1 -> zeros
        o0 = layer(q, None, None, sparse_indices=None, write_kv_cache=False)
        torch.cuda.synchronize()
        assert torch.all(o0 == 0)
        with pytest.raises(RuntimeError, match="decode only"):
            mla_backend.set_batch_context(is_prefill=True)
            layer(q, None, None, sparse_indices=idx, write_kv_cache=False)
    finally:
        mla_backend.reset_batch_context()
