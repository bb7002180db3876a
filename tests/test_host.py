"""Host-side logic of the reference-mirroring Python layer (CPU only)."""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import indexer, ops


def test_expand_decode_context_lens_mirrors_reference():
    # tests/test_shared_indexer.py:162-181
    got = indexer._expand_decode_context_lens(torch.tensor([4098, 513], dtype=torch.int64), 2)
    assert got.dtype == torch.int32 and got.tolist() == [[4097, 4098], [512, 513]]
    assert indexer._expand_decode_context_lens(torch.tensor([1], dtype=torch.int32), 8).tolist() == [[1] * 8]
    with pytest.raises(ValueError, match="batch"):
        indexer._expand_decode_context_lens(torch.zeros(2, 3), 2)
    for n in (1, 2, 3):
        c = torch.randint(1, 5000, (7,))
        assert np.array_equal(indexer._expand_decode_context_lens(c, n).numpy(),
                              O.expand_decode_context_lens(c.numpy(), n))


def test_linear_mtp_path_rule():
    # tests/test_shared_indexer.py:184-187
    assert not indexer._uses_linear_mtp_indexer_path(is_prefill=True, ntps=22)
    assert not indexer._uses_linear_mtp_indexer_path(is_prefill=False, ntps=2)
    assert indexer._uses_linear_mtp_indexer_path(is_prefill=False, ntps=3)


def test_indexer_cache_layout_checks():
    c = indexer.IndexerCache(num_layers=2, num_pages=16, page_size=64, head_dim=128, device="cpu")
    assert c.bytes_per_token == 132 and c.get_buffer(1).shape == (16, 64 * 132)
    with pytest.raises(ValueError, match="uint8"):
        indexer.IndexerCache(1, 4, 64, 128, device="cpu", buffer=torch.zeros(1, 4, 10, dtype=torch.uint8))


def test_ops_reject_host_tensors_and_bad_shapes():
    s = torch.zeros(2, 128)
    lens = torch.zeros(2, dtype=torch.int32)
    out = torch.zeros(2, 512, dtype=torch.int32)
    with pytest.raises(ValueError, match="512 or 2048"):
        ops.topk_transform(s, lens, torch.zeros(2, 2, dtype=torch.int32), out, 64, 100)
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.topk_transform(s, lens, torch.zeros(2, 2, dtype=torch.int32), out, 64, 512)
    with pytest.raises(RuntimeError, match="seq_lens"):
        ops.topk_transform(s, lens.long(), torch.zeros(2, 2, dtype=torch.int32), out, 64, 512)
    with pytest.raises(RuntimeError, match="656"):
        ops.mla_kv_geometry(torch.zeros(4, 64, 1, 576, dtype=torch.uint8))
    kv = torch.zeros(4, 65, 1, 656, dtype=torch.uint8)[:, :64]
    assert ops.mla_kv_geometry(kv) == (65 * 656, 64)


def test_golden_fixture_reproduces_from_the_oracle():
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "config0_indexer.npz"))
    logits = O.indexer_logits(g["q_fp8"], g["cache"], g["weights"], g["context_lens"], g["block_tables"],
                              g["logits"].shape[1])
    np.testing.assert_array_equal(np.isfinite(logits), np.isfinite(g["logits"]))
    np.testing.assert_allclose(logits[np.isfinite(logits)], g["logits"][np.isfinite(g["logits"])], rtol=1e-6)
    page, raw = O.topk_transform(g["logits"], g["context_lens"].reshape(-1), g["block_tables"], 64, 2048)
    assert np.array_equal(raw, g["topk_raw"]) and np.array_equal(page, g["topk_page"])
    # the selected set agrees with torch.topk on every row
    for b, L in enumerate(g["context_lens"].reshape(-1)):
        k = min(int(L), 2048)
        ref = torch.topk(torch.from_numpy(g["logits"][b, :L]), k).indices.numpy()
        assert set(ref.tolist()) == set(raw[b, :k].tolist())


def test_prefill_chunk_rows_follow_the_logits_workspace(monkeypatch):
    """Chunk rows = the [rows, num_keys] f32 logits that fit in the call's
    workspace (a fixed fraction of the device's HBM), capped by query_chunk."""
    class Props:
        total_memory = 32 * 4 * 100_000 * 10      # a workspace of 10 rows of 100K keys
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda _i: Props())
    monkeypatch.setattr(indexer, "_HBM_BYTES", {})
    dev = torch.device("cuda", 0)
    assert indexer._prefill_chunk_rows(100, 100_000, dev) == 10
    assert indexer._prefill_chunk_rows(100, 100_000, dev, query_chunk=7) == 7
    assert indexer._prefill_chunk_rows(4, 100_000, dev) == 4
    assert indexer._prefill_chunk_rows(100, 10_000_000, dev) == 1   # never below one row
    with pytest.raises(ValueError, match="at least one key"):
        indexer._prefill_chunk_rows(10, 0, dev)


def test_gather_indexer_cache_argument_checks():
    from nanoengine_amd.indexer_cache_gather import gather_indexer_cache
    cache = torch.zeros(4, 64 * 132, dtype=torch.uint8)
    bt = torch.zeros(2, 3, dtype=torch.int32)
    with pytest.raises(ValueError, match="cu_seqlens_k and block_table batch dimensions differ"):
        gather_indexer_cache(cache, bt, torch.tensor([0, 5]), page_size=64, head_dim=128)
    with pytest.raises(ValueError, match="Indexer cache page has"):
        gather_indexer_cache(cache, bt, torch.tensor([0, 5, 9]), page_size=32, head_dim=128)
    with pytest.raises(ValueError, match="contiguous 2D uint8"):
        gather_indexer_cache(cache.float(), bt, torch.tensor([0, 5, 9]), page_size=64, head_dim=128)


def test_fused_step_rejects_non_indexer_page_size():
    """The fused indexer + top-k translates through the indexer's 64-token
    pages; another MLA block size must be refused, not silently mistranslated."""
    from nanoengine_amd.pipeline import DsaDecodeStep
    with pytest.raises(ValueError, match="page_size 64"):
        DsaDecodeStep(2, 1, 4096, page_size=32, device="cpu", fused=True)


def test_merge_attention_states_equals_one_softmax():
    """Two halves of one key set, each with its own softmax output and LSE,
    merged by LSE equal the softmax over all keys (mla_utils.py:12-23); an
    empty half (LSE -inf) leaves the other unchanged."""
    from nanoengine_amd import mla_utils
    g = torch.Generator().manual_seed(0)
    T, H, D, N = 3, 4, 16, 40
    s = torch.randn(T, H, N, generator=g, dtype=torch.float64) * 4
    v = torch.randn(T, N, D, generator=g, dtype=torch.float64)

    def part(sl):
        p = torch.softmax(s[..., sl], -1)
        return torch.einsum("thn,tnd->thd", p, v[:, sl]), torch.logsumexp(s[..., sl], -1).transpose(0, 1)

    lo, llse = part(slice(0, 13))
    hi, hlse = part(slice(13, N))
    full, flse = part(slice(0, N))
    merged, mlse = mla_utils.merge_attention_states(lo, llse, hi, hlse)
    assert torch.allclose(merged, full, atol=1e-12) and torch.allclose(mlse, flse, atol=1e-12)
    empty = torch.full_like(hlse, -float("inf"))
    same, slse = mla_utils.merge_attention_states(lo, llse, torch.zeros_like(hi), empty)
    assert torch.allclose(same, lo, atol=1e-12) and torch.equal(slse, llse)
