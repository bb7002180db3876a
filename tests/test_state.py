"""IndexerTopKState and the full/shared layer schedule on the CPU, after the
reference's tests/test_shared_indexer.py cases (GLM-5.2's 78-layer schedule,
reuse by identity, HiSparse mapping ownership, stale-shape rejection)."""
from types import SimpleNamespace

import pytest
import torch

from nanoengine_amd.state import IndexerTopKState, _get_indexer_mode, _IndexerTopKState

# GLM-5.2: layers 0-2 full, then every fourth layer from 6 on
GLM52 = ["full" if i < 3 or (i - 2) % 4 == 0 else "shared" for i in range(78)]


def test_explicit_schedule():
    cfg = SimpleNamespace(num_hidden_layers=78, index_topk=2048, indexer_types=GLM52)
    modes = [_get_indexer_mode(cfg, i) for i in range(78)]
    full = [i for i, m in enumerate(modes) if m == "full"]
    assert len(full) == 21 and modes.count("shared") == 57
    assert full == [0, 1, 2] + list(range(6, 78, 4))
    assert _get_indexer_mode(cfg, 78) == "full"           # the MTP layer always has its own indexer


def test_frequency_schedule_equals_explicit_schedule():
    cfg = SimpleNamespace(num_hidden_layers=78, index_topk=2048, index_topk_freq=4, index_skip_topk_offset=3)
    assert [_get_indexer_mode(cfg, i) for i in range(78)] == GLM52
    # defaults: every layer full; no index_topk: no indexer at all
    assert {_get_indexer_mode(SimpleNamespace(num_hidden_layers=5, index_topk=2048), i) for i in range(5)} == {"full"}
    assert _get_indexer_mode(SimpleNamespace(num_hidden_layers=5), 0) == "none"


def test_pattern_schedule_and_bad_schedules():
    cfg = SimpleNamespace(num_hidden_layers=4, index_topk=2048, index_topk_pattern="FsSf")
    assert [_get_indexer_mode(cfg, i) for i in range(4)] == ["full", "shared", "shared", "full"]
    with pytest.raises(ValueError, match="one entry per backbone layer"):
        _get_indexer_mode(SimpleNamespace(num_hidden_layers=2, index_topk=2048, indexer_types=["full"]), 0)
    with pytest.raises(ValueError, match="Unsupported indexer_types"):
        _get_indexer_mode(SimpleNamespace(num_hidden_layers=1, index_topk=2048, indexer_types=["dense"]), 0)
    with pytest.raises(ValueError, match="Unsupported index_topk_pattern"):
        _get_indexer_mode(SimpleNamespace(num_hidden_layers=2, index_topk=2048, index_topk_pattern="FX"), 1)


def test_shared_layer_gets_the_published_tensors_themselves():
    logical = torch.tensor([[7, 3], [11, 5]], dtype=torch.int32)
    physical = torch.tensor([[71, 31], [111, 51]], dtype=torch.int32)
    state = _IndexerTopKState()
    state.publish(2, logical, physical)
    got_l, got_p = state.require(layer_idx=3, num_tokens=2, topk=2, require_physical=True)
    assert got_l is logical and got_p is physical and state.source_layer == 2


def test_select_rows_copies_the_seed_rows():
    logical = torch.arange(24, dtype=torch.int32).reshape(6, 4)
    state = IndexerTopKState()
    state.publish(78, logical, logical + 100)
    state.publish_hisparse(78, logical + 200)
    sub = state.select_rows(torch.tensor([1, 4]))
    assert sub.source_layer == 78
    assert torch.equal(sub.logical_indices, logical[[1, 4]])
    assert torch.equal(sub.physical_indices, logical[[1, 4]] + 100)
    assert torch.equal(sub.hisparse_indices, logical[[1, 4]] + 200)
    assert sub.logical_indices.data_ptr() != logical.data_ptr()
    empty = IndexerTopKState().select_rows(torch.tensor([0]))
    assert empty.logical_indices is None and empty.source_layer is None


def test_hisparse_mapping_belongs_to_its_layer():
    logical = torch.tensor([[7, 3]], dtype=torch.int32)
    state = IndexerTopKState()
    state.publish(78, logical, logical + 10)
    hot = logical + 20
    state.publish_hisparse(78, hot)
    assert state.require_hisparse(78, num_tokens=1, topk=2) is hot
    assert state.require_hisparse(79, num_tokens=1, topk=2) is None
    assert state.require_hisparse(78, num_tokens=2, topk=2) is None
    with pytest.raises(RuntimeError, match="Cannot publish HiSparse mapping for layer 5"):
        state.publish_hisparse(5, hot)
    state.publish(78, logical + 1, logical + 11)          # a new selection drops the old mapping
    assert state.hisparse_indices is None


def test_missing_or_stale_topk_is_refused():
    state = IndexerTopKState()
    with pytest.raises(RuntimeError, match="no TopK"):
        state.require(3, num_tokens=2, topk=2, require_physical=False)
    state.publish(2, torch.zeros((1, 2), dtype=torch.int32))
    with pytest.raises(RuntimeError, match="stale TopK shape"):
        state.require(3, num_tokens=2, topk=2, require_physical=False)
    with pytest.raises(RuntimeError, match="invalid physical TopK"):
        state.require(3, num_tokens=1, topk=2, require_physical=True)
    logical, physical = state.require(3, num_tokens=1, topk=2, require_physical=False)
    assert physical is None and tuple(logical.shape) == (1, 2)
