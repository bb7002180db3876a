"""Top-k selection shared by consecutive DSA attention layers.

Mirrors ``IndexerTopKState`` (dlengine/runtime/layers/backends/dsa/state.py:14-103)
and the layer schedule that decides which layers run their own indexer
(``_get_indexer_mode``, dlengine/runtime/models/deepseek_v2/deepseek_v2.py:84-129).
A "full" layer runs the indexer and publishes its (logical, physical) top-k; a
"shared" layer takes the published pair as is and runs only sparse MLA
(deepseek_v2.py:1865-1950). The field names, method signatures and error
messages are the interface the model and runners call and the reference's
tests match on.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


def _shape(t: torch.Tensor | None):
    return None if t is None else tuple(t.shape)


@dataclass
class IndexerTopKState:
    """The last full layer's top-k: logical positions [tokens, topk], their
    physical cache slots, an optional HiSparse hot mapping, and the layer that
    produced them. Tensors are held by reference, never copied, so a shared
    layer reads exactly what the full layer wrote."""

    logical_indices: torch.Tensor | None = None
    physical_indices: torch.Tensor | None = None
    hisparse_indices: torch.Tensor | None = None
    source_layer: int | None = None

    def publish(self, layer_idx: int, logical_indices: torch.Tensor,
                physical_indices: torch.Tensor | None = None) -> None:
        """Record a full layer's selection. A HiSparse mapping belongs to the
        previous selection and is dropped."""
        self.source_layer = layer_idx
        self.logical_indices, self.physical_indices = logical_indices, physical_indices
        self.hisparse_indices = None

    def publish_hisparse(self, layer_idx: int, hisparse_indices: torch.Tensor) -> None:
        """Attach a hot-slot mapping; only the layer that published the
        selection may attach one."""
        if layer_idx != self.source_layer:
            raise RuntimeError(f"Cannot publish HiSparse mapping for layer {layer_idx} from "
                               f"indexer source layer {self.source_layer}")
        self.hisparse_indices = hisparse_indices

    def require_hisparse(self, layer_idx: int, num_tokens: int, topk: int) -> torch.Tensor | None:
        """The hot mapping when it was made by this same layer at this shape,
        else None (the caller rebuilds it)."""
        hot = self.hisparse_indices
        if hot is not None and layer_idx == self.source_layer and _shape(hot) == (num_tokens, topk):
            return hot
        return None

    def require(self, layer_idx: int, num_tokens: int, topk: int, *,
                require_physical: bool) -> tuple[torch.Tensor, torch.Tensor | None]:
        """The published (logical, physical) pair for a shared layer; raises
        when nothing was published or the shapes do not fit this batch."""
        if self.source_layer is None or self.logical_indices is None:
            raise RuntimeError(f"Shared indexer layer {layer_idx} has no TopK from a preceding full layer")
        want = (num_tokens, topk)
        got = _shape(self.logical_indices)
        if got != want:
            raise RuntimeError(f"Shared indexer layer {layer_idx} received stale TopK shape {got} "
                               f"from layer {self.source_layer}; expected {want}")
        if require_physical and _shape(self.physical_indices) != want:
            raise RuntimeError(f"Shared indexer layer {layer_idx} received invalid physical TopK shape "
                               f"{_shape(self.physical_indices)} from layer {self.source_layer}; "
                               f"expected {want}")
        return self.logical_indices, self.physical_indices

    def select_rows(self, rows: torch.Tensor) -> "IndexerTopKState":
        """A new state holding only the given token rows (copies), for runners
        that carry one seed row per request into later draft iterations."""
        if self.source_layer is None or self.logical_indices is None:
            return IndexerTopKState()
        pick = lambda t: None if t is None else t.index_select(0, rows)   # noqa: E731
        return IndexerTopKState(pick(self.logical_indices), pick(self.physical_indices),
                                pick(self.hisparse_indices), self.source_layer)


_IndexerTopKState = IndexerTopKState


def _get_indexer_mode(config, layer_idx: int) -> str:
    """"full", "shared" or "none" for one attention layer of a DSA model.

    Precedence: no ``index_topk`` -> "none"; layers past the backbone (MTP) ->
    "full"; an explicit ``indexer_types`` list (one entry per backbone layer);
    an ``index_topk_pattern`` string of F/S markers; else every
    ``index_topk_freq``-th layer counting from ``index_skip_topk_offset - 1``
    is full (defaults 1 and 2: every layer full)."""
    if not hasattr(config, "index_topk"):
        return "none"
    n_layers = int(getattr(config, "num_hidden_layers", 0))
    if layer_idx >= n_layers:
        return "full"
    types = getattr(config, "indexer_types", None)
    if types is not None:
        if len(types) != n_layers:
            raise ValueError("indexer_types must contain one entry per backbone layer: "
                             f"got {len(types)} entries for {n_layers} layers")
        mode = str(types[layer_idx]).lower()
        if mode in ("full", "shared"):
            return mode
        raise ValueError(f"Unsupported indexer_types[{layer_idx}]={types[layer_idx]!r}")
    pattern = getattr(config, "index_topk_pattern", None)
    if pattern is not None and layer_idx < len(pattern):
        marker = pattern[layer_idx]
        if isinstance(marker, str):
            marker = marker.upper()
        name = {"F": "full", "FULL": "full", "S": "shared", "SHARED": "shared"}.get(marker) \
            if isinstance(marker, str) else None
        if name is None:
            raise ValueError(f"Unsupported index_topk_pattern[{layer_idx}]={marker!r}")
        return name
    freq = max(int(getattr(config, "index_topk_freq", 1) or 1), 1)
    offset = int(getattr(config, "index_skip_topk_offset", 2) or 0)
    return "full" if max(layer_idx - offset + 1, 0) % freq == 0 else "shared"
