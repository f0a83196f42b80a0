"""Paged attention on top of the paged KV cache (the per-step and per-layer glue).

Same operator API as the reference's app/model/paged_attention.py:
``PagedStepContext`` (same constructor and attributes), the per-layer hook
``paged_attention_forward`` registered in transformers'
ALL_ATTENTION_FUNCTIONS, ``register_paged_attention`` and
``run_paged_forward``.  On a GPU store the context is packed once per step
by the HIP packing kernel (``self.packed``: device cu_seqlens, slots,
positions and the attention work lists), and every layer then runs
reshape_and_cache + the installed backend on the device without host syncs.
"""

from __future__ import annotations

from typing import List, Optional, Sequence as SequenceABC

import torch

from .. import paged_ops
from ..memory.manager import PagedKVCacheManager
from ..scheduler.sequence import Sequence

PAGED_ATTENTION_NAME = "paged"

# Pluggable backend (paged_attention.py:22-25); None -> inline SDPA path.
_BACKEND = None
_FALLBACK_BACKEND = None


def _get_fallback_backend():
    global _FALLBACK_BACKEND
    if _FALLBACK_BACKEND is None:
        from .attention_backends import TorchSdpBackend

        _FALLBACK_BACKEND = TorchSdpBackend()
    return _FALLBACK_BACKEND


def set_backend(backend) -> None:
    """Install the backend every layer dispatches to (None = inline SDPA)."""
    global _BACKEND
    _BACKEND = backend


class PagedStepContext:
    """Slot bookkeeping and attention mask for a single engine step
    (paged_attention.py:37-118)."""

    def __init__(
        self,
        store: PagedKVCacheManager,
        sequences: List[Sequence],
        start_positions: List[int],
        new_token_counts: List[int],
        prefill_tile: Optional[int] = None,
    ) -> None:
        if not (len(sequences) == len(start_positions) == len(new_token_counts)):
            raise ValueError(
                f"sequences ({len(sequences)}), start_positions ({len(start_positions)}) "
                f"and new_token_counts ({len(new_token_counts)}) must have the same length"
            )
        self.store = store
        self.sequences = list(sequences)
        self.start_positions = list(start_positions)
        self.new_token_counts = list(new_token_counts)
        self.context_lens = [start + count for start, count in zip(start_positions, new_token_counts)]
        self.cu_seqlens = _cumulative_offsets(new_token_counts)
        self.cu_context_offsets = _cumulative_offsets(self.context_lens)
        self.packed: Optional[paged_ops.PackedStep] = None
        self._mask: Optional[torch.Tensor] = None
        self._gather_slots: Optional[torch.Tensor] = None

        if store.on_gpu:
            # Same checks as the two build_slot_mapping calls of the
            # reference (scatter range, then the whole context).
            store.check_slot_ranges(self.sequences, self.start_positions, self.new_token_counts)
            store.check_slot_ranges(self.sequences, [0] * len(self.sequences), self.context_lens)
            hq = getattr(store, "num_query_heads", None) or store.num_heads
            if prefill_tile is None:
                prefill_tile = paged_ops.prefill_tile_for(hq, store.num_heads)
            if self.sequences:
                self.packed = paged_ops.pack_step(
                    store.block_table_tensor(self.sequences),
                    self.start_positions,
                    self.new_token_counts,
                    store.block_size,
                    prefill_tile=prefill_tile,
                    num_kv_heads=store.num_heads,
                    num_query_heads=hq,
                    head_dim=store.head_dim,
                    dtype=store.dtype,
                )
                self.scatter_slots = self.packed.scatter_slots
            else:
                self.scatter_slots = torch.empty((0,), dtype=torch.long, device=store.device)
        else:
            self.scatter_slots = store.build_slot_mapping(
                self.sequences, self.start_positions, self.new_token_counts
            )
            self._gather_slots = store.build_slot_mapping(
                self.sequences, [0] * len(self.sequences), self.context_lens
            )

    def packed_for(self, num_query_heads: int) -> paged_ops.PackedStep:
        """The packed step with prefill work items sized for ``num_query_heads``
        (re-packs once if the context was built for another head count)."""
        if self.packed is None:
            raise RuntimeError("this step is not on a GPU store")
        tile = paged_ops.prefill_tile_for(num_query_heads, self.store.num_heads)
        if self.packed.prefill_tile != tile:
            self.packed = paged_ops.pack_step(
                self.packed.block_tables,
                self.start_positions,
                self.new_token_counts,
                self.store.block_size,
                prefill_tile=tile,
                partition_size=self.packed.partition_size,
                start_positions_dev=self.packed.start_positions,
                new_token_counts_dev=self.packed.new_token_counts,
            )
        return self.packed

    @property
    def gather_slots(self) -> torch.Tensor:
        """int64 [C]: slots of every context token, sequence by sequence."""
        if self._gather_slots is None:
            if self.packed is not None:
                self._gather_slots = self.packed.gather_slots
            else:
                self._gather_slots = torch.empty((0,), dtype=torch.long, device=self.store.device)
        return self._gather_slots

    @property
    def num_query_tokens(self) -> int:
        return int(self.cu_seqlens[-1])

    @property
    def num_context_tokens(self) -> int:
        return int(self.cu_context_offsets[-1])

    def position_ids(self, device: torch.device) -> torch.Tensor:
        """Flat per-token positions, restarting at every sequence boundary."""
        if self.packed is not None and torch.device(device) == self.packed.position_ids.device:
            return self.packed.position_ids.unsqueeze(0)
        positions = [
            torch.arange(start, start + count, dtype=torch.long, device=device)
            for start, count in zip(self.start_positions, self.new_token_counts)
        ]
        if not positions:
            return torch.empty((1, 0), dtype=torch.long, device=device)
        return torch.cat(positions).unsqueeze(0)

    def attention_mask(self, device: torch.device) -> torch.Tensor:
        """Block-diagonal causal mask bool (1, 1, T, C), True = attended.

        Only the SDPA backend materialises it; the HIP kernels evaluate the
        same rule from cu_seqlens / context_lens."""
        if self._mask is not None and self._mask.device == torch.device(device):
            return self._mask
        query_index = _sequence_index(self.new_token_counts, device)
        context_index = _sequence_index(self.context_lens, device)
        cu_seqlens = self.cu_seqlens.to(device)
        cu_context_offsets = self.cu_context_offsets.to(device)
        starts = torch.tensor(self.start_positions, dtype=torch.long, device=device)
        query_position = torch.arange(self.num_query_tokens, device=device)
        query_position = query_position - cu_seqlens[query_index] + starts[query_index]
        context_position = torch.arange(self.num_context_tokens, device=device)
        context_position = context_position - cu_context_offsets[context_index]
        same_sequence = context_index.unsqueeze(0) == query_index.unsqueeze(1)
        within_causal_window = context_position.unsqueeze(0) <= query_position.unsqueeze(1)
        self._mask = (same_sequence & within_causal_window).unsqueeze(0).unsqueeze(0)
        return self._mask


def _cumulative_offsets(counts: List[int]) -> torch.Tensor:
    offsets = [0]
    for count in counts:
        offsets.append(offsets[-1] + count)
    return torch.tensor(offsets, dtype=torch.long)


def _sequence_index(counts: List[int], device: torch.device) -> torch.Tensor:
    if not counts:
        return torch.empty((0,), dtype=torch.long, device=device)
    return torch.repeat_interleave(
        torch.arange(len(counts), dtype=torch.long, device=device),
        torch.tensor(counts, dtype=torch.long, device=device),
    )


def paged_attention_forward(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Optional[torch.Tensor] = None,
    dropout: float = 0.0,
    scaling: Optional[float] = None,
    **kwargs,
) -> tuple[torch.Tensor, None]:
    """Per-layer hook (paged_attention.py:138-180): scatter the new K/V into the
    paged blocks, then attend through the installed backend (falling back to
    SDPA for shapes it refuses) or the inline SDPA path."""
    context: PagedStepContext = module.paged_context
    store: PagedKVCacheManager = context.store
    layer_idx = module.layer_idx

    new_keys = key.squeeze(0).transpose(0, 1)
    new_values = value.squeeze(0).transpose(0, 1)
    store.scatter_layer_kv(layer_idx, new_keys, new_values, context.scatter_slots)

    scale = scaling if scaling is not None else module.scaling
    backend = _BACKEND
    if backend is not None and not backend.supports(context, query.shape[2]):
        backend = _get_fallback_backend()
    if backend is not None:
        return backend.attend(query, store, layer_idx, context, scale, dropout), None
    from .attention_backends import dense_sdpa

    return dense_sdpa(query, store, layer_idx, context, scale, dropout), None


def register_paged_attention(model) -> None:
    """Route every decoder layer of ``model`` through the paged attention."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    ALL_ATTENTION_FUNCTIONS.register(PAGED_ATTENTION_NAME, paged_attention_forward)
    for layer in _decoder_layers(model):
        layer.self_attn.paged_context = None
    model.config._attn_implementation = PAGED_ATTENTION_NAME


def run_paged_forward(model, context: PagedStepContext, input_ids: torch.Tensor) -> torch.Tensor:
    """Run one flat forward pass whose KV lands in the paged blocks."""
    decoder = _decoder(model)
    for layer in decoder.layers:
        layer.self_attn.paged_context = context
    position_ids = context.position_ids(input_ids.device)
    outputs = model(input_ids, position_ids=position_ids, use_cache=False)
    return outputs.logits


def _decoder(model) -> torch.nn.Module:
    for attribute in ("model", "transformer", "base_model"):
        candidate = getattr(model, attribute, None)
        if candidate is not None and hasattr(candidate, "layers"):
            return candidate
    return model


def _decoder_layers(model) -> SequenceABC[torch.nn.Module]:
    return _decoder(model).layers
