"""Paged attention on top of the paged KV cache: the per-step and per-layer glue.

The operator API is the reference's (app/model/paged_attention.py):
``PagedStepContext`` with the same constructor and attributes, the per-layer
hook ``paged_attention_forward`` registered in transformers'
ALL_ATTENTION_FUNCTIONS, ``register_paged_attention`` and
``run_paged_forward``.  The step runs flat: all sequences of a step are one
``[1, T]`` batch.

On a GPU store the context is packed once per step (``self.packed``: each
sequence's row of the device-resident block-table pool, cu_seqlens, slots,
positions and the attention work lists, from the step's host arrays handed
over in pinned memory and the packing kernels), and every layer then writes
its new K/V rows and runs the HIP attention kernels on the device without
host syncs (for a decode step the rows are written inside the decode
launches).  A GPU store always
takes the HIP path: with no backend installed the hook installs it, and the
reference's dense SDPA path is refused there (it would gather the whole
context and build a T x C mask on the device).
"""

from __future__ import annotations

from typing import List, Optional

import numpy as np
import torch

from .. import paged_ops

PAGED_ATTENTION_NAME = "paged"

# The backend every layer dispatches to (paged_attention.py:22-25).  None on a
# CPU store means the inline SDPA path; a GPU store installs the HIP backend.
_BACKEND = None
_FALLBACK_BACKEND = None


def _get_fallback_backend():
    global _FALLBACK_BACKEND
    if _FALLBACK_BACKEND is None:
        from .attention_backends import TorchSdpBackend

        _FALLBACK_BACKEND = TorchSdpBackend()
    return _FALLBACK_BACKEND


def set_backend(backend) -> None:
    """Install the backend every layer dispatches to (None = the default)."""
    global _BACKEND
    _BACKEND = backend


def _offsets(counts: np.ndarray) -> torch.Tensor:
    """int64 [n + 1]: 0 followed by the running totals of ``counts``."""
    out = np.zeros(counts.shape[0] + 1, dtype=np.int64)
    np.cumsum(counts, out=out[1:])
    return torch.from_numpy(out)


class PagedStepContext:
    """Slot bookkeeping and attention layout of one engine step
    (paged_attention.py:37-118).

    Attributes (the reference's): store, sequences, start_positions,
    new_token_counts, context_lens (lists), cu_seqlens, cu_context_offsets
    (CPU int64 tensors), scatter_slots, gather_slots (int64 on the store's
    device), num_query_tokens, num_context_tokens.  ``packed`` is the GPU
    description of the step (None on a CPU store).  The host-side lists and
    offsets are built on first use: a GPU step needs none of them.
    """

    def __init__(self, store, sequences: List, start_positions: List[int], new_token_counts: List[int],
                 prefill_tile: Optional[int] = None) -> None:
        if not (len(sequences) == len(start_positions) == len(new_token_counts)):
            raise ValueError(
                f"sequences ({len(sequences)}), start_positions ({len(start_positions)}) "
                f"and new_token_counts ({len(new_token_counts)}) must have the same length"
            )
        self.store = store
        self.sequences = sequences if isinstance(sequences, list) else list(sequences)
        self.packed: Optional[paged_ops.PackedStep] = None
        self._gather_slots: Optional[torch.Tensor] = None
        self._mask: Optional[torch.Tensor] = None
        self._rows, self._starts, self._counts = store.step_rows(self.sequences, start_positions, new_token_counts)
        if store.on_gpu:
            if self.sequences:
                self.packed = store.pack_rows(self._rows, self._starts, self._counts)
                self.scatter_slots = self.packed.scatter_slots
            else:
                self.scatter_slots = torch.empty((0,), dtype=torch.long, device=store.device)
        else:
            self.scatter_slots = torch.from_numpy(store._host_slots(self._rows, self._starts, self._counts))
            self._gather_slots = torch.from_numpy(
                store._host_slots(self._rows, np.zeros_like(self._starts), self._starts + self._counts))

    # -- host-side views of the step (built on first use) ------------------------------
    def _cached(self, name, build):
        value = self.__dict__.get(name)
        if value is None:
            value = self.__dict__[name] = build()
        return value

    @property
    def start_positions(self) -> List[int]:
        return self._cached("_start_list", self._starts.tolist)

    @property
    def new_token_counts(self) -> List[int]:
        return self._cached("_count_list", self._counts.tolist)

    @property
    def context_lens(self) -> List[int]:
        return self._cached("_ctx_list", lambda: (self._starts + self._counts).tolist())

    @property
    def cu_seqlens(self) -> torch.Tensor:
        return self._cached("_cu_q", lambda: _offsets(self._counts))

    @property
    def cu_context_offsets(self) -> torch.Tensor:
        return self._cached("_cu_c", lambda: _offsets(self._starts + self._counts))

    def packed_for(self, num_query_heads: int) -> paged_ops.PackedStep:
        """The packed step with prefill work items and decode workspace sized
        for ``num_query_heads`` (re-packs once if the store did not know the
        model's head count)."""
        if self.packed is None:
            raise RuntimeError("this step is not on a GPU store")
        tile = paged_ops.prefill_tile_for(num_query_heads, self.store.num_heads)
        if self.packed.prefill_tile != tile:
            self.packed = self.store.pack_rows(self._rows, self._starts, self._counts,
                                               num_query_heads=num_query_heads,
                                               partition_size=self.packed.partition_size)
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
        return int(self._counts.sum())

    @property
    def num_context_tokens(self) -> int:
        return int((self._starts + self._counts).sum())

    def position_ids(self, device: torch.device) -> torch.Tensor:
        """[1, T] positions, restarting at every sequence boundary."""
        if self.packed is not None and torch.device(device) == self.packed.buffer.device:
            return self.packed.position_ids.unsqueeze(0)
        counts = np.asarray(self.new_token_counts, dtype=np.int64)
        total = int(counts.sum()) if counts.size else 0
        owner = np.repeat(np.arange(counts.size), counts)
        first = self.cu_seqlens.numpy()[:-1]
        pos = np.arange(total, dtype=np.int64) - first[owner] + np.asarray(self.start_positions, np.int64)[owner]
        return torch.from_numpy(pos).to(device).unsqueeze(0)

    def attention_mask(self, device: torch.device) -> torch.Tensor:
        """Block-diagonal causal mask, bool (1, 1, T, C), True = attended:
        query token i of sequence s (position start_s + i) sees context
        position j of the same sequence when j <= start_s + i.

        Only the SDPA path materialises it; the HIP kernels evaluate the same
        rule from cu_seqlens and context_lens."""
        device = torch.device(device)
        if self._mask is not None and self._mask.device == device:
            return self._mask
        q_seq = torch.repeat_interleave(torch.arange(len(self.new_token_counts)),
                                        torch.tensor(self.new_token_counts, dtype=torch.long))
        c_seq = torch.repeat_interleave(torch.arange(len(self.context_lens)),
                                        torch.tensor(self.context_lens, dtype=torch.long))
        q_pos = self.position_ids(torch.device("cpu"))[0]
        c_pos = torch.arange(self.num_context_tokens) - self.cu_context_offsets[c_seq]
        mask = (q_seq[:, None] == c_seq[None, :]) & (c_pos[None, :] <= q_pos[:, None])
        self._mask = mask[None, None].to(device)
        return self._mask


def _default_backend(store):
    """The backend a layer uses when none is installed: the HIP backend for a
    GPU store (installed for every later layer; raises when the library is
    missing), none (inline SDPA) for a CPU store."""
    global _BACKEND
    if not store.on_gpu:
        return None
    from .attention_backends import select_backend

    _BACKEND = select_backend("native")
    return _BACKEND


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
    """Per-layer hook (paged_attention.py:138-180): write the layer's new K/V
    into the paged blocks, then attend through the installed backend.  A CPU
    store falls back to SDPA for shapes the backend refuses, or runs the
    inline SDPA path with none installed; a GPU store runs the HIP kernels."""
    context: PagedStepContext = module.paged_context
    store = context.store
    layer_idx = module.layer_idx
    # [1, H_kv, T, D] projections -> [T, H_kv, D] views (no copy)
    new_key, new_value = key[0].transpose(0, 1), value[0].transpose(0, 1)
    scale = module.scaling if scaling is None else scaling
    backend = _BACKEND if _BACKEND is not None else _default_backend(store)
    if store.on_gpu:
        from .attention_backends import NativePagedBackend

        if not isinstance(backend, NativePagedBackend):
            raise RuntimeError(
                f"a GPU store runs the HIP paged-attention backend, not {type(backend).__name__} "
                "(dense SDPA would gather every context and build a T x C mask on the device)")
        if query.shape[2] == 0:
            return query.new_empty((1, 0, query.shape[1], query.shape[3])), None
        # The backend writes the new rows (inside the decode launches for a
        # step of single-token sequences) before it attends.
        new_key, new_value = store.checked_layer_kv(layer_idx, new_key, new_value, context.num_query_tokens)
        return backend.attend(query, store, layer_idx, context, scale, dropout, new_key=new_key,
                              new_value=new_value), None
    store.scatter_layer_kv(layer_idx, new_key, new_value, context.scatter_slots)
    if backend is not None:
        if not backend.supports(context, query.shape[2]):
            backend = _get_fallback_backend()
        return backend.attend(query, store, layer_idx, context, scale, dropout), None
    from .attention_backends import dense_sdpa

    return dense_sdpa(query, store, layer_idx, context, scale, dropout), None


def _decoder(model) -> torch.nn.Module:
    """The module holding the decoder layers: the model's own decoder when it
    exposes one, else the first of its usual attributes that has ``layers``."""
    getter = getattr(model, "get_decoder", None)
    if callable(getter):
        try:
            decoder = getter()
        except (AttributeError, NotImplementedError):
            decoder = None
        if decoder is not None and hasattr(decoder, "layers"):
            return decoder
    for name in ("model", "transformer", "base_model"):
        inner = getattr(model, name, None)
        if inner is not None and hasattr(inner, "layers"):
            return inner
    return model


def register_paged_attention(model, backend=None) -> None:
    """Route every decoder layer of ``model`` through the paged hook
    (paged_attention.py:183-188) and install ``backend`` (by default the one
    select_backend names: the HIP backend when the library and a ROCm device
    are there)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    from .attention_backends import select_backend

    ALL_ATTENTION_FUNCTIONS.register(PAGED_ATTENTION_NAME, paged_attention_forward)
    for layer in _decoder(model).layers:
        layer.self_attn.paged_context = None
    model.config._attn_implementation = PAGED_ATTENTION_NAME
    set_backend(backend if backend is not None else select_backend())


def run_paged_forward(model, context: PagedStepContext, input_ids: torch.Tensor, logits_to_keep=None
                      ) -> torch.Tensor:
    """One flat forward pass whose K/V lands in the paged blocks
    (paged_attention.py:191-207).  ``logits_to_keep`` (a device index tensor
    or a count) restricts the LM head to those rows, e.g. each sequence's
    last token."""
    for layer in _decoder(model).layers:
        layer.self_attn.paged_context = context
    extra = {} if logits_to_keep is None else {"logits_to_keep": logits_to_keep}
    out = model(input_ids, position_ids=context.position_ids(input_ids.device), use_cache=False, **extra)
    return out.logits
