"""PagedKVCacheManager: the paged KV pool and its slot bookkeeping.

Same constructor, attributes, methods and error messages as the reference's
app/memory/manager.py:12-333, so the engine and the reference's tests drive
it unchanged.  On a ROCm device the caches live in HBM
(memory/strategies.py) and the per-step integer and copy work runs in the
HIP kernels:

  * build_slot_mapping    -> pa_pack (GPU), after the same host-side checks
  * scatter_layer_kv      -> pa_reshape_and_cache (GPU)
  * build_block_tables    -> host table, one non-blocking upload

On a CPU store the reference's torch code path is kept as is (it is the
reference's own CPU behaviour, not a fallback of the GPU path: a GPU store
never takes it).
"""

from __future__ import annotations

from typing import List, Optional, Tuple, Union

import numpy as np
import torch

from .. import paged_ops
from ..scheduler.sequence import Sequence
from .block_allocator import PageAllocator, SequenceBlockTable
from .strategies import KVCacheMemoryStrategy, detect_strategy, strategy_from_device


class PagedKVCacheManager:
    @classmethod
    def from_model_config(
        cls,
        config,
        total_blocks: int,
        block_size: int,
        total_cpu_blocks: int = 32,
        dtype: torch.dtype = torch.float32,
        device: Optional[Union[str, torch.device]] = None,
        strategy: Optional[KVCacheMemoryStrategy] = None,
    ) -> "PagedKVCacheManager":
        """manager.py:13-39: KV heads and head_dim from an HF-style config."""
        num_attention_heads = config.num_attention_heads
        num_kv_heads = getattr(config, "num_key_value_heads", num_attention_heads)
        head_dim = getattr(config, "head_dim", None)
        if head_dim is None:
            head_dim = config.hidden_size // num_attention_heads
        manager = cls(
            total_blocks=total_blocks,
            block_size=block_size,
            num_heads=num_kv_heads,
            head_dim=head_dim,
            total_cpu_blocks=total_cpu_blocks,
            dtype=dtype,
            num_layers=config.num_hidden_layers,
            device=device,
            strategy=strategy,
        )
        manager.num_query_heads = num_attention_heads
        return manager

    def __init__(
        self,
        total_blocks: int,
        block_size: int,
        num_heads: int,
        head_dim: int,
        total_cpu_blocks: int = 32,
        dtype: torch.dtype = torch.float32,
        num_layers: int = 1,
        device: Optional[Union[str, torch.device]] = None,
        strategy: Optional[KVCacheMemoryStrategy] = None,
    ) -> None:
        self.block_size = block_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_layers = num_layers
        self.dtype = dtype
        # Query heads of the model using the pool, when known (sizes the
        # prefill work items of a step); None until a model config says.
        self.num_query_heads: Optional[int] = None
        if strategy is not None:
            self.strategy = strategy
        elif device is not None:
            self.strategy = strategy_from_device(device)
        else:
            self.strategy = detect_strategy()
        bytes_per_token = num_layers * num_heads * head_dim * dtype.itemsize * 2
        self.allocator = PageAllocator(total_blocks, block_size, bytes_per_token, total_cpu_blocks)
        self.key_cache, self.value_cache = self.strategy.allocate_cache(
            total_blocks, block_size, num_layers, num_heads, head_dim, dtype
        )

    # -- bookkeeping (manager.py:75-102) -----------------------------------
    @property
    def device(self) -> str:
        return str(self.strategy.device)

    @property
    def on_gpu(self) -> bool:
        return self.key_cache.device.type == "cuda"

    @property
    def total_blocks(self) -> int:
        return self.allocator.get_total_blocks()

    def get_allocator(self) -> PageAllocator:
        return self.allocator

    def init_sequence_table(self, seq: Sequence) -> None:
        if seq.block_table is None:
            seq.block_table = SequenceBlockTable(self.allocator)

    def allocate_prefix_blocks(self, seq: Sequence) -> None:
        self.init_sequence_table(seq)
        needed = seq.total_len - seq.block_table.get_tokens_count()
        for _ in range(needed):
            seq.block_table.append_token()

    def allocate_slot_for_next_token(self, seq: Sequence) -> None:
        assert seq.block_table is not None
        seq.block_table.append_token()

    def free_sequence(self, seq: Sequence) -> None:
        if seq.block_table is not None:
            seq.block_table.release()
            seq.block_table = None

    # -- slot mapping (manager.py:104-128, 301-333) ------------------------
    def check_slot_ranges(self, sequences: List[Sequence], start_tokens: List[int], token_counts: List[int]) -> None:
        """The host-side checks of build_slot_mapping / _sequence_slots."""
        if not (len(sequences) == len(start_tokens) == len(token_counts)):
            raise ValueError(
                f"sequences ({len(sequences)}), start_tokens ({len(start_tokens)}) "
                f"and token_counts ({len(token_counts)}) must have the same length"
            )
        for seq, start, count in zip(sequences, start_tokens, token_counts):
            if seq.block_table is None:
                raise ValueError(f"Sequence {seq.seq_id} has no block table")
            if start < 0 or count < 0:
                raise ValueError(
                    f"Sequence {seq.seq_id}: start_token ({start}) and "
                    f"token_count ({count}) must be non-negative"
                )
            tokens_count = seq.block_table.get_tokens_count()
            if start + count > tokens_count:
                raise ValueError(
                    f"Sequence {seq.seq_id}: tokens [{start}, {start + count}) "
                    f"exceed allocated tokens ({tokens_count})"
                )

    def block_table_tensor(self, sequences: List[Sequence]) -> torch.Tensor:
        """int32 [B, max_blocks] (-1 padded) on the store's device."""
        lists = [seq.block_table.get_physical_blocks() if seq.block_table else [] for seq in sequences]
        width = max((len(b) for b in lists), default=0)
        host = np.full((len(lists), max(width, 1)), -1, dtype=np.int32)
        for i, blocks in enumerate(lists):
            if blocks:
                host[i, : len(blocks)] = blocks
        t = torch.from_numpy(host)
        if self.on_gpu:
            t = t.pin_memory().to(self.key_cache.device, non_blocking=True)
        return t

    def build_slot_mapping(
        self,
        sequences: List[Sequence],
        start_tokens: List[int],
        token_counts: List[int],
    ) -> torch.Tensor:
        self.check_slot_ranges(sequences, start_tokens, token_counts)
        if not sequences:
            return torch.empty((0,), dtype=torch.long, device=self.device)
        if self.on_gpu:
            step = paged_ops.pack_step(
                self.block_table_tensor(sequences), list(start_tokens), list(token_counts), self.block_size
            )
            return step.scatter_slots
        chunks = []
        for seq, start, count in zip(sequences, start_tokens, token_counts):
            chunk = self._sequence_slots(seq, start, count)
            if chunk.numel() > 0:
                chunks.append(chunk)
        if not chunks:
            return torch.empty((0,), dtype=torch.long, device=self.device)
        return torch.cat(chunks)

    # -- KV writes (manager.py:130-168) ---------------------------------------
    def scatter_kv(self, keys: torch.Tensor, values: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        self._validate_token_tensors(
            keys, values, (slot_mapping.numel(), self.num_layers, self.num_heads, self.head_dim)
        )
        for layer_idx in range(self.num_layers):
            self.scatter_layer_kv(layer_idx, keys[:, layer_idx], values[:, layer_idx], slot_mapping)

    def scatter_layer_kv(self, layer_idx: int, keys: torch.Tensor, values: torch.Tensor,
                         slot_mapping: torch.Tensor) -> None:
        self._validate_layer_idx(layer_idx)
        self._validate_token_tensors(keys, values, (slot_mapping.numel(), self.num_heads, self.head_dim))
        if slot_mapping.numel() == 0:
            return
        if self.on_gpu:
            paged_ops.reshape_and_cache(
                keys.to(self.key_cache.device, self.dtype),
                values.to(self.key_cache.device, self.dtype),
                self.key_cache,
                self.value_cache,
                slot_mapping.to(self.key_cache.device, torch.int64),
                layer_idx,
            )
            return
        self.key_cache[layer_idx].view(-1, self.num_heads, self.head_dim)[slot_mapping] = keys
        self.value_cache[layer_idx].view(-1, self.num_heads, self.head_dim)[slot_mapping] = values

    def gather_layer_keys(self, layer_idx: int, slot_indices: torch.Tensor) -> torch.Tensor:
        return self._gather_layer(self.key_cache, layer_idx, slot_indices)

    def gather_layer_values(self, layer_idx: int, slot_indices: torch.Tensor) -> torch.Tensor:
        return self._gather_layer(self.value_cache, layer_idx, slot_indices)

    def write_prefix_kv(self, seq: Sequence, keys: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """manager.py:176-192."""
        if keys.shape != values.shape:
            raise ValueError(f"Keys shape {keys.shape} != Values shape {values.shape}")
        seq_len = keys.shape[1]
        if seq_len == 0 or seq.block_table is None:
            return torch.empty((0,), dtype=torch.long, device=self.device)
        slot_mapping = self.build_slot_mapping([seq], [0], [seq_len])
        self.scatter_kv(keys.transpose(0, 1), values.transpose(0, 1), slot_mapping)
        return slot_mapping

    def write_single_token_kv(self, seq: Sequence, key_token: torch.Tensor, value_token: torch.Tensor) -> None:
        """manager.py:194-205."""
        if seq.block_table is None:
            raise ValueError(f"Sequence {seq.seq_id} has no block table")
        token_index = seq.block_table.get_tokens_count() - 1
        slot_mapping = self.build_slot_mapping([seq], [token_index], [1])
        self.scatter_kv(key_token.unsqueeze(0), value_token.unsqueeze(0), slot_mapping)

    def gather_kv_cache(self, seq: Sequence, read_len: Optional[int] = None):
        """manager.py:207-234: per-layer contiguous [1, H, len, D] K/V of one sequence."""
        if seq.block_table is None:
            return None
        physical_blocks = seq.block_table.get_physical_blocks()
        tokens_count = seq.block_table.get_tokens_count()
        if read_len is None:
            read_len = tokens_count
        if read_len <= 0:
            return None
        idx = torch.as_tensor(physical_blocks, dtype=torch.long, device=self.key_cache.device)
        result = []
        for layer_idx in range(self.num_layers):
            k = self.key_cache[layer_idx].index_select(0, idx).reshape(-1, self.num_heads, self.head_dim)[:read_len]
            v = self.value_cache[layer_idx].index_select(0, idx).reshape(-1, self.num_heads, self.head_dim)[:read_len]
            result.append((k.unsqueeze(0).transpose(1, 2), v.unsqueeze(0).transpose(1, 2)))
        return tuple(result)

    def build_block_tables(self, sequences: List[Sequence]) -> Tuple[torch.Tensor, torch.Tensor]:
        """manager.py:236-271: int32 [B, max_blocks] padded with -1 and int32 token counts."""
        batch_size = len(sequences)
        if batch_size == 0:
            return (
                torch.empty((0, 0), dtype=torch.int32, device=self.device),
                torch.empty((0,), dtype=torch.int32, device=self.device),
            )
        raw = [seq.block_table.get_physical_blocks() if seq.block_table else [] for seq in sequences]
        lens = [seq.block_table.get_tokens_count() if seq.block_table else 0 for seq in sequences]
        max_blocks = max(len(b) for b in raw)
        table = torch.full((batch_size, max_blocks), fill_value=-1, dtype=torch.int32)
        for i, blocks in enumerate(raw):
            if blocks:
                table[i, : len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
        context_lens = torch.tensor(lens, dtype=torch.int32)
        return (
            table.to(self.device, non_blocking=True),
            context_lens.to(self.device, non_blocking=True),
        )

    # -- validation (manager.py:273-299) --------------------------------------
    def _validate_layer_idx(self, layer_idx: int) -> None:
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise ValueError(f"Layer index {layer_idx} out of range (num_layers={self.num_layers})")

    def _validate_token_tensors(self, keys: torch.Tensor, values: torch.Tensor, expected_shape) -> None:
        if keys.shape != values.shape:
            raise ValueError(f"Keys shape {keys.shape} != Values shape {values.shape}")
        if tuple(keys.shape) != tuple(expected_shape):
            raise ValueError(f"Expected keys shape {tuple(expected_shape)}, got {tuple(keys.shape)}")

    def _gather_layer(self, cache: torch.Tensor, layer_idx: int, slot_indices: torch.Tensor) -> torch.Tensor:
        self._validate_layer_idx(layer_idx)
        return cache[layer_idx].view(-1, self.num_heads, self.head_dim).index_select(
            0, slot_indices.to(cache.device)
        )

    def _sequence_slots(self, seq: Sequence, start_token: int, token_count: int) -> torch.Tensor:
        """manager.py:301-333 (CPU store)."""
        self.check_slot_ranges([seq], [start_token], [token_count])
        if token_count == 0:
            return torch.empty((0,), dtype=torch.long, device=self.device)
        first_block = start_token // self.block_size
        last_block = (start_token + token_count - 1) // self.block_size
        physical_blocks = seq.block_table.get_physical_blocks()[first_block : last_block + 1]
        block_offsets = torch.tensor(physical_blocks, dtype=torch.long, device=self.device) * self.block_size
        slot_offsets = torch.arange(self.block_size, dtype=torch.long, device=self.device)
        all_slots = (block_offsets.unsqueeze(1) + slot_offsets.unsqueeze(0)).flatten()
        offset = start_token - first_block * self.block_size
        return all_slots[offset : offset + token_count]
