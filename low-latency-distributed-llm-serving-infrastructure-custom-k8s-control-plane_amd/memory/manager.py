"""PagedKVCacheManager: the paged KV pool, its block tables and slot mapping.

Same constructor, attributes, method names and error messages as the
reference's manager (app/memory/manager.py:12-333), so an engine and the
reference's tests drive it unchanged.  Its organisation is the MI355X
path's own:

  * every sequence's block list is also a row of one :class:`BlockTablePool`
    (memory/block_allocator.py), mirrored in HBM on a GPU store; a step
    uploads only the entries allocated since the last step and the packing
    kernel gathers the step's block table on the device (:meth:`pack_step`);
  * on a GPU store the slot mapping, positions and work lists come from the
    packing kernel (pa_pack) and K/V writes from pa_reshape_and_cache; the
    host checks a step once, vectorised, from the pool's token counts;
  * on a CPU store (the reference's CPU path) the same slot formula runs
    vectorised in NumPy over the pool's host rows;
  * preempted sequences swap their blocks to a pinned host pool and back in
    one launch per cache (:meth:`swap_out` / :meth:`swap_in`).
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from .. import paged_ops
from .block_allocator import BlockTablePool, PageAllocator, SequenceBlockTable
from .strategies import KVCacheMemoryStrategy, detect_strategy, strategy_from_device


def _no_table(seq) -> ValueError:
    return ValueError(f"Sequence {seq.seq_id} has no block table")


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
        """A pool for an HF-style model config (manager.py:13-39): its KV heads
        (``num_key_value_heads``, else the attention heads), its head dim
        (``head_dim``, else hidden_size / heads) and its layer count."""
        query_heads = int(config.num_attention_heads)
        kv_heads = int(getattr(config, "num_key_value_heads", None) or query_heads)
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // query_heads
        manager = cls(total_blocks, block_size, kv_heads, int(head_dim), total_cpu_blocks=total_cpu_blocks,
                      dtype=dtype, num_layers=int(config.num_hidden_layers), device=device, strategy=strategy)
        manager.num_query_heads = query_heads
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
        self.block_size = int(block_size)
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.num_layers = int(num_layers)
        self.dtype = dtype
        # Query heads of the model served from this pool, when a model config
        # gave them (they size the prefill work items and decode workspace).
        self.num_query_heads: Optional[int] = None
        if strategy is None:
            strategy = strategy_from_device(device) if device is not None else detect_strategy()
        self.strategy = strategy
        token_bytes = 2 * self.num_layers * self.num_heads * self.head_dim * dtype.itemsize
        self.allocator = PageAllocator(total_blocks, self.block_size, token_bytes, total_cpu_blocks)
        self.key_cache, self.value_cache = strategy.allocate_cache(
            total_blocks, self.block_size, self.num_layers, self.num_heads, self.head_dim, dtype)
        self.tables = BlockTablePool(width=max(1, min(int(total_blocks), 64)))
        self._device_table: Optional[torch.Tensor] = None
        self._host_pool: Optional[Tuple[torch.Tensor, torch.Tensor]] = None

    # -- pool bookkeeping ---------------------------------------------------------
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

    def init_sequence_table(self, seq) -> None:
        if seq.block_table is None:
            seq.block_table = SequenceBlockTable(self.allocator, self.tables)

    def allocate_prefix_blocks(self, seq) -> None:
        """Slots for every token the sequence holds (prompt + outputs)."""
        self.init_sequence_table(seq)
        table = seq.block_table
        table.append_tokens(seq.total_len - table.get_tokens_count())

    def allocate_slot_for_next_token(self, seq) -> None:
        assert seq.block_table is not None
        seq.block_table.append_token()

    def free_sequence(self, seq) -> None:
        if seq.block_table is not None:
            seq.block_table.release()
            seq.block_table = None

    # -- one step: checks, rows, packing --------------------------------------------
    def step_rows(self, sequences: Sequence, start_tokens, token_counts) -> Tuple[np.ndarray, np.ndarray,
                                                                                   np.ndarray]:
        """(rows, starts, counts) of a step after the slot-range checks of
        build_slot_mapping / _sequence_slots (manager.py:104-128, 301-315),
        each raising the reference's ValueError."""
        if not (len(sequences) == len(start_tokens) == len(token_counts)):
            raise ValueError(
                f"sequences ({len(sequences)}), start_tokens ({len(start_tokens)}) "
                f"and token_counts ({len(token_counts)}) must have the same length")
        try:
            rows = np.fromiter((seq.block_table.row for seq in sequences), dtype=np.int32, count=len(sequences))
        except AttributeError:
            raise _no_table(next(seq for seq in sequences if seq.block_table is None)) from None
        starts = np.asarray(start_tokens, dtype=np.int64).reshape(-1)
        counts = np.asarray(token_counts, dtype=np.int64).reshape(-1)
        if rows.size and rows.min() < 0:
            seq = sequences[int(np.argmin(rows))]
            raise ValueError(f"Sequence {seq.seq_id}: its block table does not belong to this store")
        if rows.size:
            negative = (starts < 0) | (counts < 0)
            beyond = starts + counts > self.tables.tokens[rows]
            if negative.any() or beyond.any():
                i = int(np.argmax(negative | beyond))
                seq, s, c = sequences[i], int(starts[i]), int(counts[i])
                if negative[i]:
                    raise ValueError(f"Sequence {seq.seq_id}: start_token ({s}) and "
                                     f"token_count ({c}) must be non-negative")
                raise ValueError(f"Sequence {seq.seq_id}: tokens [{s}, {s + c}) "
                                 f"exceed allocated tokens ({int(self.tables.tokens[rows[i]])})")
        return rows, starts, counts

    def device_block_table(self) -> Tuple[torch.Tensor, Optional[np.ndarray]]:
        """(HBM copy of the row pool, updates it still needs or None): the
        copy is rebuilt from the host rows when the pool grew, else the
        queued (row, col, block) entries are returned for pa_pack to apply."""
        rebuild, updates = self.tables.take_updates()
        host = self.tables.host
        dev = self._device_table
        if rebuild or dev is None or tuple(dev.shape) != host.shape:
            dev = torch.from_numpy(host.copy()).pin_memory().to(self.key_cache.device, non_blocking=True)
            self._device_table = dev
            return dev, None
        return dev, updates if updates.shape[0] else None

    def pack_step(self, sequences: Sequence, start_tokens, token_counts, *, num_query_heads: Optional[int] = None,
                  with_gather: bool = False, partition_size: Optional[int] = None) -> paged_ops.PackedStep:
        """Check, plan and pack one step on the GPU: the step's host arrays
        handed over in pinned memory, the queued block-table updates applied,
        one launch for a decode batch (two for a larger or prefill step)."""
        rows, starts, counts = self.step_rows(sequences, start_tokens, token_counts)
        return self.pack_rows(rows, starts, counts, num_query_heads=num_query_heads, with_gather=with_gather,
                              partition_size=partition_size)

    def pack_rows(self, rows: np.ndarray, starts: np.ndarray, counts: np.ndarray, *,
                  num_query_heads: Optional[int] = None, with_gather: bool = False,
                  partition_size: Optional[int] = None) -> paged_ops.PackedStep:
        """:meth:`pack_step` for a step :meth:`step_rows` already checked."""
        table, updates = self.device_block_table()
        hq = int(num_query_heads or self.num_query_heads or self.num_heads)
        return paged_ops.pack_step(
            table, starts, counts, self.block_size, rows=rows, updates=updates,
            num_kv_heads=self.num_heads, num_query_heads=hq, head_dim=self.head_dim, dtype=self.dtype,
            with_gather=with_gather, partition_size=partition_size)

    def _host_slots(self, rows: np.ndarray, starts: np.ndarray, counts: np.ndarray) -> np.ndarray:
        """Slots of positions [start, start + count) of every sequence, in
        order: block[p // bs] * bs + p % bs, from the pool's host rows."""
        total = int(counts.sum()) if counts.size else 0
        if total == 0:
            return np.zeros(0, dtype=np.int64)
        owner = np.repeat(np.arange(rows.shape[0]), counts)
        first = np.cumsum(counts) - counts
        pos = np.arange(total, dtype=np.int64) - first[owner] + starts[owner]
        blocks = self.tables.host[rows[owner], pos // self.block_size].astype(np.int64)
        return blocks * self.block_size + pos % self.block_size

    def build_slot_mapping(self, sequences: List, start_tokens: List[int], token_counts: List[int]) -> torch.Tensor:
        """int64 slots of the given token ranges, concatenated in sequence
        order, on the store's device (manager.py:104-128)."""
        rows, starts, counts = self.step_rows(sequences, start_tokens, token_counts)
        if self.on_gpu and rows.size:
            return self.pack_step(sequences, starts, counts).scatter_slots
        return torch.from_numpy(self._host_slots(rows, starts, counts)).to(self.device)

    def build_block_tables(self, sequences: List) -> Tuple[torch.Tensor, torch.Tensor]:
        """int32 [B, max_blocks] block table padded with -1, and int32 token
        counts, on the store's device (manager.py:236-271)."""
        tables = [seq.block_table for seq in sequences]
        rows = [t.row if t is not None else -1 for t in tables]
        width = max((int(self.tables.blocks[r]) for r in rows if r >= 0), default=0)
        out = np.full((len(rows), width), -1, dtype=np.int32)
        lens = np.zeros(len(rows), dtype=np.int32)
        for i, r in enumerate(rows):
            if r >= 0:
                out[i] = self.tables.host[r, :width]
                lens[i] = self.tables.tokens[r]
        return (torch.from_numpy(out).to(self.device, non_blocking=True),
                torch.from_numpy(lens).to(self.device, non_blocking=True))

    # -- K/V writes and reads (manager.py:130-234) -------------------------------------
    def _validate_layer_idx(self, layer_idx: int) -> None:
        if not 0 <= layer_idx < self.num_layers:
            raise ValueError(f"Layer index {layer_idx} out of range (num_layers={self.num_layers})")

    @staticmethod
    def _validate_token_tensors(keys: torch.Tensor, values: torch.Tensor, expected_shape) -> None:
        if keys.shape != values.shape:
            raise ValueError(f"Keys shape {keys.shape} != Values shape {values.shape}")
        if tuple(keys.shape) != tuple(expected_shape):
            raise ValueError(f"Expected keys shape {tuple(expected_shape)}, got {tuple(keys.shape)}")

    def scatter_kv(self, keys: torch.Tensor, values: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Every layer's K/V of the tokens ([T, L, H, D]) into their slots."""
        self._validate_token_tensors(keys, values, (slot_mapping.numel(), self.num_layers, self.num_heads,
                                                    self.head_dim))
        for layer_idx in range(self.num_layers):
            self.scatter_layer_kv(layer_idx, keys[:, layer_idx], values[:, layer_idx], slot_mapping)

    def checked_layer_kv(self, layer_idx: int, keys: torch.Tensor, values: torch.Tensor,
                         num_tokens: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """One layer's new K/V ([T, H, D]) checked as scatter_layer_kv checks
        them, on the cache's device and in its dtype: what the GPU backend
        writes itself."""
        self._validate_layer_idx(layer_idx)
        self._validate_token_tensors(keys, values, (num_tokens, self.num_heads, self.head_dim))
        dev = self.key_cache.device
        return keys.to(dev, self.dtype), values.to(dev, self.dtype)

    def scatter_layer_kv(self, layer_idx: int, keys: torch.Tensor, values: torch.Tensor,
                         slot_mapping: torch.Tensor) -> None:
        """One layer's new K/V ([T, H, D], any token / head strides) into the
        cache at ``slot_mapping`` (manager.py:150-168): pa_reshape_and_cache on
        a GPU store, an index copy on a CPU one."""
        self._validate_layer_idx(layer_idx)
        self._validate_token_tensors(keys, values, (slot_mapping.numel(), self.num_heads, self.head_dim))
        if slot_mapping.numel() == 0:
            return
        if self.on_gpu:
            dev = self.key_cache.device
            paged_ops.reshape_and_cache(keys.to(dev, self.dtype), values.to(dev, self.dtype), self.key_cache,
                                        self.value_cache, slot_mapping.to(dev, torch.int64), layer_idx)
            return
        flat = (-1, self.num_heads, self.head_dim)
        slots = slot_mapping.to(torch.int64)
        self.key_cache[layer_idx].view(flat).index_copy_(0, slots, keys.to(self.dtype))
        self.value_cache[layer_idx].view(flat).index_copy_(0, slots, values.to(self.dtype))

    def _gather_layer(self, cache: torch.Tensor, layer_idx: int, slot_indices: torch.Tensor) -> torch.Tensor:
        self._validate_layer_idx(layer_idx)
        flat = cache[layer_idx].view(-1, self.num_heads, self.head_dim)
        return flat.index_select(0, slot_indices.to(cache.device, torch.int64))

    def gather_layer_keys(self, layer_idx: int, slot_indices: torch.Tensor) -> torch.Tensor:
        return self._gather_layer(self.key_cache, layer_idx, slot_indices)

    def gather_layer_values(self, layer_idx: int, slot_indices: torch.Tensor) -> torch.Tensor:
        return self._gather_layer(self.value_cache, layer_idx, slot_indices)

    def write_prefix_kv(self, seq, keys: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """K/V of a whole prompt ([L, T, H, D]) into the sequence's first T
        slots; returns the slots (manager.py:176-192)."""
        if keys.shape != values.shape:
            raise ValueError(f"Keys shape {keys.shape} != Values shape {values.shape}")
        length = int(keys.shape[1])
        if length == 0 or seq.block_table is None:
            return torch.empty((0,), dtype=torch.long, device=self.device)
        slots = self.build_slot_mapping([seq], [0], [length])
        self.scatter_kv(keys.transpose(0, 1), values.transpose(0, 1), slots)
        return slots

    def write_single_token_kv(self, seq, key_token: torch.Tensor, value_token: torch.Tensor) -> None:
        """K/V ([L, H, D]) of the sequence's last allocated token (manager.py:194-205)."""
        if seq.block_table is None:
            raise _no_table(seq)
        last = seq.block_table.get_tokens_count() - 1
        slots = self.build_slot_mapping([seq], [last], [1])
        self.scatter_kv(key_token.unsqueeze(0), value_token.unsqueeze(0), slots)

    def gather_kv_cache(self, seq, read_len: Optional[int] = None):
        """Per layer, the sequence's first ``read_len`` tokens of K and V as
        [1, H, len, D] (manager.py:207-234); None without a table or tokens."""
        if seq.block_table is None:
            return None
        n = seq.block_table.get_tokens_count() if read_len is None else int(read_len)
        if n <= 0:
            return None
        slots = self.build_slot_mapping([seq], [0], [n])
        return tuple(
            (self.gather_layer_keys(layer, slots).permute(1, 0, 2).unsqueeze(0),
             self.gather_layer_values(layer, slots).permute(1, 0, 2).unsqueeze(0))
            for layer in range(self.num_layers))

    # -- swap to the host pool -------------------------------------------------------
    def host_pool(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """The pinned host swap space (allocated on first use): K and V of
        ``total_cpu_blocks`` blocks in the cache's block layout."""
        if self._host_pool is None:
            self._host_pool = self.strategy.allocate_host_pool(
                self.allocator.get_total_cpu_blocks(), self.block_size, self.num_layers, self.num_heads,
                self.head_dim, self.dtype)
        return self._host_pool

    def swap_out(self, seq) -> List[int]:
        """Move a sequence's blocks to the host pool: host blocks are taken
        (PageAllocator.swap_out), one launch per cache copies every layer's
        blocks out (pa_swap_blocks), and the device blocks return to the free
        list -- safe, since later writes to them follow on the same stream.
        Returns the host block ids (also kept on the sequence's table)."""
        if seq.block_table is None:
            raise _no_table(seq)
        if not self.on_gpu:
            raise RuntimeError("swap needs a store in device memory")
        table = seq.block_table
        blocks = table.get_physical_blocks()
        host_ids = [self.allocator.swap_out(b) for b in blocks]
        hk, hv = self.host_pool()
        mapping = list(zip(blocks, host_ids))
        paged_ops.swap_blocks(self.key_cache, hk, mapping, out=True)
        paged_ops.swap_blocks(self.value_cache, hv, mapping, out=True)
        table.take_blocks()
        table.swapped_blocks = host_ids
        return host_ids

    def swap_in(self, seq) -> List[int]:
        """Bring a swapped-out sequence's blocks back into fresh device blocks
        (PageAllocator.swap_in + one copy launch per cache); returns them."""
        table = seq.block_table
        host_ids = getattr(table, "swapped_blocks", None) if table is not None else None
        if not host_ids:
            raise RuntimeError(f"Sequence {seq.seq_id} is not swapped out")
        blocks = [self.allocator.swap_in(h) for h in host_ids]
        hk, hv = self.host_pool()
        mapping = list(zip(host_ids, blocks))
        paged_ops.swap_blocks(self.key_cache, hk, mapping, out=False)
        paged_ops.swap_blocks(self.value_cache, hv, mapping, out=False)
        table.put_blocks(blocks)
        table.swapped_blocks = None
        return blocks
