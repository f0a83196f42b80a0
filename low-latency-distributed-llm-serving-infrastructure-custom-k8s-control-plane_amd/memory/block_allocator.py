"""Host-side block bookkeeping that feeds the block tables the GPU path reads.

The reference keeps this in C++ (csrc/include/page_allocator.hpp, bound by
csrc/src/bindings.cpp:82-115).  It is outside the accelerated path, so this
is a small Python equivalent of the part the path needs, with the
reference's method names and exception messages:

  * :class:`PageAllocator` -- a FIFO pool of device block ids with reference
    counts (page_allocator.hpp:45-177) and a pool of host block ids that
    swapped-out blocks move to (page_allocator.hpp:179-276);
  * :class:`SequenceBlockTable` -- one sequence's block list, growing by one
    block every ``block_size`` tokens (page_allocator.hpp:376-475).  Given a
    :class:`BlockTablePool` it also keeps its list as a row of that pool,
    which a GPU store mirrors in HBM, so a step's block tables are gathered
    on the device instead of being rebuilt and uploaded from Python lists.
"""

from __future__ import annotations

import threading
from collections import deque
from typing import Dict, List, Optional

import numpy as np


class PageAllocator:
    def __init__(self, total_blocks: int, tokens_per_block: int, bytes_per_token: int,
                 total_cpu_blocks: int = 32) -> None:
        if tokens_per_block <= 0:
            raise ValueError("tokens_per_block must be greater than 0")
        if bytes_per_token <= 0:
            raise ValueError("bytes_per_token must be greater than 0")
        self._total = int(total_blocks)
        self._block_size = int(tokens_per_block)
        self._bytes_per_token = int(bytes_per_token)
        self._total_cpu = int(total_cpu_blocks)
        self._free = deque(range(self._total))
        self._refs = np.zeros(self._total, dtype=np.int32)
        # Host blocks: a stack of free ids, and for every occupied one the
        # device block it was swapped out from.
        self._cpu_free: List[int] = list(range(self._total_cpu - 1, -1, -1))
        self._cpu_owner: Dict[int, int] = {}
        self._lock = threading.Lock()

    def _validate(self, block_id: int) -> None:
        if not 0 <= block_id < self._total:
            raise IndexError(f"Block ID out of range: {block_id}")

    def _validate_cpu(self, cpu_block_id: int) -> None:
        if self._total_cpu == 0:
            raise RuntimeError("Swap unsupported: no host pool configured (total_cpu_blocks == 0)")
        if not 0 <= cpu_block_id < self._total_cpu:
            raise IndexError(f"CPU block ID out of range: {cpu_block_id}")
        if cpu_block_id not in self._cpu_owner:
            raise RuntimeError(f"CPU block {cpu_block_id} is not currently swapped out")

    # -- device blocks ---------------------------------------------------------
    def allocate_block(self) -> int:
        with self._lock:
            if not self._free:
                raise RuntimeError("Out of Memory: No free VRAM pages available in KV-Cache pool!")
            block_id = self._free.popleft()
            self._refs[block_id] = 1
            return block_id

    def allocate_blocks(self, count: int) -> List[int]:
        with self._lock:
            if len(self._free) < count:
                raise RuntimeError("Out of Memory: Not enough free blocks available in KV-Cache pool!")
            out = [self._free.popleft() for _ in range(count)]
            self._refs[out] = 1
            return out

    def share_block(self, block_id: int) -> None:
        with self._lock:
            self._validate(block_id)
            if self._refs[block_id] <= 0:
                raise RuntimeError(f"Cannot share unallocated block {block_id}")
            self._refs[block_id] += 1

    def free_block(self, block_id: int) -> None:
        with self._lock:
            self._validate(block_id)
            if self._refs[block_id] <= 0:
                raise RuntimeError(f"Double-free or free on unallocated block detected: ID {block_id}")
            self._refs[block_id] -= 1
            if self._refs[block_id] == 0:
                self._free.append(block_id)

    # -- host pool (swap) ------------------------------------------------------
    def swap_out(self, gpu_block_id: int) -> int:
        """Move a block's ownership to a free host block: the device block is
        freed at once, so its contents must be copied out (pa_swap_blocks) on
        the stream before any later write to it."""
        with self._lock:
            self._validate(gpu_block_id)
            if self._refs[gpu_block_id] != 1:
                raise RuntimeError("Cannot swap out block with ref_count != 1")
            if self._total_cpu == 0:
                raise RuntimeError("Swap unsupported: no host pool configured (total_cpu_blocks == 0)")
            if not self._cpu_free:
                raise RuntimeError("OOM: Host RAM Block Pool exhausted during swap out")
            cpu = self._cpu_free.pop()
            self._cpu_owner[cpu] = gpu_block_id
            self._refs[gpu_block_id] = 0
            self._free.append(gpu_block_id)
            return cpu

    def swap_in(self, cpu_block_id: int) -> int:
        """A fresh device block for the contents of a swapped-out host block;
        the host block is free again once its copy-in has run."""
        with self._lock:
            self._validate_cpu(cpu_block_id)
            if not self._free:
                raise RuntimeError("OOM: No free VRAM blocks available to swap in")
            gpu = self._free.popleft()
            self._refs[gpu] = 1
            del self._cpu_owner[cpu_block_id]
            self._cpu_free.append(cpu_block_id)
            return gpu

    def release_swapped_block(self, cpu_block_id: int) -> None:
        with self._lock:
            self._validate_cpu(cpu_block_id)
            del self._cpu_owner[cpu_block_id]
            self._cpu_free.append(cpu_block_id)

    def get_cpu_block_id(self, gpu_block_id: int) -> int:
        with self._lock:
            self._validate(gpu_block_id)
            for cpu, gpu in self._cpu_owner.items():
                if gpu == gpu_block_id:
                    return cpu
            raise RuntimeError(f"Block {gpu_block_id} is not swapped out")

    # -- queries ---------------------------------------------------------------
    def get_num_free_blocks(self) -> int:
        with self._lock:
            return len(self._free)

    def get_num_free_cpu_blocks(self) -> int:
        with self._lock:
            return len(self._cpu_free)

    def get_total_blocks(self) -> int:
        return self._total

    def get_total_cpu_blocks(self) -> int:
        return self._total_cpu

    def get_block_size(self) -> int:
        return self._block_size

    def get_bytes_per_token(self) -> int:
        return self._bytes_per_token

    def get_host_pool_bytes(self) -> int:
        return self._total_cpu * self._block_size * self._bytes_per_token

    def get_utilization_percentage(self) -> float:
        with self._lock:
            return 100.0 * (self._total - len(self._free)) / self._total if self._total else 0.0


class BlockTablePool:
    """The block lists of all live sequences as rows of one int32 table.

    ``host`` is the authoritative copy: row r, column c is the c-th physical
    block of the sequence holding row r, -1 past its last block.  Every
    change made since the last step is queued as a (row, col, block) triple;
    the packing kernel applies the queue to the device copy before it
    gathers the step's rows (pa_pack), so a decode step uploads a few
    entries instead of its whole table.  The table grows by doubling; after
    a growth the device copy is rebuilt from ``host`` once.
    """

    def __init__(self, rows: int = 64, width: int = 64) -> None:
        self.host = np.full((max(rows, 1), max(width, 1)), -1, dtype=np.int32)
        self.blocks = np.zeros(self.host.shape[0], dtype=np.int32)  # blocks per row
        self.tokens = np.zeros(self.host.shape[0], dtype=np.int64)  # tokens per row
        self._free_rows: List[int] = list(range(self.host.shape[0] - 1, -1, -1))
        self._pending: List[int] = []  # flat (row, col, block) triples
        self._rebuild = True  # the device copy must be rebuilt from `host`
        self._lock = threading.Lock()

    @property
    def num_rows(self) -> int:
        return int(self.host.shape[0])

    @property
    def width(self) -> int:
        return int(self.host.shape[1])

    def _grow(self, rows: int, width: int) -> None:
        old = self.host
        self.host = np.full((rows, width), -1, dtype=np.int32)
        self.host[: old.shape[0], : old.shape[1]] = old
        for name in ("blocks", "tokens"):
            arr = getattr(self, name)
            grown = np.zeros(rows, dtype=arr.dtype)
            grown[: arr.shape[0]] = arr
            setattr(self, name, grown)
        self._free_rows = list(range(rows - 1, old.shape[0] - 1, -1)) + self._free_rows
        self._pending.clear()
        self._rebuild = True

    def acquire(self) -> int:
        with self._lock:
            if not self._free_rows:
                self._grow(2 * self.num_rows, self.width)
            return self._free_rows.pop()

    def release(self, row: int) -> None:
        with self._lock:
            n = int(self.blocks[row])
            if n and not self._rebuild:
                cols = np.arange(n, dtype=np.int32)
                triples = np.stack([np.full(n, row, np.int32), cols, np.full(n, -1, np.int32)], axis=1)
                self._pending.extend(triples.reshape(-1).tolist())
            self.host[row, :n] = -1
            self.blocks[row] = 0
            self.tokens[row] = 0
            self._free_rows.append(row)

    def set(self, row: int, col: int, block: int) -> None:
        with self._lock:
            if col >= self.width:
                width = self.width
                while width <= col:
                    width *= 2
                self._grow(self.num_rows, width)
            self.host[row, col] = block
            if col >= self.blocks[row]:
                self.blocks[row] = col + 1
            if not self._rebuild:
                self._pending += (row, col, block)

    def take_updates(self):
        """(rebuild, updates): whether the device copy must be rebuilt from
        ``host``, else the int32 [n, 3] triples to apply; clears the queue.

        The queue can hold one (row, col) several times: a row released and
        taken again before the next step queues its -1 resets and then the
        new blocks.  pa_pack stores the triples in no fixed order, so only
        the last value queued per (row, col) is returned, and it equals
        ``host[row, col]``."""
        with self._lock:
            rebuild, self._rebuild = self._rebuild, False
            updates = np.asarray(self._pending, dtype=np.int32).reshape(-1, 3)
            self._pending.clear()
            if updates.shape[0] > 1:
                keys = updates[:, 0].astype(np.int64) * self.width + updates[:, 1]
                # first occurrence in the reversed queue = last one queued
                _, last = np.unique(keys[::-1], return_index=True)
                keep = np.sort(updates.shape[0] - 1 - last)
                if keep.shape[0] != updates.shape[0]:
                    updates = np.ascontiguousarray(updates[keep])
            return rebuild, updates

    def mark_rebuild(self) -> None:
        """The device copy was lost (e.g. a new device): rebuild it next step."""
        with self._lock:
            self._pending.clear()
            self._rebuild = True


class SequenceBlockTable:
    """One sequence's physical blocks (page_allocator.hpp:376-475); with a
    pool, also its row there."""

    def __init__(self, allocator: PageAllocator, pool: Optional[BlockTablePool] = None) -> None:
        self._allocator = allocator
        self._block_size = allocator.get_block_size()
        self._tokens = 0
        self._blocks: List[int] = []
        self._pool = pool
        self.row = pool.acquire() if pool is not None else -1

    def _record(self, col: int, block_id: int) -> None:
        if self._pool is not None:
            if self.row < 0:  # reused after release
                self.row = self._pool.acquire()
            self._pool.set(self.row, col, block_id)

    def append_token(self) -> None:
        if self._tokens % self._block_size == 0:
            block = self._allocator.allocate_block()
            self._blocks.append(block)
            self._record(len(self._blocks) - 1, block)
        self._tokens += 1
        if self._pool is not None:
            self._pool.tokens[self.row] = self._tokens

    def append_tokens(self, n: int) -> None:
        """``n`` append_token calls, with the new blocks taken in one call."""
        if n <= 0:
            return
        have = len(self._blocks) * self._block_size
        need = max(0, -(-(self._tokens + n - have) // self._block_size))
        if need:
            first = len(self._blocks)
            new = self._allocator.allocate_blocks(need)
            self._blocks.extend(new)
            for i, block in enumerate(new):
                self._record(first + i, block)
        self._tokens += n
        if self._pool is not None:
            self._pool.tokens[self.row] = self._tokens

    def append_block(self, block_id: int) -> None:
        self._allocator._validate(block_id)
        self._blocks.append(block_id)
        self._record(len(self._blocks) - 1, block_id)

    def replace_block(self, old_block_id: int, new_block_id: int) -> None:
        self._allocator._validate(new_block_id)
        if old_block_id not in self._blocks:
            raise RuntimeError(f"Block ID {old_block_id} not found in block table")
        col = self._blocks.index(old_block_id)
        self._blocks[col] = new_block_id
        self._record(col, new_block_id)

    def release(self) -> None:
        for block in self._blocks:
            self._allocator.free_block(block)
        self._blocks = []
        self._tokens = 0
        if self._pool is not None and self.row >= 0:
            self._pool.release(self.row)
            self.row = -1

    def take_blocks(self) -> List[int]:
        """Hand the block list to the caller (who owns the blocks from now on)
        and leave the table empty but keep its token count: how a swap-out
        detaches blocks without freeing them here."""
        blocks, self._blocks = self._blocks, []
        if self._pool is not None and self.row >= 0:
            tokens = self._tokens
            self._pool.release(self.row)
            self.row = self._pool.acquire()
            self._pool.tokens[self.row] = tokens
        return blocks

    def put_blocks(self, blocks: List[int]) -> None:
        """Install a block list (swap-in), replacing an empty one."""
        if self._blocks:
            raise RuntimeError("put_blocks needs an empty block table")
        for block in blocks:
            self.append_block(block)

    def get_physical_blocks(self) -> List[int]:
        return list(self._blocks)

    def get_tokens_count(self) -> int:
        return self._tokens
