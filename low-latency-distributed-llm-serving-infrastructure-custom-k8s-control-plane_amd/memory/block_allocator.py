"""Host-side block bookkeeping that produces the block tables the GPU path reads.

The reference keeps this in C++ (csrc/include/page_allocator.hpp, bound by
csrc/src/bindings.cpp:82-115); it is outside the accelerated path, so this is
a small Python equivalent of the part the path needs: a FIFO pool of block
ids with reference counts (PageAllocator, page_allocator.hpp:45-177) and a
per-sequence block list that grows one block every ``block_size`` tokens
(SequenceBlockTable, page_allocator.hpp:376-475).  Swap bookkeeping is not
carried over.
"""

from __future__ import annotations

import threading
from collections import deque
from typing import List


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
        self._total_cpu_blocks = int(total_cpu_blocks)
        self._free = deque(range(self._total))
        self._refs = [0] * self._total
        self._lock = threading.Lock()

    def _validate(self, block_id: int) -> None:
        if block_id < 0 or block_id >= self._total:
            raise IndexError(f"Block ID out of range: {block_id}")

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
            for b in out:
                self._refs[b] = 1
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

    def get_num_free_blocks(self) -> int:
        with self._lock:
            return len(self._free)

    def get_total_blocks(self) -> int:
        return self._total

    def get_block_size(self) -> int:
        return self._block_size

    def get_bytes_per_token(self) -> int:
        return self._bytes_per_token

    def get_host_pool_bytes(self) -> int:
        return self._total_cpu_blocks * self._block_size * self._bytes_per_token

    def get_utilization_percentage(self) -> float:
        with self._lock:
            if self._total == 0:
                return 0.0
            return 100.0 * (self._total - len(self._free)) / self._total


class SequenceBlockTable:
    def __init__(self, allocator: PageAllocator) -> None:
        self._allocator = allocator
        self._block_size = allocator.get_block_size()
        self._tokens = 0
        self._blocks: List[int] = []

    def append_token(self) -> None:
        if self._tokens % self._block_size == 0:
            self._blocks.append(self._allocator.allocate_block())
        self._tokens += 1

    def append_block(self, block_id: int) -> None:
        self._allocator._validate(block_id)
        self._blocks.append(block_id)

    def replace_block(self, old_block_id: int, new_block_id: int) -> None:
        self._allocator._validate(new_block_id)
        try:
            i = self._blocks.index(old_block_id)
        except ValueError:
            raise RuntimeError(f"Block ID {old_block_id} not found in block table") from None
        self._blocks[i] = new_block_id

    def release(self) -> None:
        for b in self._blocks:
            self._allocator.free_block(b)
        self._blocks = []
        self._tokens = 0

    def get_physical_blocks(self) -> List[int]:
        return list(self._blocks)

    def get_tokens_count(self) -> int:
        return self._tokens
