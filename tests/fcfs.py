"""A first-come-first-served scheduler for driving the engine in tests.

Scheduling policy is outside the paged-attention path; this is the least a
scheduler must do for the engine (the contract of the reference's
app/scheduler/scheduler.py:84-150): every running request gets a slot for
its next token and is scheduled as a decode, every waiting request that
fits gets slots for all its tokens and is scheduled as a prefill.
"""

from dataclasses import dataclass, field
from typing import List


@dataclass
class Scheduled:
    scheduled_prefills: List = field(default_factory=list)
    scheduled_decodes: List = field(default_factory=list)


class FcfsScheduler:
    def __init__(self, manager, max_batch_size: int = 256):
        self.manager = manager
        self.max_batch_size = max_batch_size
        self.waiting: List = []
        self.running: List = []
        self.preemption_count = 0

    def add_sequence(self, seq) -> None:
        self.waiting.append(seq)

    def has_unfinished_sequences(self) -> bool:
        return bool(self.waiting or self.running)

    def free_sequence(self, seq) -> None:
        self.manager.free_sequence(seq)
        for q in (self.waiting, self.running):
            if seq in q:
                q.remove(seq)

    def schedule(self) -> Scheduled:
        out = Scheduled()
        for seq in self.running:
            self.manager.allocate_slot_for_next_token(seq)
            out.scheduled_decodes.append(seq)
        alloc = self.manager.get_allocator()
        while self.waiting and len(self.running) < self.max_batch_size:
            seq = self.waiting[0]
            need = -(-seq.total_len // self.manager.block_size)
            if need > alloc.get_num_free_blocks():
                break
            self.waiting.pop(0)
            self.manager.allocate_prefix_blocks(seq)
            self.running.append(seq)
            out.scheduled_prefills.append(seq)
        return out
