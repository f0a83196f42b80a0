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


class PreemptingScheduler(FcfsScheduler):
    """FcfsScheduler that also preempts, for tests of preempt-and-resume.

    * Out of blocks: a running request that needs a new block when none is
      free is preempted by recompute -- its blocks are freed and it goes back
      to the front of the waiting queue, so its next prefill covers prompt
      and outputs (the reference's policy, app/scheduler/scheduler.py:
      104-112; the engine prefills whole token lists).
    * ``plan`` = {schedule() call number: [(seq_id, "recompute" | "swap")]}
      forces preemptions: "recompute" as above (the request is re-admitted
      in the same call when it fits, so its freed table row is taken again
      before the step is packed); "swap" moves the request's blocks to the
      host pool (manager.swap_out) and, ``swap_steps`` calls later, back into
      fresh device blocks (manager.swap_in), after which it decodes on.  An
      entry whose request is not running then is tried again next call.
    """

    def __init__(self, manager, plan=None, swap_steps: int = 2, max_batch_size: int = 256):
        super().__init__(manager, max_batch_size)
        self.plan = {int(k): list(v) for k, v in (plan or {}).items()}
        self.swap_steps = swap_steps
        self.swapped: List = []  # (request, call number at which it swaps back in)
        self.calls = 0
        self.preempted = {"recompute": 0, "swap": 0, "oom": 0}

    def has_unfinished_sequences(self) -> bool:
        return bool(self.waiting or self.running or self.swapped)

    def free_sequence(self, seq) -> None:
        super().free_sequence(seq)
        self.swapped = [(s, t) for s, t in self.swapped if s is not seq]

    def _recompute(self, seq) -> None:
        self.manager.free_sequence(seq)
        self.waiting.insert(0, seq)
        self.preemption_count += 1

    def schedule(self) -> Scheduled:
        call = self.calls
        self.calls += 1
        later = []
        for seq_id, kind in self.plan.pop(call, []):
            seq = next((s for s in self.running if s.seq_id == seq_id), None)
            if seq is None:
                later.append((seq_id, kind))
                continue
            self.running.remove(seq)
            if kind == "recompute":
                self._recompute(seq)
            elif kind == "swap":
                self.manager.swap_out(seq)
                self.swapped.append((seq, call + self.swap_steps))
                self.preemption_count += 1
            else:
                raise ValueError(kind)
            self.preempted[kind] += 1
        if later:
            self.plan.setdefault(call + 1, []).extend(later)
        alloc = self.manager.get_allocator()
        still = []
        for seq, due in self.swapped:  # back in once due and its blocks fit
            if due <= call and len(seq.block_table.swapped_blocks) <= alloc.get_num_free_blocks():
                self.manager.swap_in(seq)
                self.running.append(seq)
            else:
                still.append((seq, due))
        self.swapped = still

        out = Scheduled()
        kept = []
        for seq in self.running:
            tokens = seq.block_table.get_tokens_count()
            if tokens % self.manager.block_size == 0 and alloc.get_num_free_blocks() < 1:
                self._recompute(seq)
                self.preempted["oom"] += 1
                continue
            self.manager.allocate_slot_for_next_token(seq)
            out.scheduled_decodes.append(seq)
            kept.append(seq)
        self.running = kept
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
