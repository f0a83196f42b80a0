"""What the engine and the KV manager need to know about one request.

The reference's scheduler owns a richer sequence type
(app/scheduler/sequence.py); the paged-attention path only reads a
request's id, its tokens and its block table, and appends generated tokens.
Any object with these attributes and methods works with the engine and
:class:`~..memory.manager.PagedKVCacheManager`.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional


@dataclass(eq=False)
class Request:
    seq_id: int
    prompt_token_ids: List[int]
    max_tokens: int = 128
    eos_token_id: Optional[int] = None
    deadline: Optional[float] = None
    output_token_ids: List[int] = field(default_factory=list)
    block_table: Optional[object] = None  # memory.block_allocator.SequenceBlockTable
    abandon_requested: bool = False
    finished: bool = False

    def __post_init__(self) -> None:
        self.prompt_token_ids = list(self.prompt_token_ids)
        if not self.prompt_token_ids:
            raise ValueError(f"Sequence {self.seq_id}: prompt_token_ids must not be empty")

    @property
    def total_len(self) -> int:
        """Tokens the request holds: its prompt and what it has generated."""
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    def get_len(self) -> int:
        return self.total_len

    def get_token_ids(self) -> List[int]:
        return [*self.prompt_token_ids, *self.output_token_ids]

    def append_token(self, token_id: int) -> None:
        """Record a generated token; the request is done at its end-of-sequence
        token or once it has max_tokens outputs."""
        self.output_token_ids.append(int(token_id))
        self.finished = self.finished or token_id == self.eos_token_id or \
            len(self.output_token_ids) >= self.max_tokens

    def is_finished(self) -> bool:
        return self.finished
