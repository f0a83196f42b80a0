"""The engine step that drives the paged-attention path.

Public surface of the reference's LLMEngine (app/engine/llm_engine.py:20-260):
the constructor ``(kv_cache_manager, scheduler, model_client=None,
model=None)``, ``add_request``, ``step``, ``has_unfinished_requests``,
``sweep_abandoned`` and ``model_device``.  The scheduler is any object with
the reference scheduler's ``add_sequence``, ``schedule()`` (returning
``scheduled_prefills`` / ``scheduled_decodes``, with slots already allocated
for the tokens it schedules), ``free_sequence``, ``has_unfinished_sequences``
and ``running`` / ``waiting`` lists; scheduling policy is outside this path.

What the step does differently, for the GPU:

  * one pass per step: the prefills (whole token lists from position 0) and
    the decodes (the last token at position tokens - 1) of a step form ONE
    PagedStepContext and ONE flat forward -- the reference runs a separate
    pass per group (llm_engine.py:237-248);
  * the LM head runs only on each sequence's last token
    (``logits_to_keep`` = cu_seqlens[1:] - 1 on the device), and the next
    tokens come from one on-device argmax and ONE device-to-host copy -- the
    reference takes ``int(logits[...].argmax())`` per sequence, a host sync
    each (llm_engine.py:200-204);
  * the attention hook is registered once with the backend select_backend
    names installed (the HIP backend on a ROCm device); the reference
    registers the hook but never selects a backend (llm_engine.py:169-173).
"""

from __future__ import annotations

import logging
import threading
import time
from typing import Dict, List, Optional, Sequence

import torch

from ..model.paged_attention import PagedStepContext, register_paged_attention, run_paged_forward
from .request import Request

logger = logging.getLogger(__name__)


class LLMEngine:
    def __init__(self, kv_cache_manager, scheduler, model_client=None, model=None) -> None:
        self.kv_cache_manager = kv_cache_manager
        self.scheduler = scheduler
        self.model_client = model_client
        self.model = model
        self.seq_counter = 0
        self._seq_counter_lock = threading.Lock()
        self._scheduler_lock = threading.Lock()
        self.update_event = None  # an asyncio.Event the server may set
        self._paged_attention_registered = False
        self.forward_passes = 0

    @property
    def model_device(self) -> torch.device:
        if self.model is None:
            return torch.device("cpu")
        first = next(iter(self.model.parameters()), None)
        return first.device if first is not None else torch.device("cpu")

    # -- requests ---------------------------------------------------------------
    def add_request(self, prompt_token_ids: List[int], max_tokens: int = 128, deadline: Optional[float] = None,
                    eos_token_id: Optional[int] = None) -> Request:
        with self._seq_counter_lock:
            self.seq_counter += 1
            seq_id = self.seq_counter
        seq = Request(seq_id, prompt_token_ids, max_tokens=max_tokens, eos_token_id=eos_token_id,
                      deadline=deadline)
        with self._scheduler_lock:
            self.scheduler.add_sequence(seq)
        return seq

    def sweep_abandoned(self) -> List:
        """Free every request that asked to be abandoned or is past its deadline."""
        with self._scheduler_lock:
            now = time.time()
            gone = [s for s in [*self.scheduler.running, *self.scheduler.waiting]
                    if s.abandon_requested or (s.deadline is not None and now >= s.deadline)]
            for seq in gone:
                self.scheduler.free_sequence(seq)
            return gone

    def has_unfinished_requests(self) -> bool:
        with self._scheduler_lock:
            return self.scheduler.has_unfinished_sequences()

    # -- the step ---------------------------------------------------------------
    def _ensure_paged_attention(self) -> None:
        if not self._paged_attention_registered:
            register_paged_attention(self.model)
            self._paged_attention_registered = True

    def forward_step(self, prefills: Sequence, decodes: Sequence) -> List[int]:
        """Next token of every sequence (prefills first, then decodes) from one
        flat forward over the whole step."""
        if self.model is None or not callable(getattr(self.model, "forward", None)):
            raise RuntimeError("the paged engine step needs a local model (the remote model client is "
                               "outside the paged-attention path)")
        self._ensure_paged_attention()
        sequences = [*prefills, *decodes]
        tokens: List[int] = []
        starts: List[int] = []
        counts: List[int] = []
        for seq in prefills:
            ids = seq.get_token_ids()
            tokens += ids
            starts.append(0)
            counts.append(len(ids))
        for seq in decodes:
            last = seq.output_token_ids[-1] if seq.output_token_ids else seq.prompt_token_ids[-1]
            tokens.append(last)
            starts.append(seq.block_table.get_tokens_count() - 1)
            counts.append(1)
        device = self.model_device
        flat = torch.tensor(tokens, dtype=torch.long)
        if device.type == "cuda":
            flat = flat.pin_memory().to(device, non_blocking=True)
        context = PagedStepContext(self.kv_cache_manager, sequences, starts, counts)
        cu = context.packed.cu_seqlens if context.packed is not None else context.cu_seqlens.to(device)
        with torch.inference_mode():
            logits = run_paged_forward(self.model, context, flat.unsqueeze(0), logits_to_keep=cu[1:] - 1)
            self.forward_passes += 1
            return logits[0].argmax(dim=-1).tolist()

    def step(self) -> Dict[str, List]:
        with self._scheduler_lock:
            try:
                outputs = self.scheduler.schedule()
            except RuntimeError as exc:
                logger.warning("Scheduler OOM, skipping step: %s", exc)
                return {"finished": [], "running": []}
            prefills = [s for s in outputs.scheduled_prefills if s.block_table is not None]
            decodes = [s for s in outputs.scheduled_decodes if s.block_table is not None]
            active = [*outputs.scheduled_prefills, *outputs.scheduled_decodes]
        if not prefills and not decodes:
            return {"finished": [], "running": []}
        for seq, token in zip([*prefills, *decodes], self.forward_step(prefills, decodes)):
            seq.append_token(token)
        with self._scheduler_lock:
            finished = [s for s in active if s.is_finished()]
            running = [s for s in active if not s.is_finished()]
            for seq in finished:
                self.scheduler.free_sequence(seq)
            if self.update_event is not None:
                self.update_event.set()
            return {"finished": finished, "running": running}
