"""Serving metrics of the paged-attention path: per-layer attention latency,
algorithmic KV-read GB/s and tokens/s, in the plain-text exposition format
of the reference's ``/metrics`` endpoint (app/api/server.py:275-310).

Timing never synchronises the host: every recorded call brackets the
attention launches with two HIP events on the launch stream, and
:meth:`AttentionMetrics.poll` folds in only the events that have already
completed (``Event.query()``), so a serving loop can render metrics at any
time without stalling the GPU.  Recording is off unless enabled
(:func:`enable` or ``LLM_PAGED_METRICS=1``).
"""

from __future__ import annotations

import collections
import os
import threading
from dataclasses import dataclass
from typing import Deque, List, Optional

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


@dataclass
class _Pending:
    start: object
    stop: object
    nbytes: int
    tokens: int


class AttentionMetrics:
    """Aggregates of the attention launches recorded so far."""

    def __init__(self, ema: float = 0.1, max_pending: int = 4096) -> None:
        self.ema = ema
        self.max_pending = max_pending
        self._pending: Deque[_Pending] = collections.deque()
        self._lock = threading.Lock()
        self.calls = 0
        self.dropped = 0
        self.total_ms = 0.0
        self.total_bytes = 0
        self.total_tokens = 0
        self.last_ms: Optional[float] = None
        self.avg_ms: Optional[float] = None
        self.last_gbps: Optional[float] = None

    # -- recording ---------------------------------------------------------
    def begin(self, stream=None):
        import torch

        ev = torch.cuda.Event(enable_timing=True)
        ev.record(stream)
        return ev

    def end(self, start, nbytes: int, tokens: int, stream=None) -> None:
        import torch

        stop = torch.cuda.Event(enable_timing=True)
        stop.record(stream)
        self.add(start, stop, nbytes, tokens)

    def add(self, start, stop, nbytes: int, tokens: int) -> None:
        """Queue a pair of recorded events (anything with ``query()`` and
        ``elapsed_time()``) for one attention call."""
        with self._lock:
            if len(self._pending) >= self.max_pending:
                self._pending.popleft()
                self.dropped += 1
            self._pending.append(_Pending(start, stop, int(nbytes), int(tokens)))

    # -- aggregation -------------------------------------------------------
    def poll(self) -> int:
        """Fold in every completed call, oldest first; returns how many."""
        done = 0
        with self._lock:
            while self._pending and self._pending[0].stop.query():
                p = self._pending.popleft()
                ms = float(p.start.elapsed_time(p.stop))
                self.calls += 1
                self.total_ms += ms
                self.total_bytes += p.nbytes
                self.total_tokens += p.tokens
                self.last_ms = ms
                self.avg_ms = ms if self.avg_ms is None else (1 - self.ema) * self.avg_ms + self.ema * ms
                self.last_gbps = p.nbytes / (ms * 1e-3) / 1e9 if ms > 0 else None
                done += 1
        return done

    @property
    def pending(self) -> int:
        return len(self._pending)

    def lines(self) -> List[str]:
        self.poll()
        gbps = self.total_bytes / (self.total_ms * 1e-3) / 1e9 if self.total_ms > 0 else 0.0
        tps = self.total_tokens / (self.total_ms * 1e-3) if self.total_ms > 0 else 0.0
        return [
            f"paged_attention_calls_total {self.calls}",
            f"paged_attention_latency_ms_last {self.last_ms or 0.0}",
            f"paged_attention_latency_ms_avg {self.avg_ms or 0.0}",
            f"paged_attention_kv_read_gbps_last {self.last_gbps or 0.0}",
            f"paged_attention_kv_read_gbps {gbps}",
            f"paged_attention_hbm_peak_fraction {gbps / HBM_PEAK_GBS}",
            f"paged_attention_tokens_per_second {tps}",
            f"paged_attention_pending_events {self.pending}",
            f"paged_attention_dropped_events_total {self.dropped}",
        ]


def step_bytes(context_lens, num_query_tokens: int, num_query_heads: int, num_kv_heads: int, head_dim: int,
               element_bytes: int, block_size: int) -> int:
    """Algorithmic HBM bytes of one layer's attention over a step: K and V of
    every context token once per KV head, the query and output rows, the
    block-table entries and the context lengths."""
    ctx = [int(c) for c in context_lens]
    kv = sum(ctx) * 2 * num_kv_heads * head_dim * element_bytes
    qo = int(num_query_tokens) * num_query_heads * head_dim * 2 * element_bytes
    tables = sum(-(-c // block_size) for c in ctx) * 4
    return kv + qo + tables + 4 * len(ctx)


def cache_lines(manager=None, scheduler=None) -> List[str]:
    """The reference's three KV-cache lines (app/api/server.py:277-306)."""
    free, total = 0, 1
    if manager is not None and hasattr(manager, "get_allocator"):
        try:
            alloc = manager.get_allocator()
            free = alloc.get_num_free_blocks()
            total = alloc.get_total_blocks()
        except Exception:
            free, total = 0, 1
    elif manager is None:
        free, total = 1, 1
    ratio = (free / total) if total else 0.0
    active = len(getattr(scheduler, "running", [])) if scheduler is not None else 0
    preemptions = getattr(scheduler, "preemption_count", 0) if scheduler is not None else 0
    return [
        f"kv_cache_free_pages_ratio {float(ratio)}",
        f"kv_cache_active_streams {active}",
        f"kv_cache_preemptions_total {preemptions}",
    ]


_METRICS: Optional[AttentionMetrics] = None


def enable(metrics: Optional[AttentionMetrics] = None) -> AttentionMetrics:
    """Start recording attention launches (returns the collector)."""
    global _METRICS
    _METRICS = metrics or AttentionMetrics()
    return _METRICS


def disable() -> None:
    global _METRICS
    _METRICS = None


def current() -> Optional[AttentionMetrics]:
    """The active collector, if recording is on (enabled explicitly or by
    LLM_PAGED_METRICS=1 in the environment)."""
    global _METRICS
    if _METRICS is None and os.environ.get("LLM_PAGED_METRICS", "0") == "1":
        _METRICS = AttentionMetrics()
    return _METRICS


def metrics_text(manager=None, scheduler=None) -> str:
    """Body of a ``/metrics`` response: the reference's KV-cache lines plus
    the attention lines when recording is on."""
    lines = cache_lines(manager, scheduler)
    m = current()
    if m is not None:
        lines += m.lines()
    return "\n".join(lines) + "\n"
