"""Torch-facing wrappers of the HIP paged-attention kernels.

Every function here takes device tensors, launches on the current HIP stream
of that device (``torch.cuda.current_stream()``) and never synchronises.
They fail loudly: a missing library, a CPU tensor or a shape the kernels
reject raises instead of falling back to another implementation.

The four jobs of the path:
  (a) :func:`pack_step`          ragged-batch packing (cu_seqlens, slots, work lists)
  (b) :func:`reshape_and_cache`  new K/V rows -> paged cache
  (c) :func:`decode`             split-K paged decode
  (d) :func:`prefill`            causal chunked prefill (MFMA)
plus :func:`attention` (decode + prefill of one flattened step) and
:func:`paged_attention_flat`, the reference C-ABI call over device tensors.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _native
from ._native import PA_DECODE_MAX_PARTITION

_DTYPES = {
    torch.float32: _native.PA_DTYPE_F32,
    torch.bfloat16: _native.PA_DTYPE_BF16,
    torch.float16: _native.PA_DTYPE_F16,
}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dtype for the HIP path: {dtype}") from exc


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_device(*tensors: torch.Tensor) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"HIP paged-attention kernels need device tensors, got a tensor on {t.device}"
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"tensors on different devices: {device} and {t.device}")
    if device is None:
        raise RuntimeError("no device tensor given")
    return device


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def prefill_tile_for(num_query_heads: int, num_kv_heads: int) -> int:
    """Query tokens per prefill work item: the tile the MFMA prefill kernel
    takes (128 query rows over one workgroup's heads; pa_prefill_tile)."""
    lib = _native.load_library()
    return int(lib.pa_prefill_tile(int(num_query_heads), int(num_kv_heads))) or 128


# ---------------------------------------------------------------------------
# (a) packing


_INT32_MAX = (1 << 31) - 1


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


_ELEM = {torch.int64: 8, torch.int32: 4, torch.uint8: 1}


class _Layout:
    """Byte offsets of named arrays inside one buffer (256-byte aligned)."""

    def __init__(self) -> None:
        self.fields = {}
        self.nbytes = 0

    def add(self, name: str, dtype: torch.dtype, shape) -> None:
        count = 1
        for d in shape:
            count *= d
        self.fields[name] = (self.nbytes, dtype, shape)
        self.nbytes += _align(count * _ELEM[dtype])


class _HostStaging:
    """A ring of pinned host buffers the packing kernel reads a step's inputs
    from (through their device addresses, pa_map_host_memory), so no copy
    launch precedes it.

    The ring's 16 slots form two halves.  Entering a half, the host records
    an event on every stream that launched from the other half (all of those
    launches are enqueued by then), and waits for the events recorded the
    last time it entered the other half, which follow every launch that
    read this half.  So the host never overwrites bytes a pending launch
    still reads, whatever streams the launches went to, and in the steady
    state it never waits.  Recording events once per 8 steps instead of once
    per step matters: every event record puts a few microseconds of idle
    time between two kernels."""

    SLOTS = 16
    HALF = SLOTS // 2

    def __init__(self) -> None:
        self._bufs = [None] * self.SLOTS
        self._arrays = [None] * self.SLOTS
        self._device = [0] * self.SLOTS
        self._streams = [{}, {}]  # per half: the streams its launches went to (by handle)
        self._events = [[], []]  # per half: events that follow every launch reading it
        self._next = 0

    def take(self, nbytes: int):
        """(slot, numpy view, device address) of a free buffer of >= nbytes."""
        slot = self._next
        self._next = (slot + 1) % self.SLOTS
        if slot % self.HALF == 0:  # entering a half
            half, other = slot // self.HALF, 1 - slot // self.HALF
            marks = []
            for stream in self._streams[other].values():
                ev = torch.cuda.Event()
                ev.record(stream)
                marks.append(ev)
            self._events[other] = marks
            self._streams[other] = {}
            for ev in self._events[half]:
                ev.synchronize()
            self._events[half] = []
        buf = self._bufs[slot]
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(_align(nbytes, 1 << 16), 1 << 16), dtype=torch.uint8, pin_memory=True)
            lib = _native.load_library()
            dev = ctypes.c_void_p()
            _native.check(lib.pa_map_host_memory(buf.data_ptr(), ctypes.byref(dev)), "pa_map_host_memory")
            self._bufs[slot], self._arrays[slot], self._device[slot] = buf, buf.numpy(), int(dev.value)
        return slot, self._arrays[slot], self._device[slot]

    def done(self, slot: int, stream) -> None:
        """The launch reading ``slot`` is enqueued on ``stream``."""
        self._streams[slot // self.HALF].setdefault(stream.cuda_stream, stream)


_STAGING: dict = {}  # device -> _HostStaging
_CUS: dict = {}  # device index -> compute units


def _staging(device: torch.device) -> _HostStaging:
    key = device.index
    st = _STAGING.get(key)
    if st is None:
        st = _STAGING[key] = _HostStaging()
    return st


def _compute_units(device: torch.device) -> int:
    n = _CUS.get(device.index)
    if n is None:
        n = _CUS[device.index] = int(torch.cuda.get_device_properties(device).multi_processor_count)
    return n


class PackedStep:
    """Device-side description of one flattened ragged step (what pa_pack
    writes), in one device allocation.

    Every array is a view of ``buffer``, materialised on first access; the
    kernels are launched from the raw addresses (:meth:`ptr`), so a step
    costs one allocation and no per-array tensor objects on the hot path.
    Host-side counts come from the host planner (pa_plan_step), so no
    device-to-host synchronisation sizes the grids.

    Arrays: cu_seqlens / cu_context_offsets int64 [B+1], context_lens int32
    [B], scatter_slots / position_ids int64 [T], decode_items int32 [n, 2],
    merge_items int32 [n, 4], prefill_items int32 [n, 2]; gather_slots int64
    [C] is built on first use.  A step packed from a pool of table rows also
    has rows int32 [B] (each sequence's row): the attention kernels read the
    pool in place through it.  block_tables int32 [B, width] is the step's
    table: the caller's own, the pool rows pa_pack copied (``step_table``),
    or else gathered from the pool when first read (a convenience view, not
    used by the kernels).  start_positions / new_token_counts are the host
    arrays of the step.
    """

    def __init__(self, buffer, layout, plan, block_size, prefill_tile, table, table_rows, pooled,
                 head_shape, inputs):
        self.buffer = buffer
        self._layout = layout
        self._base = buffer.data_ptr()
        self.block_size = int(block_size)
        self.partition_size = int(plan.partition_size)
        self.prefill_tile = int(prefill_tile)
        self._inputs = inputs  # host (starts int64, counts int64, rows int32 or None)
        self.num_seqs = int(inputs[0].shape[0])
        self.num_query_tokens = int(plan.num_query_tokens)
        self.num_context_tokens = int(plan.num_context_tokens)
        self.num_decode_items = int(plan.num_decode_items)
        self.num_merge_items = int(plan.num_merge_items)
        self.num_prefill_items = int(plan.num_prefill_items)
        self.num_decode_seqs = int(plan.num_decode_seqs)
        self.num_prefill_seqs = int(plan.num_prefill_seqs)
        self.max_context = int(plan.max_context)
        self.max_new_tokens = int(plan.max_new_tokens)
        self._max_blocks = int(plan.max_blocks)
        self._source_table = table  # the table pa_pack and the kernels read (the step's own, or a pool)
        self._source_rows = table_rows
        self._pooled = bool(pooled)
        self._head_shape = head_shape  # (H_q, D) the workspace was sized for, or None
        self._gather = None
        self._extra_ws = None
        self._generation = 0  # the pool's pack count when this step was packed
        self._merge_state_bytes = 0  # merge records at the end of the decode workspace

    # -- addresses and views ---------------------------------------------------
    def ptr(self, name: str) -> int:
        """Device address of an array; "block_tables" is the table the
        kernels read (the caller's table or the pool)."""
        if name == "block_tables":
            return self._source_table.data_ptr()
        return self._base + self._layout.fields[name][0]

    def _view(self, name: str) -> torch.Tensor:
        off, dtype, shape = self._layout.fields[name]
        count = 1
        for d in shape:
            count *= d
        t = self.buffer[off : off + count * _ELEM[dtype]].view(dtype).view(shape)
        self.__dict__[name] = t
        return t

    def __getattr__(self, name: str):
        layout = self.__dict__.get("_layout")
        if layout is None:
            raise AttributeError(name)
        if name in layout.fields:
            return self._view(name)
        if name == "block_tables":
            if not self.__dict__["_pooled"]:
                return self.__dict__["_source_table"]
            table = self._gathered_table()
            self.__dict__[name] = table
            return table
        raise AttributeError(name)

    def _gathered_table(self) -> torch.Tensor:
        """[B, max_blocks] rows of the pool for the step's sequences (-1 for a
        row outside the pool and past the pool's width)."""
        src = self._source_table
        width = max(self._max_blocks, 1)
        out = torch.full((self.num_seqs, width), -1, dtype=torch.int32, device=self.buffer.device)
        if self.num_seqs == 0 or src.numel() == 0:
            return out
        rows = self.rows.long()
        ok = (rows >= 0) & (rows < self._source_rows)
        n = min(width, int(src.shape[1]))
        out[ok, :n] = src.index_select(0, rows[ok])[:, :n]
        return out

    @property
    def start_positions(self) -> np.ndarray:
        """int64 [B] (host) start position of every sequence."""
        return self._inputs[0]

    @property
    def new_token_counts(self) -> np.ndarray:
        """int64 [B] (host) new tokens of every sequence."""
        return self._inputs[1]

    def repack(self, start_positions=None, new_token_counts=None) -> None:
        """Rerun the packing kernels in place with new positions / counts of
        the same sequences (what a step captured in a graph re-reads): every
        output keeps its address.  The new step must need the same buffer
        sizes (tokens, contexts and work items)."""
        starts = self._inputs[0] if start_positions is None else _int64_array(start_positions)
        counts = self._inputs[1] if new_token_counts is None else _int64_array(new_token_counts)
        plan = _plan(starts, counts, self.block_size, self.prefill_tile, self.partition_size, 1, 1, 1, 1, 1)
        same = (plan.num_query_tokens, plan.num_decode_items, plan.num_merge_items, plan.num_prefill_items) == (
            self.num_query_tokens, self.num_decode_items, self.num_merge_items, self.num_prefill_items)
        if starts.shape[0] != self.num_seqs or not same:
            raise ValueError("repack needs a step of the same sizes; pack a new step instead")
        if self.table_width and plan.max_blocks > self.table_width:
            raise ValueError("repack: a context grew past the step's block table")
        self._inputs = (starts, counts, self._inputs[2])
        self.num_context_tokens = int(plan.num_context_tokens)
        self.max_context = int(plan.max_context)
        self._gather = None
        _run_pack(self, fresh=True)

    def rerun(self) -> None:
        """Rerun the packing kernels on the inputs the last pack or repack of
        this step left in its workspace: no host memory is read and nothing
        is allocated, so a serving loop can capture it in a HIP graph ahead
        of the layers and change the step with :meth:`repack` between
        replays."""
        _run_pack(self)

    @property
    def table_width(self) -> int:
        """Row stride of the table the kernels read."""
        return int(self._source_table.shape[1]) if self._source_table.dim() == 2 else 0

    @property
    def gather_slots(self) -> torch.Tensor:
        """int64 [C] slots of every context token (built on first use, by a
        re-run of the packing kernel over the table as it is now).  On a pool
        of rows it must be first read before the next step is packed on the
        same pool: a later step's updates (a row freed and reused) would
        change what the re-run reads, so a stale step raises instead."""
        if self._gather is None:
            if self._pooled and _pack_generation(self._source_table) != self._generation:
                raise RuntimeError("gather_slots of an earlier step: a later step was packed on the same "
                                   "block-table pool since; read gather_slots before packing the next step")
            self._gather = _run_pack(self, with_gather=True)
        return self._gather

    def workspace_ptr(self, dims: _native.PaStepDims) -> Tuple[int, int]:
        """(address, bytes) of the decode workspace of a launch with these
        dims, reused across the layers of the step (calls that share it must
        not overlap in time): the step's own region when it was sized for
        these head counts and holds what pa_decode needs, else a zeroed one
        kept for the step (the merge records at its end must start at zero;
        every launch leaves them zero)."""
        lib = _native.load_library()
        need = int(lib.pa_decode_workspace_size(dims, self.num_decode_items))
        if self._head_shape == (int(dims.num_query_heads), int(dims.head_dim)):
            off, _, shape = self._layout.fields["decode_workspace"]
            if shape[0] >= need:
                return self._base + off, shape[0]
        ws = self._extra_ws
        if ws is None or ws.numel() < need:
            ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=self.buffer.device)
            self._extra_ws = ws
        return ws.data_ptr(), ws.numel()

    def _merge_state_region(self) -> Tuple[Optional[int], int]:
        """(address, bytes) of the merge records of the step's own decode
        workspace, which pa_pack clears, or (None, 0)."""
        if self._merge_state_bytes <= 0:
            return None, 0
        off, _, shape = self._layout.fields["decode_workspace"]
        return self._base + off + shape[0] - self._merge_state_bytes, self._merge_state_bytes


def _plan(starts: np.ndarray, counts: np.ndarray, block_size: int, prefill_tile: int, partition_size: int,
          num_kv_heads: int, num_query_heads: int, workgroups_per_item: int, workgroups_per_cu: int,
          compute_units: int, allocated: Optional[np.ndarray] = None):
    lib = _native.load_library()
    params = _native.PaPlanParams(block_size=int(block_size), prefill_tile=int(prefill_tile),
                                  partition_size=int(partition_size), num_kv_heads=int(num_kv_heads),
                                  num_query_heads=int(num_query_heads),
                                  workgroups_per_item=int(workgroups_per_item),
                                  workgroups_per_cu=int(workgroups_per_cu), compute_units=int(compute_units))
    plan = _native.PaStepPlan()
    status = lib.pa_plan_step(starts.ctypes.data, counts.ctypes.data,
                              None if allocated is None else allocated.ctypes.data,
                              int(starts.shape[0]), params, ctypes.byref(plan))
    if status != _native.PA_OK:
        if plan.bad_seq >= 0:
            raise ValueError(lib.pa_last_error_message().decode(errors="replace"))
        _native.check(status, "pa_plan_step")
    return plan


def _int64_array(values) -> np.ndarray:
    if isinstance(values, np.ndarray) and values.dtype == np.int64 and values.flags.c_contiguous:
        return values
    return np.ascontiguousarray(np.asarray(values, dtype=np.int64).reshape(-1))


def work_counts(
    start_positions: Sequence[int],
    new_token_counts: Sequence[int],
    partition_size: int,
    prefill_tile: int,
):
    """Host-side sizes of a step (pa_plan_step):
    (T, C, decode items, merge items, prefill items, #decode seqs, #prefill seqs)."""
    p = _plan(_int64_array(start_positions), _int64_array(new_token_counts), 1, prefill_tile, partition_size,
              1, 1, 1, 1, 1)
    return (int(p.num_query_tokens), int(p.num_context_tokens), int(p.num_decode_items), int(p.num_merge_items),
            int(p.num_prefill_items), int(p.num_decode_seqs), int(p.num_prefill_seqs))


# Compute units of an MI355X; pack_step uses the device's own count.
_DECODE_CUS = 256


def decode_workgroups_per_item(dtype: torch.dtype, head_dim: int, num_kv_heads: int,
                               num_query_heads: int) -> int:
    """Partition workgroups the decode launches per work item: half the KV
    heads when adjacent heads run as pairs, KV heads x sub-groups for groups
    of more than 8 query heads, else the KV heads (0 for rejected counts)."""
    lib = _native.load_library()
    return int(lib.pa_decode_workgroups_per_item(dtype_code(dtype), int(head_dim), int(num_kv_heads),
                                                 int(num_query_heads)))


# (library, device, shape) -> workgroups per CU: the occupancy query is a
# function of the kernel and the device only, and pack_step runs every step.
_OCCUPANCY_CACHE: dict = {}


def decode_workgroups_per_cu(dtype: torch.dtype, head_dim: int, num_kv_heads: int,
                             num_query_heads: int) -> int:
    """Decode workgroups of this shape one compute unit of the current device
    holds at once (the occupancy of the kernel pa_decode launches; 0 for a
    shape without a tuned kernel).  Cached per library, device and shape."""
    lib = _native.load_library()
    key = (id(lib), torch.cuda.current_device(), dtype, int(head_dim), int(num_kv_heads), int(num_query_heads))
    per_cu = _OCCUPANCY_CACHE.get(key)
    if per_cu is None:
        per_cu = int(lib.pa_decode_workgroups_per_cu(dtype_code(dtype), int(head_dim), int(num_kv_heads),
                                                     int(num_query_heads)))
        _OCCUPANCY_CACHE[key] = per_cu
    return per_cu


def _occupancy_on(device: torch.device, dtype, head_dim: int, num_kv_heads: int, num_query_heads: int) -> int:
    """decode_workgroups_per_cu for ``device`` (made current only for a miss)."""
    key = (id(_native.load_library()), device.index, dtype, int(head_dim), int(num_kv_heads), int(num_query_heads))
    per_cu = _OCCUPANCY_CACHE.get(key)
    if per_cu is None:
        with torch.cuda.device(device):
            per_cu = decode_workgroups_per_cu(dtype, head_dim, num_kv_heads, num_query_heads)
    return per_cu


def choose_partition(
    start_positions: Sequence[int],
    new_token_counts: Sequence[int],
    num_kv_heads: int = 8,
    num_query_heads: Optional[int] = None,
    workgroups_per_item: Optional[int] = None,
    workgroups_per_cu: Optional[int] = None,
    compute_units: int = _DECODE_CUS,
) -> int:
    """Split-K partition for the decode sequences of a step (the rule of
    pa_plan_step, which runs it on the host in C++).

    The largest of 4096, 2048, 1024, 512 and 256 tokens whose decode launch
    (partitions x workgroups_per_item, by default the KV heads) still gives every
    resident workgroup slot of the chip (compute_units x workgroups_per_cu;
    without the occupancy, five per CU for one query head per KV head and
    four for groups) one and a half workgroups: long partitions keep the
    number of partials, merges and per-workgroup set-ups low, and pa_pack
    orders the work longest first so the short remainders fill the end of
    the launch.  On 256 lognormal contexts (median 1024) the rule picks the
    fastest partition of every measured shape: 4096 for 32/8 heads of 128,
    2048 for the same heads paired (three workgroups per CU), 1024 for 8/8.

    A step too small for that rule (a latency-bound step) takes the one of
    64 ... 4096 with the least modelled time, measured on 32-layer decode
    loops whose caches are read cold: a workgroup reads about 21 GB/s on
    its own (0.049 us per token of a 1 KB K+V row) and about 310 of them
    saturate HBM, so the longest workgroup takes P x 0.049 us x (its share
    of HBM when more run at once) x (waves of workgroups); the merge of the
    longest sequence adds 2 us per batch of 8 partials.  Ties go to the
    shorter partition.  Over 22 measured steps (1-64 sequences of 256 to
    16384 tokens, bf16 and fp32, groups of 4 and 8) the pick is the fastest
    partition on 17 and within 9.2 % on the rest; e.g. two sequences of 8192
    tokens 26.7 us per layer at 256 (the earlier rule's 128: 29.7).
    """
    p = _plan(_int64_array(start_positions), _int64_array(new_token_counts), 1, 1, 0, num_kv_heads,
              num_query_heads or 0, workgroups_per_item or 0, workgroups_per_cu or 0, compute_units)
    return int(p.partition_size)


def _pack_generation(table: torch.Tensor) -> int:
    """Fresh packs so far on a block-table pool (a tensor attribute)."""
    return getattr(table, "_pa_pack_generation", 0)


def _run_pack(step: PackedStep, with_gather: bool = False, updates: Optional[np.ndarray] = None,
              fresh: bool = False) -> Optional[torch.Tensor]:
    """Launch pa_pack for ``step``: all outputs are rewritten, plus the gather
    slots when asked for (returned).  ``fresh``: the step's host inputs (and
    ``updates``) are staged in pinned host memory the scan kernel reads;
    otherwise the kernel re-reads its own copy of them in the step's
    workspace (no host memory involved, so the call can be graph-captured)."""
    lib = _native.load_library()
    device = step.buffer.device
    gather = None
    if with_gather:
        gather = torch.empty(step.num_context_tokens, dtype=torch.int64, device=device)
    starts, counts, rows = step._inputs
    b = step.num_seqs
    pooled = step._pooled
    n_upd = 0 if updates is None else int(updates.shape[0])
    staging = slot = None
    dev = o_counts = o_rows = o_upd = 0
    if fresh or n_upd:
        o_counts = _align(8 * b, 64)
        o_rows = o_counts + _align(8 * b, 64)
        o_upd = o_rows + (_align(4 * b, 64) if pooled else 0)
        nbytes = o_upd + 12 * n_upd
        staging = _staging(device)
        slot, host, dev = staging.take(max(nbytes, 1))
        host[:o_counts].view(np.int64)[:b] = starts
        host[o_counts:o_rows].view(np.int64)[:b] = counts
        if pooled:
            host[o_rows : o_rows + 4 * b].view(np.int32)[:] = rows
        if n_upd:
            host[o_upd:nbytes].view(np.int32)[:] = updates.reshape(-1)
    table = step._source_table
    step_table = step._layout.fields.get("block_tables")
    dims = _native.PaPackDims(
        num_seqs=b,
        block_size=step.block_size,
        max_blocks_per_seq=step.table_width,
        partition_size=step.partition_size,
        prefill_tile=step.prefill_tile,
        num_table_rows=step._source_rows,
        num_updates=n_upd,
        step_table_width=step_table[2][1] if step_table else 0,
        max_new_tokens=min(step.max_new_tokens, _INT32_MAX),
        max_context=min(step.max_context, _INT32_MAX),
        max_query_tokens=step.num_query_tokens,
        max_context_tokens=step.num_context_tokens,
        max_decode_items=step.num_decode_items,
        max_merge_items=step.num_merge_items,
        max_prefill_items=step.num_prefill_items,
    )
    ws_off, _, ws_shape = step._layout.fields["pack_workspace"]
    clear, clear_bytes = step._merge_state_region()
    status = lib.pa_pack(
        table.data_ptr() if table.numel() else None,
        dev + o_rows if pooled and dev else None,
        dev + o_upd if n_upd else None,
        dev or None,
        dev + o_counts if dev else None,
        dims,
        step._base + step_table[0] if step_table else None,
        step.ptr("rows") if pooled else None,
        step.ptr("cu_seqlens"),
        step.ptr("cu_context_offsets"),
        step.ptr("context_lens"),
        step.ptr("scatter_slots"),
        step.ptr("position_ids"),
        _ptr(gather),
        step.ptr("decode_items"),
        step.ptr("merge_items"),
        step.ptr("prefill_items"),
        clear,
        clear_bytes,
        step._base + ws_off,
        ws_shape[0],
        _stream(device),
    )
    if staging is not None:
        staging.done(slot, torch.cuda.current_stream(device))
    _native.check(status, "pa_pack")
    if fresh and pooled:
        table._pa_pack_generation = _pack_generation(table) + 1
        step._generation = table._pa_pack_generation
    return gather


def pack_step(
    block_tables: torch.Tensor,
    start_positions: Sequence[int],
    new_token_counts: Sequence[int],
    block_size: int,
    *,
    prefill_tile: Optional[int] = None,
    partition_size: Optional[int] = None,
    num_kv_heads: int = 8,
    num_query_heads: Optional[int] = None,
    head_dim: Optional[int] = None,
    dtype: Optional[torch.dtype] = None,
    with_gather: bool = False,
    rows=None,
    updates: Optional[np.ndarray] = None,
    allocated_tokens=None,
    step_table: bool = False,
) -> PackedStep:
    """Plan a step on the host, upload its description once, and run the GPU
    packing kernels.

    ``block_tables``: int32 [B, max_blocks] device tensor (-1 padded), the
    step's own table; or, with ``rows`` (one row index per sequence), a
    device-resident pool of table rows that pa_pack first applies
    ``updates`` (int32 [n, 3] (row, col, block) triples, host array) to, and
    that the attention kernels then read in place through the step's
    ``rows``.  ``step_table``: also have pa_pack copy the step's rows of
    the pool into a table of its own (``PackedStep.block_tables``).
    ``start_positions`` / ``new_token_counts``: the host lists of the step.
    ``allocated_tokens``: per sequence, the tokens it has slots for; a step
    reaching past them is a ValueError (as the reference's slot mapping).
    ``partition_size``: decode split-K partition in tokens; by default the
    planner picks it from the step and the head counts (and, when
    ``head_dim`` and the cache ``dtype`` are given, from how many KV heads
    one decode workgroup reads and the kernel's occupancy).
    ``prefill_tile``: query tokens per prefill work item; by default the
    MFMA kernel's tile for the head counts (:func:`prefill_tile_for`).
    With ``head_dim`` given, the decode workspace for the query heads is
    part of the step's one allocation.
    """
    device = _require_device(block_tables)
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2:
        raise ValueError("block_tables must be an int32 [B, max_blocks] tensor")
    if not block_tables.is_contiguous():
        raise ValueError("block_tables must be contiguous")
    starts = _int64_array(start_positions)
    counts = _int64_array(new_token_counts)
    b = int(starts.shape[0])
    if counts.shape[0] != b:
        raise ValueError("start_positions / new_token_counts must have one entry per sequence")
    if rows is None and b != int(block_tables.shape[0]):
        raise ValueError("start_positions / new_token_counts must have one entry per block-table row")
    hq = int(num_query_heads or 4 * num_kv_heads)
    if prefill_tile is None:
        prefill_tile = prefill_tile_for(hq, int(num_kv_heads))
    if prefill_tile <= 0:
        raise ValueError("prefill_tile must be positive")
    if partition_size is not None and partition_size <= 0:
        raise ValueError("partition_size must be positive")
    per_item = per_cu = 0
    if partition_size is None and head_dim is not None and dtype is not None:
        per_item = decode_workgroups_per_item(dtype, head_dim, num_kv_heads, hq)
        per_cu = _occupancy_on(device, dtype, head_dim, num_kv_heads, hq)
    allocated = None if allocated_tokens is None else _int64_array(allocated_tokens)
    plan = _plan(starts, counts, block_size, prefill_tile, partition_size or 0, num_kv_heads, hq, per_item,
                 per_cu, _compute_units(device), allocated)
    pooled = rows is not None
    n_upd = 0 if updates is None else int(updates.shape[0])

    # One device buffer per step; the inputs go over in pinned host memory.
    layout = _Layout()
    t, c = int(plan.num_query_tokens), int(plan.num_context_tokens)
    if pooled:
        layout.add("rows", torch.int32, (b,))
        if step_table:
            layout.add("block_tables", torch.int32, (b, max(int(plan.max_blocks), 1)))
    layout.add("cu_seqlens", torch.int64, (b + 1,))
    layout.add("cu_context_offsets", torch.int64, (b + 1,))
    layout.add("context_lens", torch.int32, (b,))
    layout.add("scatter_slots", torch.int64, (t,))
    layout.add("position_ids", torch.int64, (t,))
    layout.add("decode_items", torch.int32, (int(plan.num_decode_items), 2))
    layout.add("merge_items", torch.int32, (int(plan.num_merge_items), 4))
    layout.add("prefill_items", torch.int32, (int(plan.num_prefill_items), 2))
    lib = _native.load_library()
    layout.add("pack_workspace", torch.uint8, (int(lib.pa_pack_workspace_size(b)),))
    head_shape = None
    ws_bytes = state_bytes = 0
    if head_dim is not None:
        head_shape = (hq, int(head_dim))
        # An unknown cache dtype is sized as fp32, whose unpaired KV heads
        # need the most merge records.
        ws_dims = _native.PaStepDims(num_seqs=b, num_query_heads=hq, num_kv_heads=int(num_kv_heads),
                                     head_dim=int(head_dim), dtype=dtype_code(dtype or torch.float32))
        ws_bytes = int(lib.pa_decode_workspace_size(ws_dims, int(plan.num_decode_items)))
        state_bytes = int(lib.pa_decode_merge_state_size(ws_dims, int(plan.num_decode_items)))
        layout.add("decode_workspace", torch.uint8, (max(ws_bytes, 1),))
    buffer = torch.empty(layout.nbytes, dtype=torch.uint8, device=device)
    rows_arr = None if rows is None else np.ascontiguousarray(np.asarray(rows, dtype=np.int32).reshape(-1))
    table_rows = int(block_tables.shape[0]) if block_tables.numel() else 0
    step = PackedStep(buffer, layout, plan, block_size, prefill_tile, block_tables, table_rows, pooled,
                      head_shape, (starts, counts, rows_arr))
    step._merge_state_bytes = state_bytes  # cleared by every pa_pack of the step
    upd = None if not n_upd else np.ascontiguousarray(updates, dtype=np.int32)
    gather = _run_pack(step, with_gather=with_gather, updates=upd, fresh=True)
    if with_gather:
        step._gather = gather
    return step


# ---------------------------------------------------------------------------
# (b) cache write


def reshape_and_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    layer_idx: int,
) -> None:
    """key_cache[layer].view(-1, H_kv, D)[slot_mapping] = key (and value), on the GPU.

    ``key`` / ``value``: [T, H_kv, D] (any token / head strides, unit stride on D);
    caches: (L, N, bs, H_kv, D) contiguous; ``slot_mapping``: int64 [T].
    """
    device = _require_device(key, value, key_cache, value_cache, slot_mapping)
    if key_cache.dim() != 5 or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be 5-D (layers, blocks, block_size, heads, dim) and alike")
    if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    num_layers, total_blocks, block_size, num_kv_heads, head_dim = key_cache.shape
    if key.shape != value.shape or key.dim() != 3 or tuple(key.shape[1:]) != (num_kv_heads, head_dim):
        raise ValueError(f"Expected keys shape (T, {num_kv_heads}, {head_dim}), got {tuple(key.shape)}")
    if key.dtype != key_cache.dtype or value.dtype != key_cache.dtype:
        raise ValueError("key/value dtype must match the cache dtype")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != key.shape[0]:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    if key.stride(2) != 1:
        key = key.contiguous()
    if value.stride(2) != 1:
        value = value.contiguous()
    slot_mapping = slot_mapping.contiguous()
    lib = _native.load_library()
    status = lib.pa_reshape_and_cache(
        key.data_ptr(),
        value.data_ptr(),
        key.stride(0),
        key.stride(1),
        value.stride(0),
        value.stride(1),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        slot_mapping.data_ptr(),
        int(key.shape[0]),
        num_kv_heads,
        head_dim,
        block_size,
        total_blocks,
        num_layers,
        int(layer_idx),
        dtype_code(key_cache.dtype),
        _stream(device),
    )
    _native.check(status, "pa_reshape_and_cache")


# ---------------------------------------------------------------------------
# (c)/(d) attention


def copy_blocks(src_cache: torch.Tensor, dst_cache: torch.Tensor, block_mapping) -> None:
    """Copy physical blocks between two device caches of one layout, every
    layer at once (pa_copy_blocks).

    ``block_mapping``: (src block, dst block) pairs, an int64 [n, 2] tensor or
    a sequence of pairs; ``src_cache`` / ``dst_cache``: (L, N, bs, H_kv, D)
    contiguous device tensors of the same dtype and block shape.
    """
    if src_cache.dim() != 5 or dst_cache.dim() != 5:
        raise ValueError("caches must be 5-D (layers, blocks, block_size, heads, dim)")
    if src_cache.dtype != dst_cache.dtype or src_cache.shape[0] != dst_cache.shape[0] or \
            src_cache.shape[2:] != dst_cache.shape[2:]:
        raise ValueError("caches differ in dtype, layer count or block shape")
    if not (src_cache.is_contiguous() and dst_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    device = _require_device(src_cache, dst_cache)
    mapping = torch.as_tensor(block_mapping, dtype=torch.int64)
    mapping = mapping.reshape(-1, 2).to(device, non_blocking=True).contiguous()
    if mapping.shape[0] == 0:
        return
    block_bytes = src_cache[0, 0].numel() * src_cache.element_size()
    lib = _native.load_library()
    status = lib.pa_copy_blocks(
        src_cache.data_ptr(),
        dst_cache.data_ptr(),
        mapping.data_ptr(),
        int(mapping.shape[0]),
        int(src_cache.shape[0]),
        int(src_cache.shape[1]),
        int(dst_cache.shape[1]),
        int(block_bytes),
        _stream(device),
    )
    _native.check(status, "pa_copy_blocks")


def swap_blocks(device_cache: torch.Tensor, host_cache: torch.Tensor, block_mapping, out: bool) -> None:
    """Copy blocks between a device cache and a pinned host pool of the same
    block shape, every layer in one launch (pa_swap_blocks): ``out`` copies
    device -> host for (device block, host block) pairs, else host -> device
    for (host block, device block) pairs.  Asynchronous on the current stream."""
    if device_cache.dim() != 5 or host_cache.dim() != 5:
        raise ValueError("caches must be 5-D (layers, blocks, block_size, heads, dim)")
    if device_cache.dtype != host_cache.dtype or device_cache.shape[0] != host_cache.shape[0] or \
            device_cache.shape[2:] != host_cache.shape[2:]:
        raise ValueError("device cache and host pool differ in dtype, layer count or block shape")
    if not (device_cache.is_contiguous() and host_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if host_cache.device.type != "cpu" or not host_cache.is_pinned():
        raise ValueError("the host pool must be pinned host memory")
    device = _require_device(device_cache)
    mapping = torch.as_tensor(block_mapping, dtype=torch.int64).reshape(-1, 2)
    if mapping.shape[0] == 0:
        return
    mapping = mapping.pin_memory().to(device, non_blocking=True)
    block_bytes = device_cache[0, 0].numel() * device_cache.element_size()
    lib = _native.load_library()
    with torch.cuda.device(device):
        status = lib.pa_swap_blocks(
            device_cache.data_ptr(),
            host_cache.data_ptr(),
            mapping.data_ptr(),
            int(mapping.shape[0]),
            int(device_cache.shape[0]),
            int(device_cache.shape[1]),
            int(host_cache.shape[1]),
            int(block_bytes),
            _native.PA_SWAP_OUT if out else _native.PA_SWAP_IN,
            _stream(device),
        )
    _native.check(status, "pa_swap_blocks")


def decode_workspace_bytes(num_decode_items: int, num_query_heads: int, head_dim: int) -> int:
    """Bytes of pa_decode's split-K partials: fp32 acc[items, H_q, D] and
    (max, sum)[items, H_q], each rounded up to 256 bytes (the workspace adds
    the merge records, pa_decode_merge_state_size, after them)."""
    if num_decode_items <= 0:
        return 0
    rows = num_decode_items * num_query_heads
    acc = (rows * head_dim * 4 + 255) & ~255
    ml = (rows * 2 * 4 + 255) & ~255
    return acc + ml


def _step_dims(query_t: torch.Tensor, key_cache: torch.Tensor, step: PackedStep) -> _native.PaStepDims:
    """query_t is the [T, H_q, D] view of the query."""
    num_layers, total_blocks, block_size, num_kv_heads, head_dim = key_cache.shape
    return _native.PaStepDims(
        num_seqs=step.num_seqs,
        num_query_tokens=int(query_t.shape[0]),
        num_query_heads=int(query_t.shape[1]),
        num_kv_heads=int(num_kv_heads),
        head_dim=int(head_dim),
        block_size=int(block_size),
        total_blocks=int(total_blocks),
        num_layers=int(num_layers),
        max_blocks_per_seq=step.table_width,
        partition_size=step.partition_size,
        dtype=dtype_code(key_cache.dtype),
        num_table_rows=step._source_rows,
        q_token_stride=query_t.stride(0),
        q_head_stride=query_t.stride(1),
        block_table_rows=step.ptr("rows") if step._pooled else None,
    )


def _query_view(query: torch.Tensor) -> torch.Tensor:
    """Accept [1, H_q, T, D] (reference layout) or [T, H_q, D]; return a [T, H_q, D] view."""
    if query.dim() == 4:
        if query.shape[0] != 1:
            raise ValueError("query must be (1, heads, tokens, dim)")
        q = query[0].transpose(0, 1)
    elif query.dim() == 3:
        q = query
    else:
        raise ValueError("query must be (1, H_q, T, D) or (T, H_q, D)")
    if q.stride(2) != 1:
        q = q.contiguous()
    return q


def _check_attention_inputs(q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, step: PackedStep):
    if key_cache.dim() != 5 or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be 5-D (layers, blocks, block_size, heads, dim) and alike")
    if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if q.dtype != key_cache.dtype or value_cache.dtype != key_cache.dtype:
        raise ValueError(f"query dtype {q.dtype} differs from cache dtype {key_cache.dtype}")
    num_kv_heads, head_dim = key_cache.shape[3], key_cache.shape[4]
    if q.shape[2] != head_dim:
        raise ValueError("query head_dim differs from the cache head_dim")
    if q.shape[1] % num_kv_heads != 0:
        raise RuntimeError("num_query_heads must be a multiple of num_kv_heads for GQA")
    if q.shape[0] != step.num_query_tokens:
        raise ValueError(f"query has {q.shape[0]} tokens, the step has {step.num_query_tokens}")


def _output_for(q: torch.Tensor, key_cache: torch.Tensor, out: Optional[torch.Tensor]) -> torch.Tensor:
    """``out`` checked against what the kernels write ([T, H_q, D] contiguous rows
    of the cache dtype on the query's device; a [1, T, H_q, D] tensor is taken
    as the same rows), or a new such tensor when ``out`` is None."""
    if out is None:
        return torch.empty(q.shape, dtype=key_cache.dtype, device=q.device)
    rows = out[0] if out.dim() == 4 and out.shape[0] == 1 else out
    if tuple(rows.shape) != tuple(q.shape):
        raise ValueError(f"out must have shape {tuple(q.shape)} (or (1, *that)), got {tuple(out.shape)}")
    if out.dtype != key_cache.dtype:
        raise ValueError(f"out dtype {out.dtype} differs from the cache dtype {key_cache.dtype}")
    if out.device != q.device:
        raise ValueError(f"out is on {out.device}, the query on {q.device}")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    return rows


def _checked(query, key_cache, value_cache, step: PackedStep):
    """([T, H_q, D] query view, launch dims) after the input checks.  The
    checks and dims of the last call on ``step`` are kept, keyed by
    everything they depend on, so the layers of a step after the first skip
    them."""
    q = _query_view(query)
    key = (tuple(q.shape), q.stride(), q.dtype, q.device, key_cache.data_ptr(), value_cache.data_ptr(),
           tuple(key_cache.shape), key_cache.dtype, value_cache.dtype)
    cached = step.__dict__.get("_launch_key")
    if cached is not None and cached[0] == key:
        return q, cached[1]
    _require_device(q, key_cache, value_cache, step.buffer)
    _check_attention_inputs(q, key_cache, value_cache, step)
    dims = _step_dims(q, key_cache, step)
    step.__dict__["_launch_key"] = (key, dims)
    return q, dims


def _launch_decode(q, key_cache, value_cache, layer_idx, step, scaling, out, dims, phases) -> None:
    ws_ptr, ws_bytes = step.workspace_ptr(dims)
    lib = _native.load_library()
    status = lib.pa_decode_phases(
        int(phases),
        q.data_ptr(),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int(layer_idx),
        dims,
        step.ptr("block_tables"),
        step.ptr("context_lens"),
        step.ptr("cu_seqlens"),
        step.ptr("decode_items") if step.num_decode_items else None,
        step.num_decode_items,
        step.ptr("merge_items") if step.num_merge_items else None,
        step.num_merge_items,
        float(scaling),
        out.data_ptr(),
        ws_ptr,
        ws_bytes,
        _stream(q.device),
    )
    _native.check(status, "pa_decode")


def _launch_prefill(q, key_cache, value_cache, layer_idx, step, scaling, out, dims) -> None:
    lib = _native.load_library()
    status = lib.pa_prefill(
        q.data_ptr(),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int(layer_idx),
        dims,
        step.ptr("block_tables"),
        step.ptr("context_lens"),
        step.ptr("cu_seqlens"),
        step.ptr("prefill_items") if step.num_prefill_items else None,
        step.num_prefill_items,
        step.prefill_tile,
        float(scaling),
        out.data_ptr(),
        _stream(q.device),
    )
    _native.check(status, "pa_prefill")


def decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    layer_idx: int,
    step: PackedStep,
    scaling: float,
    out: Optional[torch.Tensor] = None,
    phases: int = _native.PA_DECODE_PHASE_PARTITIONS | _native.PA_DECODE_PHASE_MERGE,
) -> torch.Tensor:
    """Split-K paged decode for the single-token sequences of ``step``.

    Returns (or fills) ``out`` [T, H_q, D]; rows of other tokens are untouched.
    ``phases`` launches only the partition and/or the merge phase (a merge
    call must follow a partition call of the same step and workspace).
    """
    q, dims = _checked(query, key_cache, value_cache, step)
    out = _output_for(q, key_cache, out)
    _launch_decode(q, key_cache, value_cache, layer_idx, step, scaling, out, dims, phases)
    return out


def prefill(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    layer_idx: int,
    step: PackedStep,
    scaling: float,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Causal chunked prefill for the multi-token sequences of ``step``."""
    q, dims = _checked(query, key_cache, value_cache, step)
    out = _output_for(q, key_cache, out)
    _launch_prefill(q, key_cache, value_cache, layer_idx, step, scaling, out, dims)
    return out


def _new_rows(new_key: torch.Tensor, new_value: torch.Tensor, key_cache: torch.Tensor,
              step: PackedStep) -> Tuple[torch.Tensor, torch.Tensor]:
    """The step's new K/V rows checked against the cache: [T, H_kv, D] of the
    cache dtype on its device, unit stride along D (copied otherwise)."""
    _require_device(new_key, new_value, key_cache)
    shape = (step.num_query_tokens, int(key_cache.shape[3]), int(key_cache.shape[4]))
    if tuple(new_key.shape) != shape or tuple(new_value.shape) != shape:
        raise ValueError(f"new_key / new_value must have shape {shape}, got {tuple(new_key.shape)} "
                         f"and {tuple(new_value.shape)}")
    if new_key.dtype != key_cache.dtype or new_value.dtype != key_cache.dtype:
        raise ValueError("new_key / new_value dtype must match the cache dtype")
    if new_key.stride(2) != 1:
        new_key = new_key.contiguous()
    if new_value.stride(2) != 1:
        new_value = new_value.contiguous()
    return new_key, new_value


def _launch_decode_append(q, key_cache, value_cache, layer_idx, step, scaling, out, dims, k, v) -> int:
    """pa_decode_append; returns its status (PA_ERR_UNSUPPORTED: not fused)."""
    ws_ptr, ws_bytes = step.workspace_ptr(dims)
    rows = _native.PaNewRows(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0), v.stride(1))
    lib = _native.load_library()
    return lib.pa_decode_append(
        q.data_ptr(),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int(layer_idx),
        dims,
        rows,
        step.ptr("block_tables"),
        step.ptr("context_lens"),
        step.ptr("cu_seqlens"),
        step.ptr("decode_items"),
        step.num_decode_items,
        step.ptr("merge_items") if step.num_merge_items else None,
        step.num_merge_items,
        float(scaling),
        out.data_ptr(),
        ws_ptr,
        ws_bytes,
        _stream(q.device),
    )


def _launch_prefill_append(q, key_cache, value_cache, layer_idx, step, scaling, out, dims, k, v) -> int:
    """pa_prefill_append; returns its status (PA_ERR_UNSUPPORTED: not fused)."""
    rows = _native.PaNewRows(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0), v.stride(1))
    lib = _native.load_library()
    return lib.pa_prefill_append(
        q.data_ptr(),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int(layer_idx),
        dims,
        rows,
        step.ptr("block_tables"),
        step.ptr("context_lens"),
        step.ptr("cu_seqlens"),
        step.ptr("prefill_items"),
        step.num_prefill_items,
        step.prefill_tile,
        float(scaling),
        out.data_ptr(),
        _stream(q.device),
    )


def _fused(status: int, who: str) -> bool:
    """True if a fused-write launch ran, False if it declined the shape."""
    if status == _native.PA_OK:
        return True
    if status != _native.PA_ERR_UNSUPPORTED:
        _native.check(status, who)
    return False


def attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    layer_idx: int,
    step: PackedStep,
    scaling: float,
    out: Optional[torch.Tensor] = None,
    new_key: Optional[torch.Tensor] = None,
    new_value: Optional[torch.Tensor] = None,
    fused_prefill_write: Optional[bool] = None,
) -> torch.Tensor:
    """Attention of a whole flattened step (decode + prefill sequences) -> [T, H_q, D].

    With ``new_key`` / ``new_value`` ([T, H_kv, D], the step's new rows) the
    rows are also written into the caches at the step's scatter slots, as
    :func:`reshape_and_cache` does: inside the prefill launch for the
    multi-token sequences (pa_prefill_append) and inside the decode launches
    for the single-token ones (pa_decode_append), or by the cache-write
    kernel ahead of the plain launches.  When a fused launch declines the
    shape, the cache-write kernel writes every row first (rows a fused
    launch already wrote get the same bytes again) and the plain launches
    follow.  ``fused_prefill_write``: whether to write the multi-token rows
    inside the prefill launch.  By default: on a step of prefill chunks
    alone, for 16-bit caches (fp32 prefills measured 2-4 % slower with the
    write inside than after the cache-write kernel); on a step with decodes
    too, never -- there the prefill that follows the long decode launch
    read its chunks' new rows 5-6 us slower than the same rows from the
    cache, and the cache-write kernel and plain launches measured 4-5 us
    cheaper per step than the fused writes.  A decode-only step writes its
    rows inside the decode launches.
    """
    q, dims = _checked(query, key_cache, value_cache, step)
    out = _output_for(q, key_cache, out)
    if (new_key is None) != (new_value is None):
        raise ValueError("new_key and new_value are given together")
    need_prefill = step.num_prefill_items > 0
    need_decode = step.num_decode_items > 0
    if new_key is not None:
        k, v = _new_rows(new_key, new_value, key_cache, step)
        if fused_prefill_write is None:
            fused_prefill_write = key_cache.dtype != torch.float32 and not need_decode
        fused = False  # a fused launch wrote rows
        if not step.__dict__.get("_no_append"):
            declined = False
            if need_prefill and fused_prefill_write:
                if _fused(_launch_prefill_append(q, key_cache, value_cache, layer_idx, step, scaling, out, dims,
                                                 k, v), "pa_prefill_append"):
                    need_prefill, fused = False, True
                else:
                    declined = True
            if need_decode and not need_prefill:
                if _fused(_launch_decode_append(q, key_cache, value_cache, layer_idx, step, scaling, out, dims,
                                                k, v), "pa_decode_append"):
                    need_decode, fused = False, True
                else:
                    declined = True
            if declined:
                step.__dict__["_no_append"] = True
        if (need_prefill or need_decode or not fused) and step.num_query_tokens > 0:
            reshape_and_cache(k, v, key_cache, value_cache, step.scatter_slots, layer_idx)
    if need_prefill:
        _launch_prefill(q, key_cache, value_cache, layer_idx, step, scaling, out, dims)
    if need_decode:
        _launch_decode(q, key_cache, value_cache, layer_idx, step, scaling, out, dims,
                       _native.PA_DECODE_PHASE_PARTITIONS | _native.PA_DECODE_PHASE_MERGE)
    if step.num_query_tokens > 0 and step.num_decode_items == 0 and step.num_prefill_items == 0:
        out.zero_()
    return out


def paged_attention_flat(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    layer_idx: int,
    gather_slots: torch.Tensor,
    attention_mask: torch.Tensor,
    scaling: float,
) -> torch.Tensor:
    """The reference's ``llm_allocator_cpp.paged_attention`` (csrc/src/bindings.cpp:10-76)
    over device tensors: fp32, query [1, H_q, T, D], caches (L, N, bs, H_kv, D),
    gather_slots int32 [C], mask uint8 [1, 1, T, C]; returns [1, T, H_q, D]."""
    device = _require_device(query, key_cache, value_cache, gather_slots, attention_mask)
    if query.dim() != 4:
        raise RuntimeError("query must be 4-D (1, heads, seq, dim)")
    if key_cache.dim() != 5:
        raise RuntimeError("key_cache must be 5-D (layers, blocks, block_size, heads, dim)")
    if gather_slots.dim() != 1:
        raise RuntimeError("gather_slots must be 1-D")
    if attention_mask.dim() != 4:
        raise RuntimeError("attention_mask must be 4-D (1, 1, query, context)")
    query = query.to(torch.float32).contiguous()
    key_cache = key_cache.to(torch.float32).contiguous()
    value_cache = value_cache.to(torch.float32).contiguous()
    gather_slots = gather_slots.to(torch.int32).contiguous()
    attention_mask = attention_mask.to(torch.uint8).contiguous()
    dims = _native.PagedAttentionDims(
        num_query_heads=int(query.shape[1]),
        num_query_tokens=int(query.shape[2]),
        head_dim=int(query.shape[3]),
        num_layers=int(key_cache.shape[0]),
        total_blocks=int(key_cache.shape[1]),
        block_size=int(key_cache.shape[2]),
        num_kv_heads=int(key_cache.shape[3]),
        num_context_tokens=int(gather_slots.shape[0]),
    )
    out = torch.empty((1, dims.num_query_tokens, dims.num_query_heads, dims.head_dim), dtype=torch.float32, device=device)
    lib = _native.load_library()
    lib.paged_attention(
        query.data_ptr(),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int(layer_idx),
        dims,
        gather_slots.data_ptr(),
        attention_mask.data_ptr(),
        float(scaling),
        out.data_ptr(),
        None,
        _stream(device),
    )
    status = lib.pa_last_error()
    if status != _native.PA_OK:
        raise RuntimeError(lib.pa_last_error_message().decode(errors="replace"))
    return out
