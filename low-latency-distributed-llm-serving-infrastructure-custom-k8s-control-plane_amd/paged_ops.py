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

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

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


@dataclass
class PackedStep:
    """Device-side description of one flattened ragged step (output of pa_pack).

    Host-side counts are derived from the host lists the scheduler already
    holds, so no device->host synchronisation is needed to size the grids.
    """

    block_tables: torch.Tensor  # int32 [B, max_blocks]
    start_positions: torch.Tensor  # int64 [B]
    new_token_counts: torch.Tensor  # int64 [B]
    cu_seqlens: torch.Tensor  # int64 [B+1]
    cu_context_offsets: torch.Tensor  # int64 [B+1]
    context_lens: torch.Tensor  # int32 [B]
    scatter_slots: torch.Tensor  # int64 [T]
    position_ids: torch.Tensor  # int64 [T]
    decode_items: torch.Tensor  # int32 [num_decode_items, 2]
    # int32 [num_merge_items, 4]: (first full-partition item, full partitions,
    # seq, remainder item or -1)
    merge_items: torch.Tensor
    prefill_items: torch.Tensor  # int32 [num_prefill_items, 2]
    block_size: int
    partition_size: int
    prefill_tile: int
    num_query_tokens: int
    num_context_tokens: int
    num_decode_items: int
    num_merge_items: int
    num_prefill_items: int
    num_decode_seqs: int
    num_prefill_seqs: int
    _gather_slots: Optional[torch.Tensor] = field(default=None, repr=False)
    _workspace: Optional[torch.Tensor] = field(default=None, repr=False)

    @property
    def num_seqs(self) -> int:
        return int(self.block_tables.shape[0])

    @property
    def gather_slots(self) -> torch.Tensor:
        """int64 [C] slots of every context token (built on first use)."""
        if self._gather_slots is None:
            self._gather_slots = _run_pack(self, with_gather=True)
        return self._gather_slots

    def workspace(self, num_query_heads: int, head_dim: int, device: torch.device) -> torch.Tensor:
        """Decode workspace (split-K partials), reused across the layers of the
        step; calls that share it must not overlap in time."""
        need = decode_workspace_bytes(self.num_decode_items, num_query_heads, head_dim)
        ws = self._workspace
        if ws is None or ws.numel() < need or ws.device != device:
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
            self._workspace = ws
        return ws


def work_counts(
    start_positions: Sequence[int],
    new_token_counts: Sequence[int],
    partition_size: int,
    prefill_tile: int,
):
    """Host-side sizes of a step:
    (T, C, decode items, merge items, prefill items, #decode seqs, #prefill seqs)."""
    t = c = ditems = mitems = pitems = ndec = npre = 0
    for start, count in zip(start_positions, new_token_counts):
        ctx = start + count
        t += count
        c += ctx
        if count == 1:
            ditems += -(-ctx // partition_size)
            mitems += ctx > partition_size
            ndec += 1
        elif count > 1:
            pitems += -(-count // prefill_tile)
            npre += 1
    return t, c, ditems, mitems, pitems, ndec, npre


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


def choose_partition(
    start_positions: Sequence[int],
    new_token_counts: Sequence[int],
    num_kv_heads: int = 8,
    num_query_heads: Optional[int] = None,
    workgroups_per_item: Optional[int] = None,
    workgroups_per_cu: Optional[int] = None,
    compute_units: int = _DECODE_CUS,
) -> int:
    """Split-K partition for the decode sequences of a step.

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

    A step too small for that rule (a latency-bound step) takes the largest
    partition that still gives two thirds of the slots a workgroup with at
    most 64 partials per sequence, or, when none does, the smallest of 64,
    128, ... that keeps every sequence to 64 partials: short walks per
    workgroup, few partials to merge.
    Measured with graph replay, 32/8 heads of 128 paired: 1 sequence of 1024
    tokens 16.6 us at 256 -> 11.3 at 64; 16 of 4096 55.9 -> 50.7 at 512.
    """
    hkv = max(int(num_kv_heads), 1)
    group = max(int(num_query_heads or 4 * hkv) // hkv, 1)
    per_cu = int(workgroups_per_cu or 0) or (5 if group == 1 else 4)
    slots = int(compute_units) * per_cu
    width = max(int(workgroups_per_item or hkv), 1)  # workgroups per item
    ctx = [s + c for s, c in zip(start_positions, new_token_counts) if c == 1]

    def workgroups(p: int) -> int:
        return sum(-(-x // p) for x in ctx) * width

    p = PA_DECODE_MAX_PARTITION
    while p > 256:
        if workgroups(p) >= 3 * slots // 2:
            return p
        p //= 2
    longest = max(ctx, default=0)
    p = PA_DECODE_MAX_PARTITION
    while p >= 64:
        if workgroups(p) >= 2 * slots // 3 and -(-longest // p) <= 64:
            return p
        p //= 2
    p = 64
    while p < PA_DECODE_MAX_PARTITION and -(-longest // p) > 64:
        p *= 2
    return p


def _run_pack(step: PackedStep, with_gather: bool = False) -> Optional[torch.Tensor]:
    lib = _native.load_library()
    device = _require_device(step.block_tables)
    gather = None
    if with_gather:
        gather = torch.empty(step.num_context_tokens, dtype=torch.int64, device=device)
    dims = _native.PaPackDims(
        num_seqs=step.num_seqs,
        block_size=step.block_size,
        max_blocks_per_seq=int(step.block_tables.shape[1]) if step.block_tables.dim() == 2 else 0,
        partition_size=step.partition_size,
        prefill_tile=step.prefill_tile,
        max_query_tokens=step.num_query_tokens,
        max_context_tokens=step.num_context_tokens,
        max_decode_items=step.num_decode_items,
        max_merge_items=step.num_merge_items,
        max_prefill_items=step.num_prefill_items,
    )
    status = lib.pa_pack(
        _ptr(step.block_tables),
        _ptr(step.start_positions),
        _ptr(step.new_token_counts),
        dims,
        _ptr(step.cu_seqlens),
        _ptr(step.cu_context_offsets),
        _ptr(step.context_lens),
        _ptr(step.scatter_slots),
        _ptr(step.position_ids),
        _ptr(gather),
        _ptr(step.decode_items),
        _ptr(step.merge_items),
        _ptr(step.prefill_items),
        _stream(device),
    )
    _native.check(status, "pa_pack")
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
    start_positions_dev: Optional[torch.Tensor] = None,
    new_token_counts_dev: Optional[torch.Tensor] = None,
) -> PackedStep:
    """Run the GPU packing kernel for one step.

    ``block_tables``: int32 [B, max_blocks] device tensor (-1 padded).
    ``start_positions`` / ``new_token_counts``: the host lists of the step
    (also uploaded unless device copies are passed in).
    ``partition_size``: decode split-K partition in tokens; by default
    :func:`choose_partition` picks it from the step and the head counts
    (and, when ``head_dim`` and the cache ``dtype`` are given, from how many
    KV heads one decode workgroup reads).
    ``prefill_tile``: query tokens per prefill work item; by default the
    MFMA kernel's tile for the head counts (:func:`prefill_tile_for`).
    """
    device = _require_device(block_tables)
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2:
        raise ValueError("block_tables must be an int32 [B, max_blocks] tensor")
    if not block_tables.is_contiguous():
        block_tables = block_tables.contiguous()
    b = int(block_tables.shape[0])
    if len(start_positions) != b or len(new_token_counts) != b:
        raise ValueError("start_positions / new_token_counts must have one entry per block-table row")
    if any(s < 0 for s in start_positions) or any(c < 0 for c in new_token_counts):
        raise ValueError("start positions and token counts must be non-negative")
    if prefill_tile is None:
        prefill_tile = prefill_tile_for(int(num_query_heads or 4 * num_kv_heads), int(num_kv_heads))
    if prefill_tile <= 0:
        raise ValueError("prefill_tile must be positive")
    if partition_size is None:
        per_item, per_cu = None, None
        if head_dim is not None and dtype is not None:
            hq = int(num_query_heads or 4 * num_kv_heads)
            per_item = decode_workgroups_per_item(dtype, head_dim, num_kv_heads, hq) or None
            with torch.cuda.device(device):  # the occupancy of the step's own device
                per_cu = decode_workgroups_per_cu(dtype, head_dim, num_kv_heads, hq) or None
        partition_size = choose_partition(
            start_positions, new_token_counts, num_kv_heads, num_query_heads, per_item, per_cu,
            torch.cuda.get_device_properties(device).multi_processor_count)
    if partition_size <= 0:
        raise ValueError("partition_size must be positive")
    t, c, ditems, mitems, pitems, ndec, npre = work_counts(
        start_positions, new_token_counts, partition_size, prefill_tile)
    # Host lists go up from pinned buffers (torch's caching host allocator), so
    # the copies are asynchronous: a pageable source would make the host wait
    # for the stream to drain the previous step before the copy.
    if start_positions_dev is None:
        start_positions_dev = torch.tensor(list(start_positions), dtype=torch.int64,
                                           pin_memory=True).to(device, non_blocking=True)
    if new_token_counts_dev is None:
        new_token_counts_dev = torch.tensor(list(new_token_counts), dtype=torch.int64,
                                            pin_memory=True).to(device, non_blocking=True)
    step = PackedStep(
        block_tables=block_tables,
        start_positions=start_positions_dev,
        new_token_counts=new_token_counts_dev,
        cu_seqlens=torch.empty(b + 1, dtype=torch.int64, device=device),
        cu_context_offsets=torch.empty(b + 1, dtype=torch.int64, device=device),
        context_lens=torch.empty(b, dtype=torch.int32, device=device),
        scatter_slots=torch.empty(t, dtype=torch.int64, device=device),
        position_ids=torch.empty(t, dtype=torch.int64, device=device),
        decode_items=torch.empty((ditems, 2), dtype=torch.int32, device=device),
        merge_items=torch.empty((mitems, 4), dtype=torch.int32, device=device),
        prefill_items=torch.empty((pitems, 2), dtype=torch.int32, device=device),
        block_size=int(block_size),
        partition_size=int(partition_size),
        prefill_tile=int(prefill_tile),
        num_query_tokens=t,
        num_context_tokens=c,
        num_decode_items=ditems,
        num_merge_items=mitems,
        num_prefill_items=pitems,
        num_decode_seqs=ndec,
        num_prefill_seqs=npre,
    )
    step._gather_slots = _run_pack(step, with_gather=with_gather)
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


def decode_workspace_bytes(num_decode_items: int, num_query_heads: int, head_dim: int) -> int:
    """Bytes pa_decode needs for its split-K partials: fp32 acc[items, H_q, D]
    and (max, sum)[items, H_q], each rounded up to 256 bytes."""
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
        max_blocks_per_seq=int(step.block_tables.shape[1]),
        partition_size=step.partition_size,
        dtype=dtype_code(key_cache.dtype),
        q_token_stride=query_t.stride(0),
        q_head_stride=query_t.stride(1),
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
    if q.dtype != key_cache.dtype:
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
    q = _query_view(query)
    device = _require_device(q, key_cache, value_cache, step.block_tables)
    _check_attention_inputs(q, key_cache, value_cache, step)
    out = _output_for(q, key_cache, out)
    dims = _step_dims(q, key_cache, step)
    ws = step.workspace(int(q.shape[1]), int(q.shape[2]), device)
    lib = _native.load_library()
    status = lib.pa_decode_phases(
        int(phases),
        q.data_ptr(),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int(layer_idx),
        dims,
        step.block_tables.data_ptr(),
        step.context_lens.data_ptr(),
        step.cu_seqlens.data_ptr(),
        _ptr(step.decode_items),
        step.num_decode_items,
        _ptr(step.merge_items),
        step.num_merge_items,
        float(scaling),
        out.data_ptr(),
        ws.data_ptr(),
        ws.numel(),
        _stream(device),
    )
    _native.check(status, "pa_decode")
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
    q = _query_view(query)
    device = _require_device(q, key_cache, value_cache, step.block_tables)
    _check_attention_inputs(q, key_cache, value_cache, step)
    out = _output_for(q, key_cache, out)
    dims = _step_dims(q, key_cache, step)
    lib = _native.load_library()
    status = lib.pa_prefill(
        q.data_ptr(),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        int(layer_idx),
        dims,
        step.block_tables.data_ptr(),
        step.context_lens.data_ptr(),
        step.cu_seqlens.data_ptr(),
        _ptr(step.prefill_items),
        step.num_prefill_items,
        step.prefill_tile,
        float(scaling),
        out.data_ptr(),
        _stream(device),
    )
    _native.check(status, "pa_prefill")
    return out


def attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    layer_idx: int,
    step: PackedStep,
    scaling: float,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention of a whole flattened step (decode + prefill sequences) -> [T, H_q, D]."""
    q = _query_view(query)
    _require_device(q, key_cache, value_cache)
    _check_attention_inputs(q, key_cache, value_cache, step)
    out = _output_for(q, key_cache, out)
    if step.num_prefill_items > 0:
        prefill(q, key_cache, value_cache, layer_idx, step, scaling, out=out)
    if step.num_decode_items > 0:
        decode(q, key_cache, value_cache, layer_idx, step, scaling, out=out)
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
