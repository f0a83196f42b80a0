"""ORACLE -- test infrastructure only (tests/ and __graft_entry__.smoke();
never the product path).

NumPy restatement of the reference's ragged-batch packing and KV write, the
integer side of the paged-attention path.  Every function cites the lines it
follows; all integer outputs are int64 like the reference tensors.

Pinned by tests/test_oracle_packing.py against the known answers held in the
reference's own tests (tests/unit/test_attention_backends.py:177-226,
tests/unit/test_kv_cache.py:135-225, tests/stress/test_03_ragged_layout.py:
10-71) and against brute-force per-position enumeration.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


def cumulative_offsets(counts: Sequence[int]) -> np.ndarray:
    """Exclusive prefix sum with a leading 0 (app/model/paged_attention.py:121-125)."""
    out = np.zeros(len(counts) + 1, dtype=np.int64)
    if len(counts):
        np.cumsum(np.asarray(counts, dtype=np.int64), out=out[1:])
    return out


def sequence_slots(blocks: Sequence[int], tokens_count: int, block_size: int, start: int, count: int,
                   seq_id: int = 0) -> np.ndarray:
    """Slots of positions [start, start+count) of one sequence
    (app/memory/manager.py:301-333): block[p // bs] * bs + p % bs."""
    if start < 0 or count < 0:
        raise ValueError(
            f"Sequence {seq_id}: start_token ({start}) and token_count ({count}) must be non-negative")
    if start + count > tokens_count:
        raise ValueError(
            f"Sequence {seq_id}: tokens [{start}, {start + count}) exceed allocated tokens ({tokens_count})")
    if count == 0:
        return np.zeros(0, dtype=np.int64)
    first = start // block_size
    last = (start + count - 1) // block_size
    phys = np.asarray(blocks[first : last + 1], dtype=np.int64)
    all_slots = (phys[:, None] * block_size + np.arange(block_size, dtype=np.int64)[None, :]).reshape(-1)
    offset = start - first * block_size
    return all_slots[offset : offset + count]


def build_slot_mapping(block_lists: Sequence[Sequence[int]], tokens_counts: Sequence[int], block_size: int,
                       starts: Sequence[int], counts: Sequence[int]) -> np.ndarray:
    """Concatenated slots of every sequence in order (app/memory/manager.py:104-128)."""
    if not (len(block_lists) == len(starts) == len(counts)):
        raise ValueError(
            f"sequences ({len(block_lists)}), start_tokens ({len(starts)}) "
            f"and token_counts ({len(counts)}) must have the same length")
    chunks = [sequence_slots(b, tc, block_size, s, c, i)
              for i, (b, tc, s, c) in enumerate(zip(block_lists, tokens_counts, starts, counts))]
    chunks = [c for c in chunks if c.size]
    return np.concatenate(chunks) if chunks else np.zeros(0, dtype=np.int64)


def build_block_tables(block_lists: Sequence[Sequence[int]], tokens_counts: Sequence[int]
                       ) -> Tuple[np.ndarray, np.ndarray]:
    """int32 [B, max_blocks] padded with -1, int32 context lengths
    (app/memory/manager.py:236-271)."""
    b = len(block_lists)
    if b == 0:
        return np.zeros((0, 0), dtype=np.int32), np.zeros(0, dtype=np.int32)
    width = max(len(x) for x in block_lists)
    table = np.full((b, width), -1, dtype=np.int32)
    for i, blocks in enumerate(block_lists):
        if len(blocks):
            table[i, : len(blocks)] = np.asarray(blocks, dtype=np.int32)
    return table, np.asarray(tokens_counts, dtype=np.int32)


def position_ids(starts: Sequence[int], counts: Sequence[int]) -> np.ndarray:
    """[1, T] positions restarting per sequence (app/model/paged_attention.py:81-90)."""
    parts = [np.arange(s, s + c, dtype=np.int64) for s, c in zip(starts, counts)]
    flat = np.concatenate(parts) if parts else np.zeros(0, dtype=np.int64)
    return flat[None, :]


def sequence_index(counts: Sequence[int]) -> np.ndarray:
    """Owning sequence of every concatenated token (paged_attention.py:128-135)."""
    return np.repeat(np.arange(len(counts), dtype=np.int64), np.asarray(counts, dtype=np.int64))


def attention_mask(starts: Sequence[int], counts: Sequence[int]) -> np.ndarray:
    """Block-diagonal causal mask bool [1, 1, T, C] (paged_attention.py:92-118):
    query i of sequence s (position start_s + i - cu_seqlens[s]) attends
    context token j of the same sequence when its position <= that."""
    ctx = [s + c for s, c in zip(starts, counts)]
    cu_q = cumulative_offsets(counts)
    cu_c = cumulative_offsets(ctx)
    qi = sequence_index(counts)
    ci = sequence_index(ctx)
    st = np.asarray(starts, dtype=np.int64)
    qpos = np.arange(int(cu_q[-1]), dtype=np.int64) - cu_q[qi] + st[qi]
    cpos = np.arange(int(cu_c[-1]), dtype=np.int64) - cu_c[ci]
    mask = (ci[None, :] == qi[:, None]) & (cpos[None, :] <= qpos[:, None])
    return mask[None, None]


def scatter_layer_kv(cache: np.ndarray, layer_idx: int, rows: np.ndarray, slots: np.ndarray) -> None:
    """cache[layer].view(N*bs, H, D)[slots] = rows (app/memory/manager.py:150-168).

    Works on raw bit patterns (any dtype, e.g. uint16 for bf16) so the copy
    is exact.  Like torch's index_put on the CPU, an out-of-range slot raises.
    """
    layer = cache[layer_idx]
    n, bs, h, d = layer.shape
    if rows.shape != (slots.shape[0], h, d):
        raise ValueError(f"Expected keys shape {(slots.shape[0], h, d)}, got {tuple(rows.shape)}")
    if slots.size == 0:
        return
    if slots.min() < -(n * bs) or slots.max() >= n * bs:
        raise IndexError("slot out of range")
    flat = layer.reshape(n * bs, h, d)
    flat[slots] = rows


def copy_blocks(src: np.ndarray, dst: np.ndarray, mapping: Sequence[Tuple[int, int]]) -> None:
    """dst[:, d] = src[:, s] for every (s, d) pair in order, all layers of the
    (L, N, bs, H, D) caches; pairs with an index outside its cache are
    skipped.  The intent of KVCacheMemoryStrategy.copy_blocks
    (app/memory/strategies.py:88-90, 117-122) -- copy the named physical
    blocks -- on this layout; raw bits, so the copy is exact."""
    for s_blk, d_blk in mapping:
        if 0 <= s_blk < src.shape[1] and 0 <= d_blk < dst.shape[1]:
            dst[:, d_blk] = src[:, s_blk]


#: Length buckets that order the partial decode partitions.
PARTIAL_BUCKETS = 64


def work_items(starts: Sequence[int], counts: Sequence[int], partition: int, prefill_tile: int
               ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Attention work lists the GPU packing kernel emits alongside the
    reference outputs.

    decode: (seq, partition) of single-token sequences -- every full
    partition first, by sequence then partition, then the partial last
    partitions by decreasing length bucket, bucket = (length - 1) * 64 //
    partition (ties by sequence);
    merge: (first full item, number of full partitions, seq, item of the
    partial partition or -1) of every sequence with more than one
    partition, by sequence;
    prefill: (seq, query tile) of multi-token sequences, by sequence.
    """
    full: List[Tuple[int, int]] = []
    rems: List[Tuple[int, int, int]] = []  # (length, seq, partition)
    first_full = {}
    for i, (s, c) in enumerate(zip(starts, counts)):
        if c == 1:
            ctx = s + c
            first_full[i] = len(full)
            full += [(i, p) for p in range(ctx // partition)]
            if ctx % partition:
                rems.append((ctx % partition, i, ctx // partition))
    rems.sort(key=lambda r: (-(((r[0] - 1) * PARTIAL_BUCKETS) // partition), r[1]))
    rem_index = {seq: len(full) + k for k, (_, seq, _) in enumerate(rems)}
    dec = full + [(seq, p) for _, seq, p in rems]
    merge: List[Tuple[int, int, int, int]] = []
    pre: List[Tuple[int, int]] = []
    for i, (s, c) in enumerate(zip(starts, counts)):
        if c == 1:
            nfull = (s + c) // partition
            rem = rem_index.get(i, -1)
            if nfull + (rem >= 0) > 1:
                merge.append((first_full[i], nfull, i, rem))
        elif c > 1:
            pre += [(i, q) for q in range(-(-c // prefill_tile))]
    return (np.asarray(dec, dtype=np.int32).reshape(-1, 2), np.asarray(merge, dtype=np.int32).reshape(-1, 4),
            np.asarray(pre, dtype=np.int32).reshape(-1, 2))
