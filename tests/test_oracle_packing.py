"""The integer oracle (oracle/packing.py) against the known answers held in the
reference's own tests and against brute-force enumeration."""

import numpy as np
import pytest

from oracle import packing as op


def test_cu_seqlens_known_answer():
    # tests/unit/test_attention_backends.py:177-183
    counts = [4, 2, 3]
    assert op.cumulative_offsets(counts).tolist() == [0, 4, 6, 9]
    assert op.cumulative_offsets([0 + c for c in counts]).tolist() == [0, 4, 6, 9]
    assert op.cumulative_offsets([]).tolist() == [0]
    assert op.cumulative_offsets([4, 2, 3]).dtype == np.int64


def test_position_ids_known_answers():
    # tests/unit/test_attention_backends.py:186-207
    assert op.position_ids([0, 0], [4, 2]).tolist() == [[0, 1, 2, 3, 0, 1]]
    assert op.position_ids([4, 2], [1, 1]).tolist() == [[4, 2]]
    assert op.position_ids([], []).shape == (1, 0)


def test_attention_mask_known_answer():
    # tests/unit/test_attention_backends.py:210-226
    expected = np.array(
        [
            [1, 0, 0, 0, 0, 0],
            [1, 1, 0, 0, 0, 0],
            [1, 1, 1, 0, 0, 0],
            [1, 1, 1, 1, 0, 0],
            [0, 0, 0, 0, 1, 0],
            [0, 0, 0, 0, 1, 1],
        ],
        dtype=bool,
    )
    mask = op.attention_mask([0, 0], [4, 2])
    assert mask.shape == (1, 1, 6, 6)
    assert np.array_equal(mask[0, 0], expected)


def test_attention_mask_brute_force_with_offsets():
    starts, counts = [3, 0, 7], [2, 4, 1]
    mask = op.attention_mask(starts, counts)[0, 0]
    rows = []
    for s, (st, n) in enumerate(zip(starts, counts)):
        for i in range(n):
            row = []
            for s2, (st2, n2) in enumerate(zip(starts, counts)):
                for j in range(st2 + n2):
                    row.append(s2 == s and j <= st + i)
            rows.append(row)
    assert np.array_equal(mask, np.array(rows, dtype=bool))


def test_slot_formulas_known_answers():
    # tests/unit/test_kv_cache.py:135-165 with block size 4
    blocks = [7, 2]
    assert op.sequence_slots(blocks, 6, 4, 0, 6).tolist() == [28, 29, 30, 31, 8, 9]
    assert op.sequence_slots([5], 4, 4, 3, 1).tolist() == [5 * 4 + 3]
    first = op.build_slot_mapping([[1]], [3], 4, [0], [3])
    second = op.build_slot_mapping([[3, 0]], [5], 4, [0], [5])
    both = op.build_slot_mapping([[1], [3, 0]], [3, 5], 4, [0, 0], [3, 5])
    assert both.tolist() == first.tolist() + second.tolist()
    assert op.build_slot_mapping([], [], 4, [], []).tolist() == []


def test_slot_mapping_errors():
    # tests/unit/test_kv_cache.py:214-225 and manager.py:110-114,304-315
    with pytest.raises(ValueError):
        op.build_slot_mapping([[0]], [4], 4, [0], [5])
    with pytest.raises(ValueError):
        op.build_slot_mapping([[0]], [4], 4, [0, 1], [4])
    with pytest.raises(ValueError):
        op.sequence_slots([0], 4, 4, -1, 1)


@pytest.mark.parametrize("seed", range(5))
def test_slot_mapping_brute_force(seed):
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([1, 2, 4, 16, 32]))
    b = int(rng.integers(1, 8))
    tokens = [int(x) for x in rng.integers(1, 200, size=b)]
    nblk = [-(-t // bs) for t in tokens]
    pool = rng.permutation(sum(nblk) + 5)
    lists, off = [], 0
    for n in nblk:
        lists.append([int(x) for x in pool[off : off + n]])
        off += n
    starts = [int(rng.integers(0, t + 1)) for t in tokens]
    counts = [int(rng.integers(0, t - s + 1)) for s, t in zip(starts, tokens)]
    got = op.build_slot_mapping(lists, tokens, bs, starts, counts)
    want = []
    for blocks, s, c in zip(lists, starts, counts):
        for p in range(s, s + c):
            want.append(blocks[p // bs] * bs + p % bs)
    assert got.dtype == np.int64
    assert got.tolist() == want


def test_block_tables_known_answers():
    # tests/stress/test_03_ragged_layout.py:10-42 / 45-71 (bs = 4)
    table, lens = op.build_block_tables([[0], [1, 2], [3, 4, 5, 6]], [1, 7, 13])
    assert table.shape == (3, 4)
    assert lens.tolist() == [1, 7, 13]
    assert table[0, 1:].tolist() == [-1, -1, -1]
    assert table[1, 2:].tolist() == [-1, -1]
    assert -1 not in table[2].tolist()
    table, lens = op.build_block_tables([[9]], [4])
    assert table.shape == (1, 1) and table[0, 0] != -1 and lens.tolist() == [4]
    table, lens = op.build_block_tables([], [])
    assert table.shape == (0, 0) and table.dtype == np.int32


def test_scatter_placement_and_isolation():
    # tests/unit/test_kv_cache.py:168-203: placement in the right block rows,
    # other sequences untouched.
    cache = np.zeros((1, 10, 4, 2, 8), dtype=np.float32)
    rng = np.random.default_rng(0)
    first, second = [3], [6]
    slots = op.build_slot_mapping([first, second], [3, 2], 4, [0, 0], [3, 2])
    rows = rng.standard_normal((5, 2, 8)).astype(np.float32)
    op.scatter_layer_kv(cache, 0, rows, slots)
    for t in range(3):
        assert np.array_equal(cache[0, 3, t], rows[t])
    for t in range(2):
        assert np.array_equal(cache[0, 6, t], rows[3 + t])
    assert np.count_nonzero(cache[0, [0, 1, 2, 4, 5, 7, 8, 9]]) == 0
    with pytest.raises(ValueError):
        op.scatter_layer_kv(cache, 0, rows[:, :1], slots)


def test_scatter_is_bit_exact_on_raw_bits():
    cache = np.zeros((2, 3, 4, 1, 4), dtype=np.uint16)
    rows = np.arange(2 * 4, dtype=np.uint16).reshape(2, 1, 4) + 0xBF00
    op.scatter_layer_kv(cache, 1, rows, np.array([5, 11], dtype=np.int64))
    assert np.array_equal(cache[1, 1, 1, 0], rows[0, 0])
    assert np.array_equal(cache[1, 2, 3, 0], rows[1, 0])
    assert np.count_nonzero(cache[0]) == 0


def test_work_items():
    # contexts of the decode sequences 1, 2, 4, 5: 601, 1101, 8, 1024
    dec, merge, pre = op.work_items([0, 600, 1100, 0, 7, 1023], [300, 1, 1, 5, 1, 1], 512, 32)
    # full partitions by sequence, then partial ones longest first (89, 77, 8)
    assert dec.tolist() == [[1, 0], [2, 0], [2, 1], [5, 0], [5, 1], [1, 1], [2, 2], [4, 0]]
    assert merge.tolist() == [[0, 1, 1, 5], [1, 2, 2, 6], [3, 2, 5, -1]]
    assert pre.tolist() == [[0, q] for q in range(10)] + [[3, 0]]
    # partials of 73 and 79 tokens share a bucket ((r - 1) * 64 // 512 = 9):
    # the earlier sequence goes first although it is shorter; 89 (bucket 11)
    # and 88 (bucket 10) lead, 8 (bucket 0) ends the launch
    dec, merge, _ = op.work_items([72, 78, 7, 87, 600], [1, 1, 1, 1, 1], 512, 32)
    assert dec.tolist() == [[4, 0], [4, 1], [3, 0], [0, 0], [1, 0], [2, 0]]
    assert merge.tolist() == [[0, 1, 4, 1]]
    # with partitions of 64 tokens every length is its own bucket
    dec, _, _ = op.work_items([40, 62, 9], [1, 1, 1], 64, 32)
    assert dec.tolist() == [[1, 0], [0, 0], [2, 0]]


@pytest.mark.parametrize("seed", range(3))
def test_work_items_cover_every_partition_once(seed):
    rng = np.random.default_rng(seed)
    b = 50
    starts = [int(x) for x in rng.integers(0, 5000, size=b)]
    counts = [int(rng.choice([0, 1, 1, 1, 7])) for _ in range(b)]
    part = int(rng.choice([32, 256, 512, 1000]))
    dec, merge, _ = op.work_items(starts, counts, part, 16)
    want = sorted((i, p) for i, (s, c) in enumerate(zip(starts, counts)) if c == 1
                  for p in range(-(-(s + c) // part)))
    assert sorted(map(tuple, dec.tolist())) == want
    length = [min(part, starts[s] + 1 - p * part) for s, p in dec.tolist()]
    bucket = [64 if n == part else (n - 1) * 64 // part for n in length]
    assert bucket == sorted(bucket, reverse=True)
    # ties within a bucket keep sequence order
    for k in range(len(dec) - 1):
        if bucket[k] == bucket[k + 1] and bucket[k] < 64:
            assert dec[k][0] < dec[k + 1][0]
    for first, nfull, seq, rem in merge.tolist():
        items = [tuple(x) for x in dec[first : first + nfull].tolist()] + ([tuple(dec[rem])] if rem >= 0 else [])
        assert items == [(seq, p) for p in range(-(-(starts[seq] + 1) // part))]


def test_copy_blocks_brute_force():
    rng = np.random.default_rng(3)
    src = rng.integers(0, 2**16, size=(3, 10, 4, 2, 6), dtype=np.uint16)
    dst = rng.integers(0, 2**16, size=(3, 7, 4, 2, 6), dtype=np.uint16)
    before = dst.copy()
    mapping = [(2, 0), (9, 6), (11, 1), (0, 7), (-1, 2), (5, 3)]
    op.copy_blocks(src, dst, mapping)
    for layer in range(3):
        for blk in range(7):
            want = {0: src[layer, 2], 6: src[layer, 9], 3: src[layer, 5]}.get(blk, before[layer, blk])
            assert np.array_equal(dst[layer, blk], want)
