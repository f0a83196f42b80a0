"""GPU side of the step's host plumbing: packing from the device-resident
block-table pool (rows + queued updates, the step table gathered on the
device), the two-launch linear packing at large batches, the manager's steps
across block growth and row reuse, and swapping blocks to a pinned host pool
and back.  Integer and copy results are bit-exact against the oracle."""

import time

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import packing as op

pytestmark = pytest.mark.gpu

ops = pkg("paged_ops")
manager_mod = pkg("memory.manager")
request_mod = pkg("engine.request")


def log(msg):
    print(msg, flush=True)


def _expect(starts, counts, lists, bs, partition, tile):
    ctx = [s + c for s, c in zip(starts, counts)]
    dec, merge, pre = op.work_items(starts, counts, partition, tile)
    return dict(
        cu_seqlens=op.cumulative_offsets(counts),
        cu_context_offsets=op.cumulative_offsets(ctx),
        context_lens=np.asarray(ctx, dtype=np.int32),
        scatter_slots=op.build_slot_mapping(lists, ctx, bs, starts, counts),
        position_ids=op.position_ids(starts, counts)[0],
        gather_slots=op.build_slot_mapping(lists, ctx, bs, [0] * len(ctx), ctx),
        decode_items=dec,
        merge_items=merge,
        prefill_items=pre,
    )


def _check(step, exp):
    for name, want in exp.items():
        got = getattr(step, name).cpu().numpy()
        assert got.dtype == want.dtype, name
        assert np.array_equal(got.reshape(want.shape), want), name


@pytest.mark.parametrize("seed,one_launch", [(0, False), (1, False), (2, False), (3, True), (4, True)])
def test_pack_from_pool_rows_with_updates(device, seed, one_launch):
    """A pool of rows on the device, queued (row, col, block) updates (two of
    them outside the table, skipped) and a step over a shuffled subset of
    rows: the device pool ends updated, and the step's rows, its table
    (copied by pa_pack, or gathered from the pool), slots and work lists
    equal the oracle's on the updated rows.  With ``one_launch`` the step
    has at most 32 new tokens per sequence and no gather slots or step
    table: pa_pack does it in one launch, the table updates included."""
    rng = np.random.default_rng(seed)
    bs, rows_n, width = 16, 300, 40
    pool = np.full((rows_n, width), -1, dtype=np.int32)
    nblocks = rng.integers(0, width + 1, size=rows_n)
    for r in range(rows_n):
        pool[r, : nblocks[r]] = rng.integers(0, 100000, size=nblocks[r])
    dev_pool = torch.from_numpy(pool.copy()).to(device)
    upd = []
    for r in rng.choice(rows_n, size=50, replace=False):
        col = int(nblocks[r]) if nblocks[r] < width else int(rng.integers(0, width))
        upd.append((int(r), col, int(rng.integers(0, 100000))))
    upd += [(rows_n, 0, 7), (0, width, 7)]  # outside the table: skipped
    for r, c, b in upd:
        if r < rows_n and c < width:
            pool[r, c] = b
            nblocks[r] = max(nblocks[r], c + 1)
    rows = rng.permutation(np.flatnonzero(nblocks > 0))[:200].astype(np.int32)
    starts, counts = [], []
    for r in rows:
        cap = int(nblocks[r]) * bs
        most = 32 if one_launch else 200
        c = int(rng.choice([1, 1, 1, int(rng.integers(2, min(cap, most) + 1)) if cap > 1 else 1]))
        c = min(c, cap)
        s = int(rng.integers(0, cap - c + 1))
        starts.append(s)
        counts.append(c)
    lists = [[int(b) for b in pool[r, : nblocks[r]]] for r in rows]
    step = ops.pack_step(dev_pool, starts, counts, bs, rows=rows, updates=np.asarray(upd, dtype=np.int32),
                         prefill_tile=32, with_gather=not one_launch, step_table=not one_launch, num_kv_heads=8,
                         num_query_heads=32)
    torch.cuda.synchronize()
    log(f"pool pack seed {seed}: B={len(rows)} partition={step.partition_size} one_launch={one_launch}")
    assert np.array_equal(dev_pool.cpu().numpy(), pool)
    assert np.array_equal(step.rows.cpu().numpy(), rows)
    assert step.table_width == width and step.ptr("block_tables") == dev_pool.data_ptr()
    width_step = max(-(-(s + c) // bs) for s, c in zip(starts, counts))
    assert step.block_tables.shape == (len(rows), width_step)
    assert np.array_equal(step.block_tables.cpu().numpy(), pool[rows, :width_step])
    exp = _expect(starts, counts, lists, bs, step.partition_size, 32)
    if one_launch:
        assert max(counts) <= 32 and step.max_context // step.partition_size <= 32
    _check(step, exp)  # gather_slots of a one-launch step: built on first use by the two-launch path


def test_host_staging_ring_across_streams(device):
    """Steps packed alternately on two streams, many more than the staging
    ring's 16 slots, each from its own host arrays: every step's outputs are
    those of its own inputs (no slot is overwritten while a launch on either
    stream may still read it)."""
    rng = np.random.default_rng(11)
    bs, b = 16, 64
    table = torch.from_numpy(rng.integers(0, 1 << 16, size=(b, 64)).astype(np.int32)).to(device)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device), torch.cuda.Stream(device)]
    steps = []
    for i in range(40):
        starts = [int(x) for x in rng.integers(0, 1000, size=b)]
        counts = [int(x) for x in rng.choice([1, 1, 1, 2, 5], size=b)]
        with torch.cuda.stream(streams[i % 2]):
            steps.append((ops.pack_step(table, starts, counts, bs, prefill_tile=16, partition_size=256),
                          starts, counts))
    torch.cuda.synchronize()
    for step, starts, counts in steps:
        ctx = [s_ + c for s_, c in zip(starts, counts)]
        assert np.array_equal(step.cu_seqlens.cpu().numpy(), op.cumulative_offsets(counts))
        assert np.array_equal(step.cu_context_offsets.cpu().numpy(), op.cumulative_offsets(ctx))
        assert np.array_equal(step.position_ids.cpu().numpy(), op.position_ids(starts, counts)[0])


@pytest.mark.parametrize("b", [1, 1023, 1024, 1025, 4097])
def test_pack_large_batches(device, b):
    """Batches across the scan's 1024-sequence chunks: bit-exact outputs, and
    the partial partitions' bucket order carried across chunks."""
    rng = np.random.default_rng(b)
    bs = 16
    starts = [int(x) for x in rng.integers(0, 3000, size=b)]
    counts = [int(rng.choice([1, 1, 1, 1, 0, int(rng.integers(2, 64))])) for _ in range(b)]
    ctx = [s + c for s, c in zip(starts, counts)]
    perm = rng.permutation(sum(-(-c // bs) for c in ctx) + 1)
    lists, off = [], 0
    for c in ctx:
        n = -(-c // bs)
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    table = torch.from_numpy(op.build_block_tables(lists, ctx)[0]).to(device)
    step = ops.pack_step(table, starts, counts, bs, prefill_tile=16, with_gather=True, partition_size=512)
    log(f"large pack B={b}: items={step.num_decode_items}")
    _check(step, _expect(starts, counts, lists, bs, 512, 16))


def test_pack_time_is_linear_in_the_batch(device):
    """Pack time (replayed from a HIP graph of 20 re-runs: one launch at 256
    and 1024 decode sequences, two at 4096) per sequence does not grow from
    1024 to 4096 sequences (the kernels are linear in B), and a re-run gives
    the first run's outputs."""
    per_seq = {}
    for b in (256, 1024, 4096):
        rng = np.random.default_rng(b)
        starts = [int(x) for x in rng.integers(100, 4000, size=b)]
        counts = [1] * b
        table = torch.from_numpy(rng.integers(0, 1 << 20, size=(b, 256)).astype(np.int32)).to(device)
        step = ops.pack_step(table, starts, counts, 16, partition_size=1024)
        first = step.decode_items.clone(), step.scatter_slots.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(20):
                ops._run_pack(step)
        graph.replay()
        torch.cuda.synchronize()
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        e.record()
        e.synchronize()
        us = a.elapsed_time(e) * 1e3 / 20
        per_seq[b] = us / b
        log(f"pack B={b}: {us:.1f} us per pack ({us / b * 1e3:.1f} ns per sequence)")
        assert torch.equal(step.decode_items, first[0]) and torch.equal(step.scatter_slots, first[1])
    assert per_seq[4096] <= 1.5 * per_seq[1024]


@pytest.mark.parametrize("dtype,with_gather,free_first", [(torch.bfloat16, True, False),
                                                         (torch.float32, True, False),
                                                         (torch.bfloat16, False, False),
                                                         (torch.bfloat16, False, True),
                                                         (torch.float32, True, True)])
def test_manager_steps_track_growth_and_reuse(device, dtype, with_gather, free_first):
    """A GPU store over several steps: prompts, decodes that open new blocks,
    frees and new sequences reusing freed rows, and a pool that grows its
    rows and columns.  Every step's block table (gathered from the pool),
    slots and work lists equal the oracle's on the sequences' block lists.
    Without gather slots at pack time the decode-only steps are packed in
    one launch, queued table updates included.  With ``free_first`` the
    sequences that finish are freed before the same step admits new ones,
    so the new ones take the freed rows at once: the queue then holds a -1
    reset and a new block for one (row, col), and only the new block may
    reach the device pool."""
    m = manager_mod.PagedKVCacheManager(total_blocks=4000, block_size=16, num_heads=8, head_dim=128, dtype=dtype,
                                        num_layers=1, device=device)
    m.num_query_heads = 32
    rng = np.random.default_rng(1)
    live, next_id = [], 1

    def finish_some():
        for k in sorted(rng.choice(len(live), size=8, replace=False), reverse=True):
            m.free_sequence(live[k][0])
            del live[k]

    for step_no in range(12):
        if free_first and step_no % 4 == 3:
            finish_some()
        if step_no % 3 == 0 or (free_first and step_no % 4 == 3):
            # new requests (more than the pool's first 64 rows, over time)
            for _ in range(30):
                seq = request_mod.Request(next_id, list(range(int(rng.integers(1, 200)))))
                next_id += 1
                m.allocate_prefix_blocks(seq)
                live.append((seq, True))
        if not free_first and step_no % 4 == 3:  # some finish
            finish_some()
        seqs, starts, counts = [], [], []
        for i, (seq, fresh) in enumerate(live):
            if fresh:
                starts.append(0)
                counts.append(seq.block_table.get_tokens_count())
                live[i] = (seq, False)
            else:
                m.allocate_slot_for_next_token(seq)
                starts.append(seq.block_table.get_tokens_count() - 1)
                counts.append(1)
            seqs.append(seq)
        step = m.pack_step(seqs, starts, counts, with_gather=with_gather)
        lists = [s.block_table.get_physical_blocks() for s in seqs]
        ctx = [s + c for s, c in zip(starts, counts)]
        width = max(-(-c // 16) for c in ctx)
        want_table = np.full((len(seqs), width), -1, dtype=np.int32)
        for i, blocks in enumerate(lists):
            want_table[i, : min(len(blocks), width)] = blocks[:width]
        assert np.array_equal(step.block_tables.cpu().numpy(), want_table), step_no
        _check(step, _expect(starts, counts, lists, 16, step.partition_size, step.prefill_tile))
    assert m.tables.num_rows > 64 or m.tables.width > 64


def test_gather_slots_of_a_stale_step_raise(device):
    """Gather slots built on first read re-run the packing kernel over the
    pool as it is then: read before the next step on the same pool they
    equal the oracle's; after a later step freed a row and gave it to a new
    sequence, reading them raises instead of returning the new row's slots."""
    m = manager_mod.PagedKVCacheManager(total_blocks=256, block_size=16, num_heads=2, head_dim=64,
                                        dtype=torch.bfloat16, num_layers=1, device=device)
    m.num_query_heads = 4
    a = request_mod.Request(1, list(range(40)))
    b = request_mod.Request(2, list(range(70)))
    for seq in (a, b):
        m.allocate_prefix_blocks(seq)
    first = m.pack_step([a, b], [0, 0], [40, 70], with_gather=False)
    lists = [s.block_table.get_physical_blocks() for s in (a, b)]
    want = op.build_slot_mapping(lists, [40, 70], 16, [0, 0], [40, 70])
    assert np.array_equal(first.gather_slots.cpu().numpy(), want)
    second = m.pack_step([a, b], [0, 0], [40, 70], with_gather=False)
    m.free_sequence(a)
    c = request_mod.Request(3, list(range(25)))
    m.allocate_prefix_blocks(c)  # takes a's row
    third = m.pack_step([b, c], [0, 0], [70, 25], with_gather=False)
    with pytest.raises(RuntimeError, match="earlier step"):
        second.gather_slots
    assert torch.equal(first.gather_slots.cpu(), torch.from_numpy(want))  # built before: kept
    lists = [s.block_table.get_physical_blocks() for s in (b, c)]
    want = op.build_slot_mapping(lists, [70, 25], 16, [0, 0], [70, 25])
    assert np.array_equal(third.gather_slots.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_swap_round_trip_bit_exact(device, dtype):
    """Blocks of a sequence swapped out to the pinned host pool and back into
    fresh device blocks hold the same bits (every layer, K and V), while the
    freed device blocks were overwritten in between; reports the GB/s of a
    large swap-out and swap-in."""
    L, bs, H, D = 4, 16, 8, 128
    m = manager_mod.PagedKVCacheManager(total_blocks=2048, block_size=bs, num_heads=H, head_dim=D, dtype=dtype,
                                        num_layers=L, device=device, total_cpu_blocks=1024)
    gen = torch.Generator(device=device)
    gen.manual_seed(4)
    m.key_cache.copy_(torch.randn(m.key_cache.shape, generator=gen, device=device).to(dtype))
    m.value_cache.copy_(torch.randn(m.value_cache.shape, generator=gen, device=device).to(dtype))
    seq = request_mod.Request(1, list(range(1000)))
    m.allocate_prefix_blocks(seq)
    blocks = seq.block_table.get_physical_blocks()
    idx = torch.tensor(blocks, device=device)
    want_k, want_v = m.key_cache[:, idx].clone(), m.value_cache[:, idx].clone()
    host_ids = m.swap_out(seq)
    torch.cuda.synchronize()
    hk, hv = m.host_pool()
    assert torch.equal(hk[:, torch.tensor(host_ids)].view(torch.uint8), want_k.cpu().view(torch.uint8))
    assert torch.equal(hv[:, torch.tensor(host_ids)].view(torch.uint8), want_v.cpu().view(torch.uint8))
    # the freed device blocks are overwritten by whoever takes them next
    m.key_cache[:, idx] = 0
    m.value_cache[:, idx] = 0
    other = request_mod.Request(2, list(range(16 * 5)))
    m.allocate_prefix_blocks(other)
    new_blocks = m.swap_in(seq)
    torch.cuda.synchronize()
    nidx = torch.tensor(new_blocks, device=device)
    assert seq.block_table.get_physical_blocks() == new_blocks
    assert seq.block_table.get_tokens_count() == 1000
    assert torch.equal(m.key_cache[:, nidx].view(torch.uint8), want_k.view(torch.uint8))
    assert torch.equal(m.value_cache[:, nidx].view(torch.uint8), want_v.view(torch.uint8))
    assert m.get_allocator().get_num_free_cpu_blocks() == 1024
    # the step after swap-in reads the new blocks
    step = m.pack_step([seq], [999], [1])
    assert step.block_tables.cpu().numpy()[0].tolist() == new_blocks

    # throughput: 1024 blocks x 4 layers x K and V
    m.free_sequence(other)
    big = request_mod.Request(3, list(range(16 * 1000)))
    m.allocate_prefix_blocks(big)
    nbytes = 2 * L * len(big.block_table.get_physical_blocks()) * bs * H * D * m.key_cache.element_size()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    m.swap_out(big)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    m.swap_in(big)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    log(f"swap {dtype}: {nbytes / 1e6:.1f} MB out {nbytes / (t1 - t0) / 1e9:.1f} GB/s, "
        f"in {nbytes / (t2 - t1) / 1e9:.1f} GB/s (host-timed, incl. launch)")
