"""Host-side operator API on the CPU: backend selection and dispatch, step
bookkeeping, KV-cache manager errors, and the host helpers that size the
GPU work lists.

These follow the reference's own unit tests case by case
(tests/unit/test_attention_backends.py, tests/unit/test_kv_cache.py), with
the known answers those tests hold.  The torch SDPA backend checked here is
the reference's own fallback interface; the HIP path is covered by the GPU
parity tests.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import pkg
from oracle import packing as op

paged_attention = pkg("model.paged_attention")
backends = pkg("model.attention_backends")
manager_mod = pkg("memory.manager")
sequence_mod = pkg("engine.request")
ops = pkg("paged_ops")

NUM_LAYERS = 4
NUM_KV_HEADS = 2
HEAD_DIM = 8
BLOCK_SIZE = 4
AVAILABLE = backends.__name__ + ".native_kernel_available"


@pytest.fixture
def store():
    return manager_mod.PagedKVCacheManager(total_blocks=8, block_size=BLOCK_SIZE, num_heads=NUM_KV_HEADS,
                                           head_dim=HEAD_DIM, num_layers=NUM_LAYERS, device="cpu")


def _prefill_step(store, prompt_lens):
    seqs = []
    for i, n in enumerate(prompt_lens):
        seq = sequence_mod.Request(seq_id=i + 1, prompt_token_ids=list(range(n)))
        store.allocate_prefix_blocks(seq)
        seqs.append(seq)
    return seqs, paged_attention.PagedStepContext(store, seqs, [0] * len(seqs), list(prompt_lens))


class _Layer:
    layer_idx = 0
    scaling = 0.35

    def __init__(self, context):
        self.paged_context = context


# ---- select_backend (attention_backends.py:120-144) -----------------------


def test_auto_selects_torch_without_native_library(monkeypatch):
    monkeypatch.delenv("LLM_PAGED_BACKEND", raising=False)
    monkeypatch.setattr(AVAILABLE, lambda: False)
    assert isinstance(backends.select_backend(), backends.TorchSdpBackend)


def test_auto_prefers_native_when_available(monkeypatch):
    monkeypatch.delenv("LLM_PAGED_BACKEND", raising=False)
    monkeypatch.setattr(AVAILABLE, lambda: True)
    assert isinstance(backends.select_backend(), backends.NativePagedBackend)


def test_torch_backend_can_always_be_requested(monkeypatch):
    monkeypatch.setenv("LLM_PAGED_BACKEND", "torch")
    assert isinstance(backends.select_backend(), backends.TorchSdpBackend)


def test_native_request_without_library_raises(monkeypatch):
    monkeypatch.setenv("LLM_PAGED_BACKEND", "native")
    monkeypatch.setattr(AVAILABLE, lambda: False)
    with pytest.raises(RuntimeError):
        backends.select_backend()


def test_unknown_backend_name_raises(monkeypatch):
    monkeypatch.setenv("LLM_PAGED_BACKEND", "flash")
    with pytest.raises(ValueError):
        backends.select_backend()


def test_hip_is_an_alias_of_native(monkeypatch):
    monkeypatch.setenv("LLM_PAGED_BACKEND", "hip")
    monkeypatch.setattr(AVAILABLE, lambda: True)
    assert isinstance(backends.select_backend(), backends.NativePagedBackend)


def test_native_kernel_unavailable_without_rocm_device():
    if torch.cuda.is_available():
        pytest.skip("a ROCm device is visible")
    assert backends.native_kernel_available() is False


# ---- supports / attend / dispatch ------------------------------------------


def test_native_backend_refuses_cpu_store(store):
    # The HIP backend serves every step shape of a GPU store; a CPU store has
    # no packed step, so the hook falls back (attention_backends.py:85-86
    # refuses prefill shapes in the reference for the same effect).
    _, prefill = _prefill_step(store, [4, 2])
    assert prefill.packed is None
    assert backends.NativePagedBackend().supports(prefill, prefill.num_query_tokens) is False
    assert backends.TorchSdpBackend().supports(prefill, prefill.num_query_tokens) is True


def test_native_attend_reports_missing_library(store, monkeypatch):
    _, context = _prefill_step(store, [4, 2])
    monkeypatch.setattr(AVAILABLE, lambda: False)
    with pytest.raises(RuntimeError):
        backends.NativePagedBackend().attend(torch.randn(1, NUM_KV_HEADS, 6, HEAD_DIM), store, 0, context,
                                             0.35, 0.0)


def test_dispatch_falls_back_when_backend_refuses_shape(store, monkeypatch):
    _, context = _prefill_step(store, [4, 2])
    q, k, v = (torch.randn(1, NUM_KV_HEADS, 6, HEAD_DIM) for _ in range(3))

    class Refusing(backends.NativePagedBackend):
        calls = 0

        def supports(self, context, num_query_tokens):
            return False

        def attend(self, *args, **kwargs):
            Refusing.calls += 1
            raise AssertionError("attend must not run for a refused shape")

    monkeypatch.setattr(paged_attention, "_BACKEND", Refusing())
    out, weights = paged_attention.paged_attention_forward(_Layer(context), q, k, v, None, dropout=0.0,
                                                           scaling=0.35)
    assert Refusing.calls == 0
    assert out.shape == (1, 6, NUM_KV_HEADS, HEAD_DIM)
    assert weights is None


def test_dispatch_routes_supported_shape_to_backend(store, monkeypatch):
    _, context = _prefill_step(store, [4, 2])
    q, k, v = (torch.randn(1, NUM_KV_HEADS, 6, HEAD_DIM) for _ in range(3))

    class Recording(backends.TorchSdpBackend):
        calls = 0

        def attend(self, *args, **kwargs):
            Recording.calls += 1
            return super().attend(*args, **kwargs)

    monkeypatch.setattr(paged_attention, "_BACKEND", Recording())
    paged_attention.paged_attention_forward(_Layer(context), q, k, v, None, dropout=0.0, scaling=0.35)
    assert Recording.calls == 1


def test_inline_path_equals_installed_torch_backend(store, monkeypatch):
    _, context = _prefill_step(store, [4, 2])
    torch.manual_seed(3)
    q, k, v = (torch.randn(1, NUM_KV_HEADS, 6, HEAD_DIM) for _ in range(3))
    monkeypatch.setattr(paged_attention, "_BACKEND", None)
    inline, _ = paged_attention.paged_attention_forward(_Layer(context), q, k, v, None, scaling=0.35)
    monkeypatch.setattr(paged_attention, "_BACKEND", backends.TorchSdpBackend())
    routed, _ = paged_attention.paged_attention_forward(_Layer(context), q, k, v, None, scaling=0.35)
    assert torch.equal(inline, routed)


# ---- step bookkeeping (test_attention_backends.py:175-243) ----------------


def test_cu_seqlens_and_context_offsets(store):
    _, context = _prefill_step(store, [4, 2, 3])
    assert context.cu_seqlens.tolist() == [0, 4, 6, 9]
    assert context.cu_context_offsets.tolist() == [0, 4, 6, 9]
    assert context.context_lens == [4, 2, 3]
    assert context.num_query_tokens == 9 and context.num_context_tokens == 9


def test_position_ids_prefill_and_decode(store):
    _, context = _prefill_step(store, [4, 2])
    assert context.position_ids(torch.device("cpu")).tolist() == [[0, 1, 2, 3, 0, 1]]
    seqs = []
    other = manager_mod.PagedKVCacheManager(total_blocks=8, block_size=BLOCK_SIZE, num_heads=NUM_KV_HEADS,
                                            head_dim=HEAD_DIM, num_layers=NUM_LAYERS, device="cpu")
    for i, n in enumerate([4, 2]):
        seq = sequence_mod.Request(seq_id=i + 1, prompt_token_ids=list(range(n)))
        other.allocate_prefix_blocks(seq)
        other.allocate_slot_for_next_token(seq)
        seqs.append(seq)
    starts = [s.block_table.get_tokens_count() - 1 for s in seqs]
    decode = paged_attention.PagedStepContext(other, seqs, starts, [1, 1])
    assert decode.position_ids(torch.device("cpu")).tolist() == [[4, 2]]


def test_attention_mask_matches_oracle(store):
    _, context = _prefill_step(store, [4, 2])
    mask = context.attention_mask(torch.device("cpu"))
    assert mask.shape == (1, 1, 6, 6)
    assert mask.numpy().tolist() == op.attention_mask([0, 0], [4, 2]).tolist()


def test_scatter_then_gather_round_trip(store):
    _, context = _prefill_step(store, [4, 2])
    torch.manual_seed(123)
    kv = torch.randn(context.num_context_tokens, NUM_LAYERS, NUM_KV_HEADS, HEAD_DIM)
    store.scatter_kv(kv, kv, context.scatter_slots)
    for layer in range(NUM_LAYERS):
        assert torch.equal(store.gather_layer_keys(layer, context.gather_slots), kv[:, layer])
        assert torch.equal(store.gather_layer_values(layer, context.gather_slots), kv[:, layer])


@pytest.mark.parametrize("num_query_heads", [NUM_KV_HEADS, 6])
def test_torch_backend_matches_closed_form_attention(store, num_query_heads):
    _, context = _prefill_step(store, [4, 2])
    torch.manual_seed(42)
    kv = torch.randn(context.num_context_tokens, NUM_LAYERS, NUM_KV_HEADS, HEAD_DIM)
    store.scatter_kv(kv, kv, context.scatter_slots)
    q = torch.randn(1, num_query_heads, context.num_query_tokens, HEAD_DIM)
    out = backends.TorchSdpBackend().attend(q, store, 0, context, 0.35, 0.0)
    assert out.shape == (1, context.num_query_tokens, num_query_heads, HEAD_DIM)
    # float64 softmax attention written out, GQA by head repetition
    k = store.gather_layer_keys(0, context.gather_slots).double()  # [C, Hkv, D]
    rep = num_query_heads // NUM_KV_HEADS
    k = k.repeat_interleave(rep, dim=1).transpose(0, 1)  # [Hq, C, D]
    mask = context.attention_mask(torch.device("cpu"))[0, 0]
    s = torch.einsum("htd,hcd->htc", q[0].double(), k) * 0.35
    s = s.masked_fill(~mask, float("-inf"))
    want = torch.einsum("htc,hcd->thd", torch.softmax(s, dim=-1), k)
    assert torch.allclose(out[0].double(), want, atol=1e-6)


# ---- manager errors (test_kv_cache.py:50-62,206-225) ----------------------


def _kv_manager():
    return manager_mod.PagedKVCacheManager(total_blocks=10, block_size=4, num_heads=2, head_dim=8,
                                           device="cpu", num_layers=1)


def test_slot_mapping_requires_block_table():
    with pytest.raises(ValueError, match="no block table"):
        _kv_manager().build_slot_mapping([sequence_mod.Request(seq_id=5, prompt_token_ids=[1])], [0], [1])


def test_single_token_write_requires_block_table():
    token = torch.zeros(1, 2, 8)
    with pytest.raises(ValueError, match="no block table"):
        _kv_manager().write_single_token_kv(sequence_mod.Request(seq_id=4, prompt_token_ids=[1]), token, token)


def test_slot_mapping_range_and_length_errors():
    m = _kv_manager()
    seq = sequence_mod.Request(seq_id=1, prompt_token_ids=[1, 2, 3, 4])
    m.allocate_prefix_blocks(seq)
    with pytest.raises(ValueError):
        m.build_slot_mapping([seq], [0], [5])
    with pytest.raises(ValueError):
        m.build_slot_mapping([seq], [0, 1], [4])
    slots = m.build_slot_mapping([seq], [0], [2])
    with pytest.raises(ValueError):
        m.scatter_kv(torch.randn(2, 2, 8), torch.randn(2, 2, 8), slots)


def test_manager_slots_and_tables_match_oracle():
    m = _kv_manager()
    seqs = []
    for i, n in enumerate([3, 7, 1]):
        seq = sequence_mod.Request(seq_id=i + 1, prompt_token_ids=list(range(n)))
        m.allocate_prefix_blocks(seq)
        seqs.append(seq)
    lists = [s.block_table.get_physical_blocks() for s in seqs]
    counts = [3, 7, 1]
    got = m.build_slot_mapping(seqs, [0, 2, 0], [3, 5, 1])
    assert got.tolist() == op.build_slot_mapping(lists, counts, 4, [0, 2, 0], [3, 5, 1]).tolist()
    table, lens = m.build_block_tables(seqs)
    want_table, want_lens = op.build_block_tables(lists, counts)
    assert table.cpu().tolist() == want_table.tolist() and lens.cpu().tolist() == want_lens.tolist()


# ---- host sizing of the GPU work lists -------------------------------------


@pytest.mark.parametrize("partition,tile", [(512, 32), (1024, 16), (32, 128), (100, 4)])
def test_work_counts_match_oracle_work_lists(partition, tile):
    starts = [0, 600, 1100, 0, 7, 2047, 5000]
    counts = [300, 1, 1, 5, 1, 1, 0]
    t, c, ditems, mitems, pitems, ndec, npre = ops.work_counts(starts, counts, partition, tile)
    dec, merge, pre = op.work_items(starts, counts, partition, tile)
    assert (t, c) == (sum(counts), sum(s + n for s, n in zip(starts, counts)))
    assert (ditems, mitems, pitems) == (len(dec), len(merge), len(pre))
    assert (ndec, npre) == (4, 2)


def test_choose_partition_fills_the_chip():
    # 256 decodes x 8 KV heads give two workgroups per resident slot at 4096
    assert ops.choose_partition([3000] * 256, [1] * 256, 8, 32) == 4096
    # the single-head kernel has more resident slots, so it splits more
    assert ops.choose_partition([3000] * 896, [1] * 896, 2, 2) == 2048
    assert ops.choose_partition([3000] * 896, [1] * 896, 2, 8) == 4096
    # fewer sequences get smaller partitions
    assert ops.choose_partition([4095] * 32, [1] * 32, 8, 32) == 512
    # A latency-bound step takes the partition of least modelled time:
    # P x 0.049 us x (active workgroups / 310 when above 310) x waves, plus
    # 2 us per batch of 8 partials of the longest sequence.  4 x 3001
    # tokens, width 8, 1024 slots: 128 -> 768 workgroups, 15.5 + 3 x 2 =
    # 21.5 us; 256 -> 384, 15.5 + 2 x 2 = 19.5; 512 -> 192, 25.1 + 2 = 27.1.
    assert ops.choose_partition([3000] * 4, [1] * 4, 8, 32) == 256
    assert ops.choose_partition([16383] * 4, [1] * 4, 8, 32) == 1024
    # one sequence of 3001: 64 -> 3.8 + 6 x 2 = 15.8; 128 -> 6.3 + 3 x 2 =
    # 12.3; 256 -> 12.5 + 2 x 2 = 16.5
    assert ops.choose_partition([3000], [1], 8, 32) == 128
    assert ops.choose_partition([16383], [1], 8, 32) == 512
    # short contexts (16, 301, 512): 64 -> 3.1 + 2 = 5.1; 128 -> 6.3 + 2
    assert ops.choose_partition([15, 300, 511], [1, 1, 1], 8, 8) == 64
    # a bandwidth-bound tie (the same bytes over more or fewer workgroups,
    # the same merge batches) goes to the shorter partition: 24 x 1024
    # tokens over 768 slots, 128 -> 768 workgroups and 256 -> 384 both
    # model 15.5 + 2 us
    assert ops.choose_partition([1023] * 24, [1] * 24, 8, 32, workgroups_per_item=4, workgroups_per_cu=3) == 128
    # prefill rows do not count as decode work
    assert ops.choose_partition([0, 3000], [500, 1], 8, 32) == 128
    assert ops.choose_partition([0, 16383], [500, 1], 8, 32) == 512
    assert ops.choose_partition([], [], 8) == 64
    assert ops.choose_partition([0], [64], 8) == 64
    # paired KV heads halve the launch width: the same step splits further
    assert ops.choose_partition([3000] * 256, [1] * 256, 8, 32, workgroups_per_item=4) == 2048
    assert ops.choose_partition([3000] * 256, [1] * 256, 8, 8, workgroups_per_item=4) == 2048
    # split query-head groups widen it
    assert ops.choose_partition([3000] * 64, [1] * 64, 8, 128, workgroups_per_item=16) == 2048
    assert ops.choose_partition([3000] * 64, [1] * 64, 8, 128) == 1024
    # the kernel's occupancy sets the resident slots: fewer slots, longer partitions
    assert ops.choose_partition([3000] * 256, [1] * 256, 8, 32, 4, workgroups_per_cu=2) == 4096
    assert ops.choose_partition([3000] * 256, [1] * 256, 8, 32, 4, workgroups_per_cu=8) == 1024
    # a chip with fewer compute units fills at longer partitions
    assert ops.choose_partition([3000] * 256, [1] * 256, 8, 8, 4, compute_units=128) == 4096


# ---- caller-supplied outputs ------------------------------------------------


def test_output_checked_against_what_the_kernels_write():
    """decode / prefill / attention write [T, H_q, D] contiguous rows of the
    cache dtype: any other `out` is refused before a launch."""
    q = torch.zeros(5, 4, 64, dtype=torch.bfloat16)
    cache = torch.zeros(1, 2, 16, 2, 64, dtype=torch.bfloat16)
    ok = torch.empty(5, 4, 64, dtype=torch.bfloat16)
    assert ops._output_for(q, cache, ok) is ok
    alias = torch.empty(1, 5, 4, 64, dtype=torch.bfloat16)
    assert ops._output_for(q, cache, alias).data_ptr() == alias.data_ptr()
    assert ops._output_for(q, cache, None).shape == (5, 4, 64)
    with pytest.raises(ValueError, match="shape"):
        ops._output_for(q, cache, torch.empty(4, 4, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="dtype"):
        ops._output_for(q, cache, torch.empty(5, 4, 64, dtype=torch.float32))
    with pytest.raises(ValueError, match="contiguous"):
        ops._output_for(q, cache, torch.empty(4, 5, 64, dtype=torch.bfloat16).transpose(0, 1))
    with pytest.raises(ValueError, match="is on"):
        ops._output_for(q, cache, torch.empty(5, 4, 64, dtype=torch.bfloat16, device="meta"))


# ---- block-table pool and host swap bookkeeping -----------------------------

alloc_mod = pkg("memory.block_allocator")


def test_pool_rows_track_block_lists_and_queue_updates():
    alloc = alloc_mod.PageAllocator(64, 4, 8, total_cpu_blocks=4)
    pool = alloc_mod.BlockTablePool(rows=2, width=2)
    a, b = alloc_mod.SequenceBlockTable(alloc, pool), alloc_mod.SequenceBlockTable(alloc, pool)
    assert pool.take_updates()[0] is True  # a fresh pool is uploaded whole once
    for _ in range(9):  # 3 blocks: the row grows past width 2
        a.append_token()
    b.append_token()
    rebuild, upd = pool.take_updates()
    assert rebuild and upd.shape == (0, 3)  # growth: rebuilt from the host rows
    assert pool.host[a.row, :3].tolist() == a.get_physical_blocks()
    assert pool.tokens[a.row] == 9 and pool.blocks[a.row] == 3
    for _ in range(4):
        a.append_token()  # tokens 10-13: block 4 at token 13
    rebuild, upd = pool.take_updates()
    assert not rebuild and upd.tolist() == [[a.row, 3, a.get_physical_blocks()[3]]]
    c = alloc_mod.SequenceBlockTable(alloc, pool)  # a third row: the pool doubles its rows
    assert pool.num_rows == 4 and c.row not in (a.row, b.row)
    pool.take_updates()
    row = a.row
    a.release()
    rebuild, upd = pool.take_updates()
    assert not rebuild and sorted(upd.tolist()) == [[row, col, -1] for col in range(4)]
    assert (pool.host[row] == -1).all() and pool.tokens[row] == 0
    assert alloc.get_num_free_blocks() == 64 - 1  # b's block only


def test_pool_updates_unique_after_release_and_reuse():
    """A row freed and taken again before the next step queues its -1 resets
    and then its new blocks for the same (row, col).  The packing kernel
    stores the triples in no fixed order, so the queue handed over must hold
    each (row, col) once, with the last value: applied in any order, it
    turns the previous device copy into the host rows."""
    rng = np.random.default_rng(3)
    alloc = alloc_mod.PageAllocator(256, 4, 8, total_cpu_blocks=16)
    pool = alloc_mod.BlockTablePool(rows=8, width=8)
    live = [alloc_mod.SequenceBlockTable(alloc, pool) for _ in range(5)]
    for t in live:
        t.append_tokens(int(rng.integers(1, 20)))
    assert pool.take_updates()[0]  # first upload: the whole table
    device = pool.host.copy()
    for step in range(40):
        # free some sequences, then admit new ones: LIFO rows are reused at once
        for _ in range(int(rng.integers(0, 3))):
            if live:
                live.pop(int(rng.integers(0, len(live)))).release()
        for _ in range(int(rng.integers(0, 3))):
            t = alloc_mod.SequenceBlockTable(alloc, pool)
            t.append_tokens(int(rng.integers(1, 12)))
            live.append(t)
        if live and step % 5 == 2:  # a swap-style detach: row released and re-acquired
            t = live[int(rng.integers(0, len(live)))]
            blocks = t.take_blocks()
            t.put_blocks(blocks)
        for t in live:
            t.append_tokens(int(rng.integers(0, 6)))
        rebuild, upd = pool.take_updates()
        if rebuild:
            device = pool.host.copy()
            continue
        keys = upd[:, 0].astype(np.int64) * pool.width + upd[:, 1]
        assert np.unique(keys).shape[0] == keys.shape[0], f"duplicate (row, col) at step {step}"
        for order in (upd, upd[::-1], upd[rng.permutation(upd.shape[0])]):
            got = device.copy()
            got[order[:, 0], order[:, 1]] = order[:, 2]
            assert (got == pool.host).all(), f"step {step}"
        device[upd[:, 0], upd[:, 1]] = upd[:, 2]
    # a release followed by a reuse of the same row within one step
    t = live[0]
    row = t.row
    t.release()
    u = alloc_mod.SequenceBlockTable(alloc, pool)
    assert u.row == row
    u.append_tokens(5)
    rebuild, upd = pool.take_updates()
    assert not rebuild
    entries = {(r, c): b for r, c, b in upd.tolist()}
    assert len(entries) == upd.shape[0]
    for col, block in enumerate(u.get_physical_blocks()):
        assert entries[(row, col)] == block


def test_swap_bookkeeping_matches_reference_messages():
    alloc = alloc_mod.PageAllocator(4, 4, 8, total_cpu_blocks=2)
    blocks = alloc.allocate_blocks(3)
    cpu = alloc.swap_out(blocks[0])
    assert alloc.get_num_free_blocks() == 2 and alloc.get_num_free_cpu_blocks() == 1
    assert alloc.get_cpu_block_id(blocks[0]) == cpu
    alloc.share_block(blocks[1])
    with pytest.raises(RuntimeError, match="ref_count != 1"):
        alloc.swap_out(blocks[1])
    alloc.swap_out(blocks[2])
    alloc.allocate_block()
    with pytest.raises(RuntimeError, match="Host RAM Block Pool exhausted"):
        alloc.swap_out(alloc.allocate_block())
    gpu = alloc.swap_in(cpu)
    assert alloc.get_num_free_cpu_blocks() == 1 and 0 <= gpu < 4
    with pytest.raises(RuntimeError, match="not currently swapped out"):
        alloc.swap_in(cpu)
    with pytest.raises(IndexError, match="CPU block ID out of range"):
        alloc.release_swapped_block(7)
    none = alloc_mod.PageAllocator(4, 4, 8, total_cpu_blocks=0)
    with pytest.raises(RuntimeError, match="no host pool configured"):
        none.swap_out(none.allocate_block())


def test_swap_needs_a_device_store(store):
    seqs, _ = _prefill_step(store, [4])
    with pytest.raises(RuntimeError, match="device memory"):
        store.swap_out(seqs[0])


def test_cpu_store_slots_match_oracle_after_growth():
    """Slots from the pool's host rows equal the oracle's per-sequence
    formula, also after rows and columns grew."""
    m = manager_mod.PagedKVCacheManager(total_blocks=400, block_size=4, num_heads=2, head_dim=8, device="cpu")
    rng = __import__("numpy").random.default_rng(5)
    seqs = []
    for i in range(70):  # more rows than the pool starts with
        seq = sequence_mod.Request(seq_id=i + 1, prompt_token_ids=list(range(int(rng.integers(1, 30)))))
        m.allocate_prefix_blocks(seq)
        seqs.append(seq)
    lists = [s.block_table.get_physical_blocks() for s in seqs]
    toks = [s.block_table.get_tokens_count() for s in seqs]
    starts = [int(rng.integers(0, t)) for t in toks]
    counts = [t - s for s, t in zip(starts, toks)]
    got = m.build_slot_mapping(seqs, starts, counts)
    assert got.tolist() == op.build_slot_mapping(lists, toks, 4, starts, counts).tolist()
    table, lens = m.build_block_tables(seqs)
    want_table, want_lens = op.build_block_tables(lists, toks)
    assert table.tolist() == want_table.tolist() and lens.tolist() == want_lens.tolist()


def test_append_tokens_equals_repeated_append_token():
    for start in (0, 1, 3, 4, 9):
        for n in (0, 1, 2, 4, 7, 16):
            tables = []
            for bulk in (True, False):
                alloc = alloc_mod.PageAllocator(64, 4, 8)
                pool = alloc_mod.BlockTablePool()
                t = alloc_mod.SequenceBlockTable(alloc, pool)
                for _ in range(start):
                    t.append_token()
                if bulk:
                    t.append_tokens(n)
                else:
                    for _ in range(n):
                        t.append_token()
                tables.append((t.get_physical_blocks(), t.get_tokens_count(), pool.host.copy(), pool.tokens.copy()))
            (b1, n1, h1, k1), (b2, n2, h2, k2) = tables
            assert b1 == b2 and n1 == n2 and (h1 == h2).all() and (k1 == k2).all(), (start, n)
