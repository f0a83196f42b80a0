"""pa_decode_no_alloc: the decode entry point that allocates nothing.

It runs the same kernels as pa_decode with the split-K partials in the
library's file-scope scratch array instead of a caller workspace, so its
output must equal pa_decode's bit for bit.  Two calls in a row, the second
over a smaller step, check that nothing left in the shared array from the
first call leaks into the second.  A step whose partials exceed the array
is refused before anything is launched.
"""

import math

import numpy as np
import pytest
import torch

from helpers import pkg

pytestmark = pytest.mark.gpu

ops = pkg("paged_ops")
wl = pkg("workloads")
native = pkg("_native")


def log(msg):
    print(msg, flush=True)


def _step(seed, num_seqs, hq, hkv, d, dtype, max_ctx):
    rng = np.random.Generator(np.random.PCG64(seed))
    raw = rng.lognormal(mean=math.log(1024.0), sigma=1.0, size=num_seqs)
    ctx = [int(c) for c in np.clip(np.round(raw), 1, max_ctx)]
    need = [-(-c // 16) for c in ctx]
    perm = rng.permutation(sum(need))
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    return wl.StepWorkload("no_alloc", hq, hkv, d, 16, dtype, 1.0, [c - 1 for c in ctx], [1] * num_seqs,
                           lists, sum(need))


def _no_alloc(lib, t, w, step, out):
    q = t.query[0].transpose(0, 1)  # [T, H_q, D] view
    dims = ops._step_dims(q, t.key_cache, step)
    stream = torch.cuda.current_stream(t.key_cache.device).cuda_stream
    return lib.pa_decode_no_alloc(q.data_ptr(), t.key_cache.data_ptr(), t.value_cache.data_ptr(), 0, dims,
                                  step.block_tables.data_ptr(), step.context_lens.data_ptr(),
                                  step.cu_seqlens.data_ptr(), step.decode_items.data_ptr(), step.num_decode_items,
                                  step.merge_items.data_ptr() if step.num_merge_items else None,
                                  step.num_merge_items, w.scaling, out.data_ptr(), stream)


@pytest.mark.parametrize("hq,hkv,d,dtype", [(32, 8, 128, torch.bfloat16), (8, 8, 64, torch.float32),
                                           (32, 2, 128, torch.float16)])
def test_no_alloc_decode_equals_pa_decode(device, hq, hkv, d, dtype):
    lib = native.load_library()
    # a long step first, then a smaller one on the same (shared) scratch array
    for seed, num_seqs, max_ctx in ((1, 200, 12000), (2, 23, 3000)):
        w = _step(seed, num_seqs, hq, hkv, d, dtype, max_ctx)
        t = wl.make_tensors(w, device, seed=seed)
        table = torch.from_numpy(w.block_table_array()).to(device)
        step = ops.pack_step(table, w.start_positions, w.new_token_counts, 16, num_kv_heads=hkv,
                             num_query_heads=hq, head_dim=d, dtype=dtype)
        need = ops.decode_workspace_bytes(step.num_decode_items, hq, d)
        log(f"no_alloc {dtype} {hq}/{hkv}/{d}: B={num_seqs} items={step.num_decode_items} "
            f"merges={step.num_merge_items} partition={step.partition_size} partials={need} B")
        assert 0 < need <= native.PA_DECODE_SCRATCH_BYTES - native.PA_DECODE_SCRATCH_STATE_BYTES
        assert step.num_merge_items > 0
        want = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
        got = torch.full_like(want, float("nan"))
        rc = _no_alloc(lib, t, w, step, got)
        native.check(rc, "pa_decode_no_alloc")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), (seed, num_seqs)


def test_no_alloc_with_more_merge_records_than_its_region(device):
    """10000 sequences of 16 KV heads need 160000 merge records of 8 bytes,
    more than the array's fixed 1 MiB region holds, while their partials
    still fit: the merge runs as a second launch.  Every tenth sequence spans
    two partitions.  The output equals pa_decode's (whose workspace holds
    every record: merged in the partition launch) bit for bit, and so does
    that of a smaller step afterwards, which merges in place."""
    lib = native.load_library()
    hq = hkv = 16
    d, dtype, part = 64, torch.float32, 64
    for seed, num_seqs in ((3, 10000), (4, 300)):
        rng = np.random.Generator(np.random.PCG64(seed))
        ctx = [int(rng.integers(part + 1, 2 * part + 1)) if i % 10 == 0 else int(rng.integers(1, part + 1))
               for i in range(num_seqs)]
        need = [-(-c // 16) for c in ctx]
        perm = rng.permutation(sum(need))
        lists, off = [], 0
        for n in need:
            lists.append([int(x) for x in perm[off : off + n]])
            off += n
        w = wl.StepWorkload("no_alloc", hq, hkv, d, 16, dtype, 1.0, [c - 1 for c in ctx], [1] * num_seqs,
                            lists, sum(need))
        t = wl.make_tensors(w, device, seed=seed)
        table = torch.from_numpy(w.block_table_array()).to(device)
        step = ops.pack_step(table, w.start_positions, w.new_token_counts, 16, partition_size=part,
                             num_kv_heads=hkv, num_query_heads=hq, head_dim=d, dtype=dtype)
        q = t.query[0].transpose(0, 1)
        dims = ops._step_dims(q, t.key_cache, step)
        records = lib.pa_decode_merge_state_size(dims, step.num_decode_items)
        partials = ops.decode_workspace_bytes(step.num_decode_items, hq, d)
        log(f"no_alloc records: B={num_seqs} items={step.num_decode_items} records={records} B partials={partials} B")
        assert step.num_merge_items == -(-num_seqs // 10)
        assert partials <= native.PA_DECODE_SCRATCH_BYTES - native.PA_DECODE_SCRATCH_STATE_BYTES
        assert (records > native.PA_DECODE_SCRATCH_STATE_BYTES) == (num_seqs == 10000)
        want = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
        got = torch.full_like(want, float("nan"))
        native.check(_no_alloc(lib, t, w, step, got), "pa_decode_no_alloc")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), num_seqs
        del t


def test_no_alloc_refuses_steps_beyond_the_scratch(device):
    """Partials above PA_DECODE_SCRATCH_BYTES: PA_ERR_WORKSPACE, nothing launched
    (the pointers are never dereferenced)."""
    lib = native.load_library()
    dims = native.PaStepDims(num_seqs=1, num_query_tokens=1, num_query_heads=32, num_kv_heads=8, head_dim=128,
                             block_size=16, total_blocks=8, num_layers=1, max_blocks_per_seq=1,
                             partition_size=512, dtype=native.PA_DTYPE_BF16, q_token_stride=4096,
                             q_head_stride=128)
    items = native.PA_DECODE_SCRATCH_BYTES // (32 * 128 * 4) + 1
    fake = [0x10000 * (i + 1) for i in range(8)]
    rc = lib.pa_decode_no_alloc(fake[0], fake[1], fake[2], 0, dims, fake[3], fake[4], fake[5], fake[6], items,
                                None, 0, 1.0, fake[7], None)
    assert rc == native.PA_ERR_WORKSPACE
    assert b"more than the" in lib.pa_last_error_message()
