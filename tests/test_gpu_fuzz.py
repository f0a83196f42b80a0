"""Randomised parity of a whole step on the GPU against the oracle.

Each seed draws a head layout (H_kv in {1, 2, 3, 4, 8}; a group of 1-8, from
seed 32 on also 9, 10, 12 or 16, which run as sub-groups; D 64 or 128,
256 from seed 80 on, 80 or 96 from seed 96 on), a dtype (bf16 or fp32; fp16
from seed 64 on, bf16 or fp16 from seed 80 on), a block size (1-64), a ragged
batch of decodes (contexts 1-700) and prefill chunks (2-90 tokens at starts
0-400) and a split-K partition (automatic or 32-512 tokens); every fourth
seed (seed % 4 == 1) is a decode-only batch.  The step is packed, its new
K/V rows are written into a random non-contiguous pool -- by the cache-write
kernel for even seeds, handed to the attention for odd ones (written inside
the prefill and decode launches) -- decode and prefill run, and
every output row is compared with the oracle run on the cache the GPU read
(fp32 to 1e-4 absolute, bf16 and fp16 to the relative bound of the parity
tests).  This covers the combinations the
fixed-shape tests do not name: paired and unpaired heads of 64 and 128,
groups that do not divide 128, groups above 8, tiny blocks with short
partitions, and prefill chunks beside split-K decodes.  The long cases add
contexts up to 3000, partitions up to 4096, fp32 heads of 80 and 96 and all
three ways of writing the new rows, and compare the whole pools bit-exactly.
"""

import numpy as np
import pytest
import torch

from helpers import pkg
from oracle import packing as op
from test_gpu_parity import check_rows, log, oracle_rows

pytestmark = pytest.mark.gpu

ops = pkg("paged_ops")
wl = pkg("workloads")


def random_case(seed):
    rng = np.random.Generator(np.random.PCG64(1000 + seed))
    hkv = int(rng.choice([1, 2, 3, 4, 8]))
    group = int(rng.integers(1, 9)) if seed < 32 else int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 16]))
    d = int(rng.choice([64, 128]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float32
    if seed >= 64:
        dtype = torch.float16
    if seed >= 80:
        d = 256 if seed < 96 else (96 if seed % 4 < 2 else 80)
        dtype = torch.bfloat16 if seed % 2 else torch.float16
    bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64]))
    starts, counts = [], []
    decode_only = seed % 4 == 1
    for _ in range(int(rng.integers(1, 11))):
        if decode_only or rng.random() < 0.6:
            c = int(rng.integers(1, 700))
            starts.append(c - 1)
            counts.append(1)
        else:
            starts.append(int(rng.integers(0, 400)))
            counts.append(int(rng.integers(2, 90)))
    ctx = [s + c for s, c in zip(starts, counts)]
    need = [-(-c // bs) for c in ctx]
    pool = sum(need) + 5
    perm = rng.permutation(pool)
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    partition = int(rng.choice([0, 32, 64, 256, 512]))
    w = wl.StepWorkload(f"fuzz{seed}", hkv * group, hkv, d, bs, dtype, 1.0, starts, counts, lists, pool)
    return w, (partition or None)


@pytest.mark.parametrize("seed", range(112))
def test_random_steps_match_oracle(device, seed):
    w, partition = random_case(seed)
    log(f"fuzz seed={seed}: H_q={w.num_query_heads} H_kv={w.num_kv_heads} D={w.head_dim} {w.dtype} "
        f"bs={w.block_size} B={w.num_seqs} counts={w.new_token_counts} partition={partition}")
    t = wl.make_tensors(w, device, seed=seed)
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                         partition_size=partition, num_kv_heads=w.num_kv_heads,
                         num_query_heads=w.num_query_heads, head_dim=w.head_dim, dtype=w.dtype)
    if seed % 2:
        out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, new_key=t.new_keys,
                            new_value=t.new_values)
    else:
        ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
        out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    check_rows(w, out, oracle_rows(w, t, range(w.num_seqs)), fp32=w.dtype == torch.float32)


def random_wide_case(seed):
    """A wide step: 40 sequences of ragged decodes and prefill chunks (2-200
    tokens at starts 0-600) over 4 or 8 KV heads, so that the prefill has
    from about 200 to 1600 (query tile, KV head) units and its workgroups
    (one per CU) walk one to several of them."""
    rng = np.random.Generator(np.random.PCG64(5000 + seed))
    hkv = int(rng.choice([4, 8]))
    group = int(rng.choice([2, 4] if hkv == 8 else [2, 4, 8]))
    d = int(rng.choice([64, 128]))
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    bs = int(rng.choice([2, 4, 8, 16, 32]))
    starts, counts = [], []
    for _ in range(40):
        if rng.random() < 0.3:
            c = int(rng.integers(1, 900))
            starts.append(c - 1)
            counts.append(1)
        else:
            starts.append(int(rng.integers(0, 600)))
            counts.append(int(rng.integers(2, 200)))
    ctx = [s + c for s, c in zip(starts, counts)]
    lists, pool = wl._block_tables(rng, ctx, bs, pool=sum(-(-c // bs) for c in ctx) + 7)
    w = wl.StepWorkload(f"wide{seed}", hkv * group, hkv, d, bs, dtype, 1.0, starts, counts, lists, pool)
    return w


@pytest.mark.parametrize("seed", range(12))
def test_random_wide_steps_match_oracle(device, seed):
    w = random_wide_case(seed)
    t = wl.make_tensors(w, device, seed=100 + seed)
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                         num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads, head_dim=w.head_dim,
                         dtype=w.dtype)
    log(f"wide seed={seed}: H_q={w.num_query_heads} H_kv={w.num_kv_heads} D={w.head_dim} {w.dtype} "
        f"bs={w.block_size} prefill units={step.num_prefill_items * w.num_kv_heads}")
    ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
    out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    check_rows(w, out, oracle_rows(w, t, range(w.num_seqs)), fp32=False)


def _bits(x):
    return x.view({torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[x.dtype])


@pytest.mark.parametrize("seed", range(40))
def test_random_steps_fused_write_is_bit_exact(device, seed):
    """The new K/V rows written inside the attention launches (pa_prefill_append
    and pa_decode_append), and by the default policy (which takes the
    cache-write kernel on a step with both kinds of sequences), leave the
    same cache bytes and give the same output bits as writing them with the
    cache-write kernel first, on the random steps above (seeds below 28) and
    the wide ones (28 on), with token-major or head-major new rows, and with
    a random table entry of a multi-token sequence set outside the pool or
    to -1."""
    rng = np.random.Generator(np.random.PCG64(9000 + seed))
    if seed < 28:
        w, partition = random_case(3 * seed + 2)
    else:
        w, partition = random_wide_case(seed - 28), None
    t = wl.make_tensors(w, device, seed=200 + seed)
    table_np = w.block_table_array()
    multi = [i for i, c in enumerate(w.new_token_counts) if c > 1]
    if multi and rng.random() < 0.5:
        i = int(rng.choice(multi))
        col = int(rng.integers(0, len(w.block_lists[i])))
        table_np[i, col] = w.total_blocks + 2 if rng.random() < 0.5 else -1
    table = torch.from_numpy(table_np).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                         partition_size=partition, num_kv_heads=w.num_kv_heads,
                         num_query_heads=w.num_query_heads, head_dim=w.head_dim, dtype=w.dtype)
    nk, nv = t.new_keys, t.new_values
    if seed % 2:  # head-major rows: token stride D, head stride T * D
        nk = nk.transpose(0, 1).contiguous().transpose(0, 1)
        nv = nv.transpose(0, 1).contiguous().transpose(0, 1)
    log(f"fused-write seed={seed}: H_q={w.num_query_heads} H_kv={w.num_kv_heads} D={w.head_dim} {w.dtype} "
        f"bs={w.block_size} B={w.num_seqs} prefill items={step.num_prefill_items}")
    kc2, vc2 = t.key_cache.clone(), t.value_cache.clone()
    kc3, vc3 = t.key_cache.clone(), t.value_cache.clone()
    ops.reshape_and_cache(nk, nv, t.key_cache, t.value_cache, step.scatter_slots, 0)
    want = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    got = ops.attention(t.query, kc2, vc2, 0, step, w.scaling, new_key=nk, new_value=nv, fused_prefill_write=True)
    step.__dict__.pop("_no_append", None)  # (a decline above must not steer the default call)
    got_default = ops.attention(t.query, kc3, vc3, 0, step, w.scaling, new_key=nk, new_value=nv)
    torch.cuda.synchronize()
    assert torch.equal(_bits(kc2), _bits(t.key_cache)) and torch.equal(_bits(vc2), _bits(t.value_cache))
    assert torch.equal(_bits(got), _bits(want))
    assert torch.equal(_bits(kc3), _bits(t.key_cache)) and torch.equal(_bits(vc3), _bits(t.value_cache))
    assert torch.equal(_bits(got_default), _bits(want))


def random_long_case(seed):
    """Any head dim (64, 80, 96, 128, 256) and dtype (fp32 but for heads of
    256), a group of 1-16, a block size of 1-64, up to 12 sequences: decodes
    of contexts up to 3000 and prefill chunks of 2-300 tokens at starts up to
    1500 (capped so the oracle stays fast), as a mixed, decode-only or
    prefill-only batch; a split-K partition of automatic or 32-4096 tokens and
    a K/V write mode: the cache-write kernel first (0), the default policy
    (1) or the prefill's fused write (2)."""
    rng = np.random.Generator(np.random.PCG64(77000 + seed))
    hkv = int(rng.choice([1, 2, 3, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 16]))
    d = int(rng.choice([64, 128, 128, 256, 80, 96]))
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    if d == 256 and dtype == torch.float32:
        dtype = torch.bfloat16
    bs = int(rng.choice([1, 2, 4, 8, 16, 16, 32, 64]))
    budget = 4e8 / (hkv * group * d)  # sum of n * (start + n) over the batch
    kind = int(rng.integers(0, 3))  # 0 mixed, 1 decodes only, 2 prefill chunks only
    starts, counts, cost = [], [], 0
    for _ in range(int(rng.integers(1, 13))):
        if kind == 1 or (kind == 0 and rng.random() < 0.6):
            c = int(rng.integers(1, 3000))
            s, n = c - 1, 1
        else:
            s, n = int(rng.integers(0, 1500)), int(rng.integers(2, 300))
        if starts and cost + n * (s + n) > budget:
            break
        starts.append(s)
        counts.append(n)
        cost += n * (s + n)
    ctx = [s + c for s, c in zip(starts, counts)]
    need = [-(-c // bs) for c in ctx]
    pool = sum(need) + int(rng.integers(1, 40))
    perm = rng.permutation(pool)
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    partition = [None, 32, 64, 128, 256, 512, 1024, 2048, 4096][int(rng.integers(0, 9))]
    mode = int(rng.integers(0, 3))
    w = wl.StepWorkload(f"long{seed}", hkv * group, hkv, d, bs, dtype, 1.0, starts, counts, lists, pool)
    return w, partition, mode


@pytest.mark.parametrize("seed", range(200))
def test_random_long_steps_match_oracle(device, seed):
    """Every output row against the oracle, and the whole K and V pools
    against the pools before the step with the new rows placed at the oracle's
    slots (bit-exact)."""
    w, partition, mode = random_long_case(seed)
    log(f"long seed={seed}: H_q={w.num_query_heads} H_kv={w.num_kv_heads} D={w.head_dim} {w.dtype} "
        f"bs={w.block_size} counts={w.new_token_counts} starts={w.start_positions} partition={partition} "
        f"mode={mode}")
    t = wl.make_tensors(w, device, seed=seed)
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                         partition_size=partition, num_kv_heads=w.num_kv_heads,
                         num_query_heads=w.num_query_heads, head_dim=w.head_dim, dtype=w.dtype)
    want_k, want_v = t.key_cache.clone(), t.value_cache.clone()
    if mode == 0:
        ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
        out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    else:
        out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, new_key=t.new_keys,
                            new_value=t.new_values, fused_prefill_write=True if mode == 2 else None)
    torch.cuda.synchronize()
    slots = op.build_slot_mapping(w.block_lists, w.context_lens, w.block_size, w.start_positions,
                                  w.new_token_counts)
    idx = torch.as_tensor(slots, dtype=torch.long, device=device)
    want_k.view(-1, w.num_kv_heads, w.head_dim)[idx] = t.new_keys
    want_v.view(-1, w.num_kv_heads, w.head_dim)[idx] = t.new_values
    assert torch.equal(_bits(want_k), _bits(t.key_cache)) and torch.equal(_bits(want_v), _bits(t.value_cache))
    check_rows(w, out, oracle_rows(w, t, range(w.num_seqs)), fp32=w.dtype == torch.float32)
