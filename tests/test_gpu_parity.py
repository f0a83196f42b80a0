"""GPU parity of the HIP path against the oracle and the reference's golden vectors.

Integer work (packing, cache write) must be bit-exact.  Attention: fp32
max-abs-err <= 1e-4 against the reference kernel; bf16 inputs against the
reference kernel run on exact fp32 up-casts of the same values, with
max|g - r| / max|r| <= 2e-2 and |g - r| <= 2e-2 |r| + 2e-2 rms(r)
elementwise (helpers.bf16_close).  Full-size workloads are checked on every
sequence (the oracle runs per sequence on the CPU) plus size-independent
properties on the whole batch.
"""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import bf16_close, load_golden, pkg, sha256
from oracle import attention as oa
from oracle import packing as op

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu

ops = pkg("paged_ops")
wl = pkg("workloads")

FP32_TOL = 1e-4


def log(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------------
# helpers


def pack_workload(w, device, prefill_tile=None, with_gather=False, partition=None):
    table = torch.from_numpy(w.block_table_array()).to(device)
    tile = prefill_tile or ops.prefill_tile_for(w.num_query_heads, w.num_kv_heads)
    return ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                         prefill_tile=tile, with_gather=with_gather, partition_size=partition,
                         num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads,
                         head_dim=w.head_dim, dtype=w.dtype)


def oracle_rows(w, t, seqs):
    """Oracle output rows ([n_i, H_q, D] fp32 per sequence) for `seqs`, on
    fp32 copies of exactly the values the GPU read."""
    cu = op.cumulative_offsets(w.new_token_counts)
    q_all = t.query[0].transpose(0, 1)  # [T, H_q, D]
    out = {}
    for i in seqs:
        blocks = torch.tensor(w.block_lists[i], dtype=torch.long, device=t.key_cache.device)
        k = t.key_cache[:, blocks].float().cpu().numpy()  # [1, nb, bs, H_kv, D]
        v = t.value_cache[:, blocks].float().cpu().numpy()
        nb = len(w.block_lists[i])
        ctx = w.context_lens[i]
        slots = np.arange(nb * w.block_size, dtype=np.int64)[:ctx]
        q = q_all[cu[i] : cu[i + 1]].float().cpu().numpy().transpose(1, 0, 2)  # [H_q, n, D]
        o, _ = oa.paged_attention_per_sequence(q, k, v, 0, [w.start_positions[i]], [w.new_token_counts[i]],
                                               slots, w.scaling)
        out[i] = o
    return out


def check_rows(w, got, ref_rows, fp32):
    cu = op.cumulative_offsets(w.new_token_counts)
    g = got.float().cpu().numpy()
    for i, ref in ref_rows.items():
        rows = g[cu[i] : cu[i + 1]]
        if fp32:
            err = np.max(np.abs(rows - ref))
            assert err <= FP32_TOL, f"seq {i}: max abs err {err}"
        else:
            ok, worst = bf16_close(rows, ref)
            assert ok, f"seq {i}: bf16 relative error {worst}"


def golden_case(name):
    g = load_golden(name)
    if "query" not in g:
        case = make_golden.fp32_mha_decode_case(0)
        assert sha256(case["query"], case["key_cache"], case["value_cache"]) == str(g["input_sha256"])
        g.update({k: case[k] for k in ("query", "key_cache", "value_cache", "gather_slots", "mask")})
    return g


# ---------------------------------------------------------------------------
# (a) packing


def _pack_expect(starts, counts, lists, bs, partition, tile):
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


def _check_pack(step, exp):
    for name in ("cu_seqlens", "cu_context_offsets", "context_lens", "scatter_slots", "position_ids",
                 "decode_items", "merge_items", "prefill_items"):
        got = getattr(step, name).cpu().numpy()
        assert got.dtype == exp[name].dtype, name
        assert np.array_equal(got.reshape(exp[name].shape), exp[name]), name
    g = step.gather_slots.cpu().numpy()
    assert g.dtype == np.int64 and np.array_equal(g, exp["gather_slots"])


@pytest.mark.parametrize("seed,name", [(1, "fp32_mha_decode"), (2, "kv_write_pack"), (5, "mixed_step")])
def test_pack_matches_oracle_on_workloads(device, seed, name):
    w = wl.WORKLOADS[name](seed=seed)
    log(f"pack {name}: B={w.num_seqs} T={w.num_query_tokens} C={w.num_context_tokens}")
    tile = ops.prefill_tile_for(w.num_query_heads, w.num_kv_heads)
    step = pack_workload(w, device, with_gather=True)
    exp = _pack_expect(w.start_positions, w.new_token_counts, w.block_lists, w.block_size,
                       step.partition_size, tile)
    _check_pack(step, exp)


@pytest.mark.parametrize("seed", range(4))
def test_pack_matches_oracle_on_ragged_edges(device, seed):
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([1, 4, 16, 32]))
    b = int(rng.integers(1, 40))
    starts = [int(x) for x in rng.integers(0, 700, size=b)]
    counts = [int(rng.choice([0, 1, 1, 2, int(rng.integers(3, 90))])) for _ in range(b)]
    lists, off = [], 0
    perm = rng.permutation(100000)
    for s, c in zip(starts, counts):
        n = -(-(s + c) // bs)
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    table = torch.from_numpy(op.build_block_tables(lists, [s + c for s, c in zip(starts, counts)])[0]).to(device)
    partition = [None, 32, 512, 100][seed]
    step = ops.pack_step(table, starts, counts, bs, prefill_tile=16, with_gather=True, partition_size=partition)
    _check_pack(step, _pack_expect(starts, counts, lists, bs, step.partition_size, 16))


@pytest.mark.parametrize("seed", range(4))
def test_pack_one_launch_matches_oracle(device, seed):
    """Steps that pa_pack does in one launch (at most 1024 sequences, at most
    32 new tokens and 32 full partitions per sequence, no gather slots):
    every output equals the oracle's, and so does a two-launch re-run of the
    same step that adds the gather slots."""
    rng = np.random.default_rng(100 + seed)
    bs = [16, 1, 32, 4][seed]
    b = [1, 37, 1000, 1024][seed]
    partition = [None, 100, 512, 64][seed]
    starts = [int(x) for x in rng.integers(0, 1900, size=b)]
    counts = [int(rng.choice([0, 1, 1, 1, 1, 2, int(rng.integers(3, 33))])) for _ in range(b)]
    lists, off = [], 0
    perm = rng.permutation(1 << 19)  # enough distinct blocks for 1024 contexts of up to 1932 tokens at bs 4
    for s_, c in zip(starts, counts):
        n = -(-(s_ + c) // bs)
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    table = torch.from_numpy(op.build_block_tables(lists, [s_ + c for s_, c in zip(starts, counts)])[0]).to(device)
    step = ops.pack_step(table, starts, counts, bs, prefill_tile=16, partition_size=partition)
    log(f"one-launch pack B={b} bs={bs} partition={step.partition_size} items={step.num_decode_items}")
    assert step.max_context // step.partition_size <= 32 and max(counts) <= 32
    exp = _pack_expect(starts, counts, lists, bs, step.partition_size, 16)
    _check_pack(step, exp)  # reading gather_slots re-runs the step in two launches
    _check_pack(step, exp)


def test_pack_empty_batch(device):
    table = torch.empty((0, 1), dtype=torch.int32, device=device)
    step = ops.pack_step(table, [], [], 16, with_gather=True)
    assert step.cu_seqlens.cpu().tolist() == [0]
    assert step.cu_context_offsets.cpu().tolist() == [0]
    assert step.scatter_slots.numel() == 0 and step.gather_slots.numel() == 0


# ---------------------------------------------------------------------------
# (b) cache write


def test_reshape_and_cache_bit_exact_kv_write_pack(device):
    w = wl.kv_write_pack(seed=2)
    t = wl.make_tensors(w, device, seed=7)
    step = pack_workload(w, device)
    before_k = t.key_cache.view(torch.int16).cpu().numpy().view(np.uint16).copy()
    before_v = t.value_cache.view(torch.int16).cpu().numpy().view(np.uint16).copy()
    # the model's projections arrive as [1, H_kv, T, D]; the hook passes a
    # transposed [T, H_kv, D] view
    k_hf = t.new_keys.transpose(0, 1).contiguous().unsqueeze(0)
    v_hf = t.new_values.transpose(0, 1).contiguous().unsqueeze(0)
    ops.reshape_and_cache(k_hf[0].transpose(0, 1), v_hf[0].transpose(0, 1), t.key_cache, t.value_cache,
                          step.scatter_slots, 0)
    torch.cuda.synchronize()
    slots = op.build_slot_mapping(w.block_lists, w.context_lens, w.block_size, w.start_positions,
                                  w.new_token_counts)
    op.scatter_layer_kv(before_k, 0, t.new_keys.view(torch.int16).cpu().numpy().view(np.uint16), slots)
    op.scatter_layer_kv(before_v, 0, t.new_values.view(torch.int16).cpu().numpy().view(np.uint16), slots)
    assert np.array_equal(t.key_cache.view(torch.int16).cpu().numpy().view(np.uint16), before_k)
    assert np.array_equal(t.value_cache.view(torch.int16).cpu().numpy().view(np.uint16), before_v)


@pytest.mark.parametrize("dtype,head_dim", [(torch.float32, 6), (torch.float32, 8), (torch.bfloat16, 12)])
def test_reshape_and_cache_bit_exact_odd_shapes(device, dtype, head_dim):
    gen = torch.Generator(device=device)
    gen.manual_seed(3)
    L, N, bs, H = 3, 5, 4, 2
    kc = torch.randn((L, N, bs, H, head_dim), generator=gen, device=device).to(dtype)
    vc = torch.randn((L, N, bs, H, head_dim), generator=gen, device=device).to(dtype)
    keys = torch.randn((7, H, head_dim), generator=gen, device=device).to(dtype)
    vals = torch.randn((7, H, head_dim), generator=gen, device=device).to(dtype)
    slots = torch.tensor([0, 5, 19, 3, 8, -1, 100], dtype=torch.int64, device=device)  # last two skipped
    ek, ev = kc.clone(), vc.clone()
    ek[1].view(-1, H, head_dim)[slots[:5]] = keys[:5]
    ev[1].view(-1, H, head_dim)[slots[:5]] = vals[:5]
    ops.reshape_and_cache(keys, vals, kc, vc, slots, 1)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.uint8), ek.view(torch.uint8))
    assert torch.equal(vc.view(torch.uint8), ev.view(torch.uint8))


# ---------------------------------------------------------------------------
# reference ABI and golden vectors


@pytest.mark.parametrize("name", ["fp32_mha_decode", "gqa_prefill", "gqa_decode", "mixed_small", "masked_rows",
                                  "empty_context"])
def test_reference_abi_matches_golden(device, name):
    g = golden_case(name)
    log(f"reference ABI on {name}")
    out = ops.paged_attention_flat(
        torch.from_numpy(g["query"]).to(device), torch.from_numpy(g["key_cache"]).to(device),
        torch.from_numpy(g["value_cache"]).to(device), 0,
        torch.from_numpy(g["gather_slots"].astype(np.int32)).to(device),
        torch.from_numpy(g["mask"].astype(np.uint8)).to(device), float(g["scale"]))
    err = np.max(np.abs(out.cpu().numpy() - g["expected"]), initial=0.0)
    assert err <= FP32_TOL, err


@pytest.mark.parametrize("name", ["fp32_mha_decode", "gqa_prefill", "gqa_decode", "mixed_small"])
def test_block_table_path_matches_golden(device, name):
    g = golden_case(name)
    starts, counts = [int(x) for x in g["starts"]], [int(x) for x in g["counts"]]
    table = torch.from_numpy(g["block_table"]).to(device)
    hq, hkv = int(g["hq"]), int(g["hkv"])
    step = ops.pack_step(table, starts, counts, int(g["bs"]), prefill_tile=ops.prefill_tile_for(hq, hkv))
    q = torch.from_numpy(g["query"]).to(device)
    out = ops.attention(q, torch.from_numpy(g["key_cache"]).to(device),
                        torch.from_numpy(g["value_cache"]).to(device), 0, step, float(g["scale"]))
    err = np.max(np.abs(out.cpu().numpy() - g["expected"][0]))
    assert err <= FP32_TOL, err


# ---------------------------------------------------------------------------
# (c) decode at full size


@pytest.mark.parametrize("seed,name", [(3, "llama7b_mha_decode"), (4, "llama3_8b_gqa_decode")])
def test_decode_bf16_full_size(device, seed, name):
    """Every sequence of the full-size workload (64 MHA and 256 GQA decodes)
    against the oracle."""
    w = wl.WORKLOADS[name](seed=seed)
    log(f"decode {name}: B={w.num_seqs} C={w.num_context_tokens} checking all {w.num_seqs} sequences")
    t = wl.make_tensors(w, device, seed=seed)
    step = pack_workload(w, device)
    out = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    rows = oracle_rows(w, t, range(w.num_seqs))
    assert len(rows) == w.num_seqs
    check_rows(w, out, rows, fp32=False)


def test_decode_fp32_matches_oracle(device):
    w = wl.fp32_mha_decode(seed=11)
    t = wl.make_tensors(w, device, seed=11)
    step = pack_workload(w, device)
    out = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    check_rows(w, out, oracle_rows(w, t, range(w.num_seqs)), fp32=True)


@pytest.mark.parametrize("hq,hkv,d,dtype", [
    (32, 8, 128, torch.bfloat16), (64, 8, 128, torch.bfloat16), (8, 4, 128, torch.bfloat16),
    (4, 4, 128, torch.bfloat16), (16, 16, 64, torch.bfloat16), (8, 4, 64, torch.bfloat16),
    (32, 8, 64, torch.bfloat16), (16, 2, 64, torch.bfloat16), (16, 2, 64, torch.float32),
    (8, 4, 128, torch.float32), (8, 8, 128, torch.float32), (32, 8, 128, torch.float32),
    (8, 1, 64, torch.float32), (12, 4, 32, torch.bfloat16), (12, 4, 128, torch.bfloat16),
    # groups that are not powers of two (9/3/64 is SmolLM-135M's shape)
    (9, 3, 64, torch.bfloat16), (9, 3, 64, torch.float32), (10, 2, 128, torch.bfloat16),
    (12, 2, 64, torch.bfloat16), (28, 4, 128, torch.bfloat16), (14, 2, 128, torch.float32),
    # paired KV heads (bf16, even H_kv): heads of 64 with groups of 3 and 4,
    # heads of 128 with a group of 2
    (24, 8, 64, torch.bfloat16), (16, 8, 128, torch.bfloat16),
    # groups above 8 as sub-groups of at most 8 (16 = 2 x 8, 12 = 2 x 6, 11 = 11 x 1)
    (32, 2, 128, torch.bfloat16), (24, 2, 64, torch.bfloat16), (11, 1, 64, torch.float32),
    # fp16 caches (the reference's LLM_DTYPE=fp16): unpaired, paired, sub-groups
    (32, 8, 128, torch.float16), (40, 8, 128, torch.float16), (16, 8, 64, torch.float16),
    (8, 8, 128, torch.float16), (32, 2, 128, torch.float16), (9, 3, 64, torch.float16),
    # reduce-scatter scores (unpaired groups of more than half a row group):
    # rows of 4 lanes with groups of 3 and 4, rows of 8 with groups of 5-8
    (12, 3, 64, torch.bfloat16), (21, 3, 128, torch.float16), (15, 3, 64, torch.float32),
    # heads of 256 (Gemma's; 16-bit rows of 512 bytes): MHA, groups of 2 and 8,
    # a group of 16 as two sub-groups; fp32 heads of 256 run the generic kernel
    (4, 4, 256, torch.bfloat16), (16, 8, 256, torch.bfloat16), (16, 2, 256, torch.float16),
    (32, 2, 256, torch.bfloat16), (4, 2, 256, torch.float32),
    # heads of 96 (Phi-3-mini) and 80 (Phi-2) on the lane layout of 128 with
    # the pieces past the head masked: MHA, a group of 6 (reduce-scatter
    # scores), fp16, and a group of 12 as two sub-groups
    (8, 8, 96, torch.bfloat16), (24, 4, 96, torch.bfloat16), (8, 8, 80, torch.float16),
    (12, 2, 80, torch.bfloat16), (24, 2, 96, torch.float16), (8, 8, 96, torch.float32),
    (12, 2, 80, torch.float32)])
def test_decode_shapes_and_long_contexts(device, hq, hkv, d, dtype):
    rng = np.random.Generator(np.random.PCG64(hq * 1000 + d))
    ctx = [1, 2, 15, 16, 17, 511, 512, 513, 1024, 3000, 9000]
    need = [-(-c // 16) for c in ctx]
    perm = rng.permutation(sum(need))
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    w = wl.StepWorkload("decode_edges", hq, hkv, d, 16, dtype, 1.0, [c - 1 for c in ctx], [1] * len(ctx),
                        lists, sum(need))
    t = wl.make_tensors(w, device, seed=5)
    step = pack_workload(w, device)
    out = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    check_rows(w, out, oracle_rows(w, t, range(len(ctx))), fp32=dtype == torch.float32)


@pytest.mark.parametrize("bs", [1, 2, 4, 8, 32, 64, 256, 12])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_block_sizes_mixed_step(device, bs, dtype):
    """Decode (every K/V addressing path: per-lane, wave-uniform, 16-row
    runs) and prefill over block sizes from 1 to 256 tokens, plus a
    non-power-of-two size that takes the generic kernel, in one mixed step."""
    starts = [0, 6, 32, 99, 599, 2999, 50]
    counts = [1, 1, 1, 1, 1, 1, 90]
    ctx = [s + c for s, c in zip(starts, counts)]
    rng = np.random.Generator(np.random.PCG64(bs))
    need = [-(-c // bs) for c in ctx]
    perm = rng.permutation(sum(need) + 2)
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    hq, hkv, d = (16, 4, 128) if dtype == torch.bfloat16 else (8, 4, 64)
    w = wl.StepWorkload("block_sizes", hq, hkv, d, bs, dtype, 1.0, starts, counts, lists, sum(need) + 2)
    t = wl.make_tensors(w, device, seed=bs)
    step = pack_workload(w, device, partition=256)
    log(f"block size {bs} {dtype}: decode items {step.num_decode_items}, prefill items {step.num_prefill_items}")
    out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    check_rows(w, out, oracle_rows(w, t, range(w.num_seqs)), fp32=dtype == torch.float32)


@pytest.mark.parametrize("partition", [32, 256, 1024, 2048, 4096, 96, 100, 8192])
def test_decode_partition_sizes(device, partition):
    """Every split-K partition gives the oracle's result: multiples of 32 up
    to 4096 on the fast kernel, others (100, 8192) on the generic one."""
    rng = np.random.Generator(np.random.PCG64(partition))
    ctx = [1, 31, 32, 33, 100, 2047, 2048, 2049, 5000, 4096, 9000]
    need = [-(-c // 16) for c in ctx]
    perm = rng.permutation(sum(need))
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    w = wl.StepWorkload("decode_partitions", 32, 8, 128, 16, torch.bfloat16, 1.0, [c - 1 for c in ctx],
                        [1] * len(ctx), lists, sum(need))
    t = wl.make_tensors(w, device, seed=6)
    step = pack_workload(w, device, partition=partition)
    log(f"decode partition={partition} items={step.num_decode_items} merges={step.num_merge_items}")
    out = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    check_rows(w, out, oracle_rows(w, t, range(len(ctx))), fp32=False)


def test_decode_extremes(device):
    """A 131072-token context next to 2048 short decodes (64-bit offsets, a
    32-partition merge, a grid of ~2100 items)."""
    rng = np.random.Generator(np.random.PCG64(77))
    ctx = [131072] + [int(x) for x in rng.integers(1, 200, size=2048)]
    need = [-(-c // 16) for c in ctx]
    perm = rng.permutation(sum(need))
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    w = wl.StepWorkload("extremes", 32, 8, 128, 16, torch.bfloat16, 1.0, [c - 1 for c in ctx], [1] * len(ctx),
                        lists, sum(need))
    t = wl.make_tensors(w, device, seed=77)
    step = pack_workload(w, device)
    log(f"extremes: partition {step.partition_size}, items {step.num_decode_items}, merges {step.num_merge_items}")
    out = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    check_rows(w, out, oracle_rows(w, t, [0, 1, 2, 1000, 2048]), fp32=False)


def test_decode_occupancy_query(device):
    """The resident workgroups per CU of every tuned decode kernel, as the
    partition choice reads them; unsupported shapes report 0."""
    for dtype in (torch.bfloat16, torch.float32):
        for d in (64, 128):
            for g in range(1, 9):
                per_cu = ops.decode_workgroups_per_cu(dtype, d, 8, 8 * g)
                log(f"occupancy {dtype} D={d} G={g}: {per_cu} per CU, "
                    f"{ops.decode_workgroups_per_item(dtype, d, 8, 8 * g)} workgroups per item")
                assert 1 <= per_cu <= 8
    assert ops.decode_workgroups_per_cu(torch.bfloat16, 128, 2, 32) >= 1  # group 16: two sub-groups
    assert ops.decode_workgroups_per_cu(torch.bfloat16, 256, 8, 16) >= 1  # heads of 256
    assert ops.decode_workgroups_per_cu(torch.bfloat16, 96, 8, 8) >= 1  # masked heads of 96
    assert ops.decode_workgroups_per_cu(torch.float32, 96, 8, 8) >= 1  # fp32 heads of 96
    assert ops.decode_workgroups_per_cu(torch.float32, 256, 8, 8) == 0  # fp32 256: generic kernel
    assert ops.decode_workgroups_per_cu(torch.bfloat16, 112, 8, 8) == 0
    assert ops.decode_workgroups_per_cu(torch.bfloat16, 128, 1, 72) == 0


def test_pack_step_partition_uses_the_kernel_queries(device):
    """pack_step's automatic partition is choose_partition fed with the
    library's launch-shape queries and the device's compute units."""
    for hq, hkv, d, dtype in ((32, 8, 128, torch.bfloat16), (8, 8, 128, torch.float32),
                              (128, 8, 128, torch.bfloat16), (16, 8, 64, torch.float16)):
        w = wl.llama3_8b_gqa_decode(seed=0)
        table = torch.from_numpy(w.block_table_array()).to(device)
        step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                             num_kv_heads=hkv, num_query_heads=hq, head_dim=d, dtype=dtype)
        want = ops.choose_partition(
            w.start_positions, w.new_token_counts, hkv, hq,
            ops.decode_workgroups_per_item(dtype, d, hkv, hq), ops.decode_workgroups_per_cu(dtype, d, hkv, hq),
            torch.cuda.get_device_properties(device).multi_processor_count)
        log(f"partition {hq}/{hkv}/{d} {dtype}: {step.partition_size}")
        assert step.partition_size == want


def test_decode_phases_equal_one_call(device):
    """The partition phase alone gives pa_decode's bits (its last workgroup
    per sequence merges in the launch); the merge phase alone, over the
    partials the partition phase left, rewrites the multi-partition rows
    with the same bits (the merge kernel runs the same arithmetic) and
    touches no other row."""
    w = wl.llama3_8b_gqa_decode(seed=2)
    t = wl.make_tensors(w, device, seed=2)
    step = pack_workload(w, device, partition=512)
    assert step.num_merge_items > 0
    whole = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    split = torch.zeros_like(whole)
    ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=split, phases=1)
    torch.cuda.synchronize()
    assert torch.equal(whole.view(torch.int16), split.view(torch.int16))
    split.fill_(float("nan"))
    ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=split, phases=2)
    torch.cuda.synchronize()
    merged = torch.tensor([c > 512 for c in w.context_lens], device=device)
    assert int(merged.sum()) == step.num_merge_items
    assert torch.equal(whole[merged].view(torch.int16), split[merged].view(torch.int16))
    assert torch.isnan(split[~merged]).all()


def test_decode_with_many_items_merges_in_a_second_launch(device):
    """A step of 76800 decode items (600 sequences of 4096 tokens, partitions
    of 32): too many for the merge records' fields, so the partials are
    merged by a second launch.  Sampled sequences match the oracle, and the
    same step with partitions of 64 (38400 items, merged inside the
    partition launch) agrees within the fp32 tolerance."""
    rng = np.random.Generator(np.random.PCG64(9))
    b, ctx, bs = 600, 4096, 16
    perm = rng.permutation(b * ctx // bs)
    lists = [[int(x) for x in perm[i * ctx // bs : (i + 1) * ctx // bs]] for i in range(b)]
    w = wl.StepWorkload("many_items", 1, 1, 64, bs, torch.float32, 1.0, [ctx - 1] * b, [1] * b, lists,
                        b * ctx // bs)
    t = wl.make_tensors(w, device, seed=9)
    step = pack_workload(w, device, partition=32)
    assert step.num_decode_items == b * ctx // 32 >= 65535 and step.num_merge_items == b
    out = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    other = ops.decode(t.query, t.key_cache, t.value_cache, 0, pack_workload(w, device, partition=64), w.scaling)
    torch.cuda.synchronize()
    check_rows(w, out, oracle_rows(w, t, range(0, b, 15)), fp32=True)
    assert (out - other).abs().max().item() <= FP32_TOL


def test_decode_properties_full_size(device):
    """Size-independent properties on the whole GQA batch: the output depends
    only on logical context (moving blocks + table gives identical bits) and
    not on the other sequences of the batch."""
    w = wl.llama3_8b_gqa_decode(seed=4)
    t = wl.make_tensors(w, device, seed=4)
    step = pack_workload(w, device)
    base = ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    # relocate every block through a permutation of the pool
    gen = torch.Generator()
    gen.manual_seed(1)
    perm = torch.randperm(w.total_blocks, generator=gen)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(w.total_blocks)
    kc = torch.empty_like(t.key_cache)
    vc = torch.empty_like(t.value_cache)
    kc[:, perm.to(device)] = t.key_cache
    vc[:, perm.to(device)] = t.value_cache
    lists = [[int(perm[b]) for b in blocks] for blocks in w.block_lists]
    w2 = wl.StepWorkload(w.name, w.num_query_heads, w.num_kv_heads, w.head_dim, w.block_size, w.dtype, 1.0,
                         w.start_positions, w.new_token_counts, lists, w.total_blocks)
    moved = ops.decode(t.query, kc, vc, 0, pack_workload(w2, device), w.scaling)
    assert torch.equal(base.view(torch.int16), moved.view(torch.int16))
    # batch independence: sequences 10..19 alone
    sub = list(range(10, 20))
    w3 = wl.StepWorkload(w.name, w.num_query_heads, w.num_kv_heads, w.head_dim, w.block_size, w.dtype, 1.0,
                         [w.start_positions[i] for i in sub], [1] * len(sub), [w.block_lists[i] for i in sub],
                         w.total_blocks)
    q_sub = t.query[:, :, 10:20]
    # (the same split-K partition: a different one changes the rounding)
    alone = ops.decode(q_sub, t.key_cache, t.value_cache, 0,
                       pack_workload(w3, device, partition=step.partition_size), w.scaling)
    assert torch.equal(alone.view(torch.int16), base[10:20].view(torch.int16))


# ---------------------------------------------------------------------------
# block copy (copy_blocks)


@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (3, 40, 16, 8, 128)), (torch.float32, (2, 33, 16, 2, 64)),
                                         (torch.bfloat16, (2, 9, 2, 1, 6))])
def test_copy_blocks_bit_exact(device, dtype, shape):
    gen = torch.Generator().manual_seed(11)
    src = torch.randn(shape, generator=gen).to(dtype)
    dst_shape = (shape[0], shape[1] + 5) + shape[2:]
    dst = torch.randn(dst_shape, generator=gen).to(dtype)
    n = shape[1]
    mapping = [(int(s), int(d)) for s, d in zip(torch.randperm(n, generator=gen)[: n // 2],
                                                  torch.randperm(n + 5, generator=gen)[: n // 2])]
    mapping += [(n + 3, 0), (0, n + 9), (-1, 1)]  # out of range: skipped
    bits = torch.int16 if dtype == torch.bfloat16 else torch.int32
    want = dst.view(bits).numpy().copy()
    op.copy_blocks(src.view(bits).numpy(), want, mapping)
    log(f"copy_blocks {dtype} {shape} pairs={len(mapping)}")
    src_d, dst_d = src.to(device), dst.to(device)
    ops.copy_blocks(src_d, dst_d, mapping)
    torch.cuda.synchronize()
    assert np.array_equal(dst_d.cpu().view(bits).numpy(), want)
    assert torch.equal(src_d.cpu().view(bits), src.view(bits))


def test_device_strategy_copy_blocks(device):
    strategies = pkg("memory.strategies")
    strat = strategies.DeviceKVCacheStrategy(device.index or 0)
    k_src, _ = strat.allocate_cache(12, 16, 2, 4, 64, torch.bfloat16)
    k_dst, _ = strat.allocate_cache(12, 16, 2, 4, 64, torch.bfloat16)
    k_src.copy_(torch.randn(k_src.shape, device=device).to(torch.bfloat16))
    strat.copy_blocks(k_src, k_dst, [3, 7, 11])
    strat.sync()
    for b in range(12):
        want = k_src[:, b] if b in (3, 7, 11) else torch.zeros_like(k_src[:, b])
        assert torch.equal(k_dst[:, b].view(torch.int16), want.view(torch.int16))


# ---------------------------------------------------------------------------
# (d) prefill


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 128), (16, 2, 64), (8, 1, 64),
                                     (9, 3, 64), (12, 4, 128), (10, 2, 128), (12, 2, 64), (28, 4, 128),
                                     # groups above 8: sub-groups of 8 and of 6 query heads
                                     (32, 2, 128), (24, 2, 64),
                                     # heads of 96 (Phi-3-mini) and 80 (Phi-2) on rows of 128
                                     (8, 8, 96), (24, 4, 96), (12, 2, 80), (32, 32, 80),
                                     # heads of 256 (Gemma): the one-wave-per-SIMD kernel
                                     (16, 16, 256), (16, 8, 256), (8, 1, 256), (24, 2, 256)])
def test_prefill_bf16_matches_oracle(device, hq, hkv, d):
    _prefill_case(device, hq, hkv, d, torch.bfloat16)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 2, 64), (32, 2, 128), (8, 8, 80), (16, 4, 96),
                                     (16, 4, 256)])
def test_prefill_fp16_matches_oracle(device, hq, hkv, d):
    """fp16 caches run the same MFMA kernel with the f16 MFMA (the reference's
    LLM_DTYPE=fp16, app/memory/strategies.py:14-33)."""
    _prefill_case(device, hq, hkv, d, torch.float16)


@pytest.mark.parametrize("hq,hkv,d,dtype,bs", [(32, 8, 128, torch.bfloat16, 16), (16, 2, 64, torch.float16, 16),
                                              (32, 8, 128, torch.bfloat16, 4), (24, 4, 96, torch.bfloat16, 32),
                                              # a group of 16: two sub-group units per item and KV head
                                              (32, 2, 128, torch.bfloat16, 16),
                                              # fp32 on the matrix cores, blocks of 16, 1 and 4
                                              (32, 8, 128, torch.float32, 16), (16, 4, 128, torch.float32, 1),
                                              (16, 2, 64, torch.float32, 4)])
def test_prefill_many_units_matches_oracle(device, hq, hkv, d, dtype, bs):
    """Several times more (query tile, KV head) units than CUs, of ragged
    lengths and starts, with decodes mixed in: each prefill workgroup walks
    several units in turn (the rounds of its longest/shortest order), and
    every sequence's rows are checked against the oracle."""
    rng = np.random.Generator(np.random.PCG64(1000 + hq + d + bs))
    counts = [int(c) for c in rng.integers(1, 256, size=40)]
    counts[::7] = [1] * len(counts[::7])  # decodes between the chunks
    starts = [int(s) for s in rng.integers(0, 900, size=40)]
    ctx = [s + c for s, c in zip(starts, counts)]
    lists, total = wl._block_tables(rng, ctx, bs, pool=sum(-(-c // bs) for c in ctx) + 5)
    w = wl.StepWorkload("prefill_many_units", hq, hkv, d, bs, dtype, 1.0, starts, counts, lists, total)
    t = wl.make_tensors(w, device, seed=11)
    step = pack_workload(w, device)
    units = step.num_prefill_items * hkv * max(1, (hq // hkv) // 8)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    log(f"prefill many units {dtype} hq={hq} hkv={hkv} d={d} bs={bs} items={step.num_prefill_items} "
        f"units~{units} cus={cus}")
    assert units > 2 * cus
    out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    check_rows(w, out, oracle_rows(w, t, range(w.num_seqs)), fp32=dtype == torch.float32)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (16, 2, 64), (32, 2, 128), (9, 3, 64)])
def test_prefill_fp32_matches_oracle(device, hq, hkv, d):
    """fp32 caches prefill on the fp32 MFMA kernel (fp32 products and
    accumulation throughout), to 1e-4."""
    _prefill_case(device, hq, hkv, d, torch.float32)


@pytest.mark.parametrize("hq,hkv,d,dtype", [(32, 8, 128, torch.bfloat16), (16, 2, 64, torch.float16),
                                           (8, 8, 64, torch.float32), (8, 2, 80, torch.bfloat16),
                                           (16, 4, 256, torch.bfloat16)])
def test_attention_skips_out_of_pool_blocks(device, hq, hkv, d, dtype):
    """Block ids outside [0, total_blocks) (negative or past the pool) in a
    step's table: the positions they cover are skipped by every kernel --
    the MFMA prefill (bf16, fp16), the fp32 prefill, the generic kernel (head
    dim 80) and decode -- and the result is the closed-form attention over
    the remaining positions (float64)."""
    starts, counts = [100, 0, 300, 40], [40, 70, 1, 33]
    bs = 16
    rng = np.random.Generator(np.random.PCG64(d + hq))
    ctx = [s_ + c for s_, c in zip(starts, counts)]
    need = [-(-c // bs) for c in ctx]
    total = sum(need) + 2
    perm = rng.permutation(total)
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    w = wl.StepWorkload("bad_block_ids", hq, hkv, d, bs, dtype, 1.0, starts, counts, lists, total)
    t = wl.make_tensors(w, device, seed=4)
    table = torch.from_numpy(w.block_table_array()).to(device)
    tile = ops.prefill_tile_for(hq, hkv)
    step = ops.pack_step(table, starts, counts, bs, prefill_tile=tile, num_kv_heads=hkv, num_query_heads=hq,
                         head_dim=d, dtype=dtype)
    bad = {(0, 2): -7, (1, 1): total + 3, (2, 5): -1, (2, 17): total, (3, 0): -2}
    host_table = w.block_table_array().copy()
    for (r, c), b in bad.items():
        host_table[r, c] = b
    table.copy_(torch.from_numpy(host_table))  # the kernels read the caller's table in place
    out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    log(f"out-of-pool ids {dtype} {hq}/{hkv}/{d}: prefill items {step.num_prefill_items}")

    kc = t.key_cache[0].float().cpu().numpy()  # [N, bs, H_kv, D]
    vc = t.value_cache[0].float().cpu().numpy()
    q_all = t.query[0].float().cpu().numpy()  # [H_q, T, D]
    got = out.float().cpu().numpy()
    cu = op.cumulative_offsets(counts)
    for i in range(len(starts)):
        pos = np.arange(ctx[i])
        blocks = host_table[i, pos // bs]
        valid = (blocks >= 0) & (blocks < total)
        safe = np.where(valid, blocks, 0)
        keys = kc[safe, pos % bs].transpose(1, 0, 2)  # [H_kv, ctx, D]
        vals = vc[safe, pos % bs].transpose(1, 0, 2)
        mask = (pos[None, :] <= starts[i] + np.arange(counts[i])[:, None]) & valid[None, :]
        want = oa.attention_f64(q_all[:, cu[i] : cu[i + 1]], keys, vals, mask, w.scaling)
        rows = got[cu[i] : cu[i + 1]]
        if dtype == torch.float32:
            assert np.max(np.abs(rows - want)) <= FP32_TOL, i
        else:
            ok, worst = bf16_close(rows, want)
            assert ok, f"seq {i}: relative error {worst}"


@pytest.mark.parametrize("hq,hkv,d,dtype", [(32, 8, 128, torch.bfloat16), (8, 8, 64, torch.float32),
                                           (16, 4, 256, torch.float16), (16, 4, 80, torch.bfloat16),
                                           (32, 8, 128, torch.float32)])
def test_attention_rows_outside_the_pool(device, hq, hkv, d, dtype):
    """A step packed from a pool of table rows in which two sequences (one
    prefill chunk, one decode) name a row outside the pool (past its end, and
    -1): such a row reads as all -1, so those sequences attend no position
    and their outputs are exactly zero, while every other sequence, read from
    its shuffled pool row, equals the oracle -- the MFMA prefill (heads of
    128 and of 80 on rows of 128), the heads-of-256 prefill, the fp32
    prefill and decode."""
    starts, counts = [100, 0, 300, 40, 700, 9], [40, 70, 1, 33, 1, 150]
    outside = {1: 1000, 4: -1}  # sequence -> row outside the pool
    bs = 16
    rng = np.random.Generator(np.random.PCG64(hq + d))
    lists, total = wl._block_tables(rng, [s_ + c for s_, c in zip(starts, counts)], bs, pool=120)
    w = wl.StepWorkload("rows_outside", hq, hkv, d, bs, dtype, 1.0, starts, counts, lists, total)
    t = wl.make_tensors(w, device, seed=5)
    table = w.block_table_array()
    b = len(starts)
    pool_rows = b + 3
    place = rng.permutation(pool_rows)[:b]
    pool = np.full((pool_rows, table.shape[1]), -1, dtype=np.int32)
    pool[place] = table
    rows = place.astype(np.int32)
    for i, r in outside.items():
        rows[i] = r
    tile = ops.prefill_tile_for(hq, hkv)
    step = ops.pack_step(torch.from_numpy(pool).to(device), starts, counts, bs, rows=rows, prefill_tile=tile,
                         num_kv_heads=hkv, num_query_heads=hq, head_dim=d, dtype=dtype)
    out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    log(f"rows outside the pool {dtype} {hq}/{hkv}/{d}: prefill items {step.num_prefill_items}, "
        f"decode items {step.num_decode_items}")
    cu = op.cumulative_offsets(counts)
    for i in outside:
        got = out[cu[i] : cu[i + 1]]
        assert torch.count_nonzero(got).item() == 0, f"seq {i}"
    inside = [i for i in range(b) if i not in outside]
    check_rows(w, out, oracle_rows(w, t, inside), fp32=dtype == torch.float32)


def _bits(t):
    return t.view({torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[t.dtype])


@pytest.mark.parametrize("hq,hkv,d,dtype", [(32, 8, 128, torch.bfloat16), (64, 8, 128, torch.bfloat16),
                                           (32, 2, 128, torch.bfloat16), (8, 8, 64, torch.float32),
                                           (16, 4, 80, torch.bfloat16), (16, 4, 256, torch.float16),
                                           (12, 4, 96, torch.float32), (16, 8, 64, torch.float16)])
def test_decode_append_equals_write_then_decode(device, hq, hkv, d, dtype):
    """A decode step given its new K/V rows (the rows written inside the decode
    launches, pa_decode_append) leaves the same cache bytes and returns the
    same output bits as pa_reshape_and_cache followed by pa_decode -- paired
    heads, groups of 8, sub-groups, heads of 80, 96 and 256, fp32 and fp16,
    strided rows (the model's head-major view), and one sequence whose last
    block id lies outside the pool (written by neither)."""
    rng = np.random.Generator(np.random.PCG64(hq * 7 + d))
    ctx = [int(c) for c in np.clip(np.round(rng.lognormal(np.log(600.0), 1.0, size=24)), 1, 5000)]
    ctx[0], ctx[1] = 1, 4096  # a one-token context and a full multi-partition one
    need = [-(-c // 16) for c in ctx]
    total = sum(need) + 4
    perm = rng.permutation(total)
    lists, off = [], 0
    for n_ in need:
        lists.append([int(x) for x in perm[off : off + n_]])
        off += n_
    w = wl.StepWorkload("decode_append", hq, hkv, d, 16, dtype, 1.0, [c - 1 for c in ctx], [1] * len(ctx),
                        lists, total)
    t = wl.make_tensors(w, device, seed=3)
    table_np = w.block_table_array()
    table_np[5, need[5] - 1] = total + 3  # the last block of sequence 5 is outside the pool
    table = torch.from_numpy(table_np).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, 16, partition_size=512,
                         num_kv_heads=hkv, num_query_heads=hq, head_dim=d, dtype=dtype)
    # the model hands over its head-major projections: token stride D, head stride T * D
    nk = t.new_keys.transpose(0, 1).contiguous().transpose(0, 1)
    nv = t.new_values.transpose(0, 1).contiguous().transpose(0, 1)
    kc2, vc2 = t.key_cache.clone(), t.value_cache.clone()
    ops.reshape_and_cache(nk, nv, t.key_cache, t.value_cache, step.scatter_slots, 0)
    want = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    got = ops.attention(t.query, kc2, vc2, 0, step, w.scaling, new_key=nk, new_value=nv)
    torch.cuda.synchronize()
    log(f"decode append {dtype} {hq}/{hkv}/{d}: items {step.num_decode_items}, merges {step.num_merge_items}")
    assert not step.__dict__.get("_no_append"), "the fused write was not taken"
    assert torch.equal(_bits(kc2), _bits(t.key_cache)) and torch.equal(_bits(vc2), _bits(t.value_cache))
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("bs,partition", [(1, 4096), (1, 2048), (2, 4096)])
def test_decode_append_with_small_blocks_and_long_partitions(device, bs, partition):
    """The decode launch's fused write where the partition's block ids fill
    the LDS that otherwise parks the new rows (one-token blocks, partition
    4096: the rows are stored before the staging barrier) and where they
    leave room (the rows parked and stored by the last tile's wave): the
    same cache bytes and output bits as pa_reshape_and_cache + pa_decode."""
    rng = np.random.Generator(np.random.PCG64(bs * 7 + partition))
    hq, hkv, d, dtype = 16, 4, 128, torch.bfloat16
    ctx = [int(c) for c in rng.integers(1, 9000, size=6)] + [4096, 4097, 1]
    need = [-(-c // bs) for c in ctx]
    total = sum(need) + 4
    perm = rng.permutation(total)
    lists, off = [], 0
    for n_ in need:
        lists.append([int(x) for x in perm[off : off + n_]])
        off += n_
    w = wl.StepWorkload("decode_append_small_blocks", hq, hkv, d, bs, dtype, 1.0, [c - 1 for c in ctx],
                        [1] * len(ctx), lists, total)
    t = wl.make_tensors(w, device, seed=8)
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, bs, partition_size=partition,
                         num_kv_heads=hkv, num_query_heads=hq, head_dim=d, dtype=dtype)
    kc2, vc2 = t.key_cache.clone(), t.value_cache.clone()
    ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
    want = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    got = ops.attention(t.query, kc2, vc2, 0, step, w.scaling, new_key=t.new_keys, new_value=t.new_values)
    torch.cuda.synchronize()
    log(f"decode append bs {bs} partition {step.partition_size}: items {step.num_decode_items}")
    assert step.partition_size == partition
    assert not step.__dict__.get("_no_append"), "the fused write was not taken"
    assert torch.equal(_bits(kc2), _bits(t.key_cache)) and torch.equal(_bits(vc2), _bits(t.value_cache))
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("fused_prefill_write", [True, None])
def test_attention_with_new_rows_on_a_mixed_step(device, fused_prefill_write):
    """The mixed step (four 512-token chunks + 128 long decodes) given its new
    rows writes them inside its prefill and decode launches (or, by default,
    with the cache-write kernel ahead of the plain launches): the same cache
    bytes and output bits as writing them beforehand."""
    w = wl.WORKLOADS["mixed_step"](seed=2)
    t = wl.make_tensors(w, device, seed=2)
    step = pack_workload(w, device)
    kc2, vc2 = t.key_cache.clone(), t.value_cache.clone()
    ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
    want = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    got = ops.attention(t.query, kc2, vc2, 0, step, w.scaling, new_key=t.new_keys, new_value=t.new_values,
                        fused_prefill_write=fused_prefill_write)
    torch.cuda.synchronize()
    assert not step.__dict__.get("_no_append"), "a fused write was declined"
    assert torch.equal(_bits(kc2), _bits(t.key_cache)) and torch.equal(_bits(vc2), _bits(t.value_cache))
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("hq,hkv,d,dtype,bs,fused", [
    (32, 8, 128, torch.bfloat16, 16, True), (16, 16, 128, torch.float16, 32, True),
    (64, 4, 128, torch.bfloat16, 16, True), (16, 2, 96, torch.bfloat16, 16, True),
    (16, 4, 80, torch.float16, 8, True), (8, 8, 64, torch.bfloat16, 1, True),
    (32, 8, 128, torch.float32, 16, True), (8, 8, 64, torch.float32, 4, True),
    (16, 1, 64, torch.float32, 16, True), (16, 4, 256, torch.bfloat16, 16, False)])
def test_prefill_append_equals_write_then_prefill(device, hq, hkv, d, dtype, bs, fused):
    """A step with prefill chunks given its new K/V rows (written inside the
    prefill launch, pa_prefill_append, and the decode launches) leaves the
    same cache bytes and returns the same output bits as pa_reshape_and_cache
    followed by pa_prefill and pa_decode: chunks at 0 and mid-context, one
    ragged and one of two tokens, a one-token sequence beside them, groups
    of 1-16 (sub-groups), heads of 64-128 in every dtype, block sizes 1-32,
    head-major new rows (the model's projections), and chunk positions in a
    block outside the pool and in a column without a block (written by
    neither, masked by both).  Heads of 256 decline the fused write and take
    the cache-write kernel."""
    rng = np.random.Generator(np.random.PCG64(hq * 31 + d + bs))
    starts = [0, 0, 37, 512, 100, 5, 3000, 250]
    counts = [1, 200, 64, 300, 7, 129, 2, 131]
    ctx = [s_ + c for s_, c in zip(starts, counts)]
    need = [-(-c // bs) for c in ctx]
    total = sum(need) + 4
    perm = rng.permutation(total)
    lists, off = [], 0
    for n_ in need:
        lists.append([int(x) for x in perm[off : off + n_]])
        off += n_
    w = wl.StepWorkload("prefill_append", hq, hkv, d, bs, dtype, 1.0, starts, counts, lists, total)
    t = wl.make_tensors(w, device, seed=5)
    table_np = w.block_table_array()
    table_np[3, need[3] - 2] = total + 3  # a chunk block of sequence 3 outside the pool
    table_np[7, need[7] - 1] = -1  # the last column of sequence 7 without a block
    table = torch.from_numpy(table_np).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, bs,
                         prefill_tile=ops.prefill_tile_for(hq, hkv), num_kv_heads=hkv, num_query_heads=hq,
                         head_dim=d, dtype=dtype)
    # head-major projections: token stride D, head stride T * D
    nk = t.new_keys.transpose(0, 1).contiguous().transpose(0, 1)
    nv = t.new_values.transpose(0, 1).contiguous().transpose(0, 1)
    kc2, vc2 = t.key_cache.clone(), t.value_cache.clone()
    ops.reshape_and_cache(nk, nv, t.key_cache, t.value_cache, step.scatter_slots, 0)
    want = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    got = ops.attention(t.query, kc2, vc2, 0, step, w.scaling, new_key=nk, new_value=nv, fused_prefill_write=True)
    torch.cuda.synchronize()
    log(f"prefill append {dtype} {hq}/{hkv}/{d} bs {bs}: prefill items {step.num_prefill_items}")
    assert bool(step.__dict__.get("_no_append")) != fused
    assert torch.equal(_bits(kc2), _bits(t.key_cache)) and torch.equal(_bits(vc2), _bits(t.value_cache))
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_writes_on_the_second_layer(device, dtype):
    """The fused writes (prefill and decode) address the layer they are given:
    on a two-layer cache, writing layer 1 leaves layer 0 untouched and gives
    the same layer-1 bytes and output bits as the cache-write kernel."""
    base = wl.prefill_chunks("two_layers", [0, 300, 57], [90, 40, 1], dtype, 16, 4, 128)
    w = wl.StepWorkload("two_layers", 16, 4, 128, 16, dtype, 1.0, base.start_positions, base.new_token_counts,
                        base.block_lists, base.total_blocks, num_layers=2)
    t = wl.make_tensors(w, device, seed=6)
    step = pack_workload(w, device)
    kc2, vc2 = t.key_cache.clone(), t.value_cache.clone()
    ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 1)
    want = ops.attention(t.query, t.key_cache, t.value_cache, 1, step, w.scaling)
    got = ops.attention(t.query, kc2, vc2, 1, step, w.scaling, new_key=t.new_keys, new_value=t.new_values,
                        fused_prefill_write=True)
    torch.cuda.synchronize()
    assert not step.__dict__.get("_no_append")
    assert torch.equal(_bits(kc2), _bits(t.key_cache)) and torch.equal(_bits(vc2), _bits(t.value_cache))
    assert torch.equal(_bits(got), _bits(want))


def test_fp32_steps_write_prefill_rows_with_the_cache_write_kernel(device):
    """By default an fp32 step with prefill tokens writes its rows with the
    cache-write kernel and runs the plain launches (its fused prefill write
    measured slower), with the same cache bytes and output bits."""
    w = wl.prefill_chunks("fp32_policy", [0, 40], [70, 1], torch.float32, 16, 4, 64)
    t = wl.make_tensors(w, device, seed=4)
    step = pack_workload(w, device)
    kc2, vc2 = t.key_cache.clone(), t.value_cache.clone()
    ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
    want = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    got = ops.attention(t.query, kc2, vc2, 0, step, w.scaling, new_key=t.new_keys, new_value=t.new_values)
    torch.cuda.synchronize()
    assert not step.__dict__.get("_no_append")
    assert torch.equal(_bits(kc2), _bits(t.key_cache)) and torch.equal(_bits(vc2), _bits(t.value_cache))
    assert torch.equal(_bits(got), _bits(want))


def _prefill_case(device, hq, hkv, d, dtype):
    starts = [0, 0, 37, 512, 100]
    counts = [1, 200, 64, 300, 7]
    rng = np.random.Generator(np.random.PCG64(hq + d))
    ctx = [s + c for s, c in zip(starts, counts)]
    need = [-(-c // 16) for c in ctx]
    perm = rng.permutation(sum(need) + 3)
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    w = wl.StepWorkload("prefill_edges", hq, hkv, d, 16, dtype, 1.0, starts, counts, lists, sum(need) + 3)
    t = wl.make_tensors(w, device, seed=9)
    step = pack_workload(w, device)
    log(f"prefill {dtype} hq={hq} hkv={hkv} d={d} items={step.num_prefill_items} tile={step.prefill_tile}")
    out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    check_rows(w, out, oracle_rows(w, t, range(w.num_seqs)), fp32=dtype == torch.float32)


# ---------------------------------------------------------------------------
# mixed continuous-batching step


def test_mixed_step_end_to_end(device):
    """4 x 512-token prefill chunks + 128 long-context decodes: pack, write the
    step's K/V, attend -- all on the GPU -- then check the whole K and V
    pools (the oracle's scatter applied to copies taken before the step:
    the written slots hold the new rows, every other byte is untouched) and
    the output rows of all 132 sequences against the oracle."""
    w = wl.mixed_step(seed=5)
    t = wl.make_tensors(w, device, seed=5)
    before = [c.view(torch.int16).cpu().numpy().view(np.uint16) for c in (t.key_cache, t.value_cache)]
    step = pack_workload(w, device)
    ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
    out = ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling)
    torch.cuda.synchronize()
    slots = op.build_slot_mapping(w.block_lists, w.context_lens, w.block_size, w.start_positions,
                                  w.new_token_counts)
    for want, new, cache in zip(before, (t.new_keys, t.new_values), (t.key_cache, t.value_cache)):
        op.scatter_layer_kv(want, 0, new.view(torch.int16).cpu().numpy().view(np.uint16), slots)
        assert np.array_equal(cache.view(torch.int16).cpu().numpy().view(np.uint16), want)
    del before
    log(f"mixed step: checking rows of all {w.num_seqs} sequences")
    rows = oracle_rows(w, t, range(w.num_seqs))
    assert len(rows) == w.num_seqs and sum(c > 1 for c in w.new_token_counts) == 4
    check_rows(w, out, rows, fp32=False)
