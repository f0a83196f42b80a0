"""The per-layer launches of a decode step and of a mixed prefill + decode
step under HIP graph capture.

A serving loop captures its forward pass once per batch shape and replays
it every step.  The attention path must therefore launch only on the
current stream, allocate nothing outside torch's graph pool, synchronise
nothing and record no memset.  Here the K/V write + split-K decode of four
layers is captured once and replayed over several steps (positions advance,
the packing kernel re-runs eagerly into the same tensors between replays,
and eager work runs between replays); every replay must give the bits of
the same launches run eagerly.
"""

import numpy as np
import pytest
import torch

from helpers import pkg

pytestmark = pytest.mark.gpu

ops = pkg("paged_ops")
wl = pkg("workloads")


@pytest.mark.parametrize("in_launch_write", [False, True])
def test_decode_layers_replay_bit_exact(device, in_launch_write):
    """``in_launch_write``: the layers hand their new rows to the attention
    (written inside the decode launches, pa_decode_append) instead of
    writing them with the cache-write kernel first."""
    layers, b, hq, hkv, d, bs = 4, 48, 32, 8, 128, 16
    rng = np.random.Generator(np.random.PCG64(5))
    steps = 3
    # contexts that stay inside their last 1024-token partition for `steps`
    # steps, so the captured launch geometry stays valid
    ctx0 = []
    while len(ctx0) < b:
        c = int(rng.integers(100, 3000))
        if 0 < c % 1024 < 1024 - steps - 1:
            ctx0.append(c)
    need = [-(-(c + steps) // bs) for c in ctx0]
    perm = rng.permutation(sum(need))
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    nblocks = sum(need)
    gen = torch.Generator(device=device).manual_seed(0)

    def rand(*shape):
        return torch.randn(*shape, generator=gen, device=device).to(torch.bfloat16)

    key_cache = rand(layers, nblocks, bs, hkv, d)
    value_cache = rand(layers, nblocks, bs, hkv, d)
    width = max(len(x) for x in lists)
    table = torch.full((b, width), -1, dtype=torch.int32)
    for i, blocks in enumerate(lists):
        table[i, : len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
    table = table.to(device)
    starts = [c - 1 for c in ctx0]
    step = ops.pack_step(table, starts, [1] * b, bs, partition_size=1024, num_kv_heads=hkv, num_query_heads=hq)
    counts = (step.num_decode_items, step.num_merge_items)

    q = [rand(1, hq, b, d) for _ in range(layers)]
    new_k = [rand(b, hkv, d) for _ in range(layers)]
    new_v = [rand(b, hkv, d) for _ in range(layers)]
    out = [torch.empty((b, hq, d), dtype=torch.bfloat16, device=device) for _ in range(layers)]
    scale = d ** -0.5

    def run_layers(outs):
        for l in range(layers):
            if in_launch_write:
                ops.attention(q[l], key_cache, value_cache, l, step, scale, out=outs[l], new_key=new_k[l],
                              new_value=new_v[l])
            else:
                ops.reshape_and_cache(new_k[l], new_v[l], key_cache, value_cache, step.scatter_slots, l)
                ops.decode(q[l], key_cache, value_cache, l, step, scale, out=outs[l])

    run_layers(out)  # warm-up: sizes the workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_layers(out)

    for k in range(steps):
        # next step: every sequence one token further, new inputs
        starts = [s + 1 for s in starts]
        step.repack(starts)
        for l in range(layers):
            q[l].copy_(rand(1, hq, b, d))
            new_k[l].copy_(rand(b, hkv, d))
            new_v[l].copy_(rand(b, hkv, d))
        graph.replay()
        torch.cuda.synchronize()
        replayed = [o.clone() for o in out]
        eager = [torch.empty_like(o) for o in out]
        run_layers(eager)  # the K/V write is idempotent: same slots, same rows
        torch.cuda.synchronize()
        for l in range(layers):
            assert torch.equal(replayed[l].view(torch.int16), eager[l].view(torch.int16)), (k, l)
        assert not in_launch_write or not step.__dict__.get("_no_append")
        # the step geometry the graph was captured for still holds
        assert ops.work_counts(starts, [1] * b, 1024, step.prefill_tile)[2:4] == counts


def test_mixed_step_layers_replay_bit_exact(device):
    """A continuous-batching step with two prefill chunks and 40 decodes,
    captured whole: the packing re-run (from its workspace copy), then per
    layer the K/V write, the persistent MFMA prefill, the split-K decode and
    its merge, for four layers.  Between replays the step moves on (the
    chunks to their next 256 tokens, the decodes one token) by an eager
    repack, new inputs are copied in and the same launches run eagerly;
    every replay gives the eager bits, outputs and caches alike."""
    layers, hq, hkv, d, bs, part = 4, 32, 8, 128, 16, 512
    rng = np.random.Generator(np.random.PCG64(11))
    steps = 3
    n_dec, chunk = 40, 256
    dec_ctx = []
    while len(dec_ctx) < n_dec:  # stays inside its last partition for `steps` steps
        c = int(rng.integers(600, 4000))
        if 0 < c % part < part - steps - 1:
            dec_ctx.append(c)
    pre_start = [int(rng.integers(0, 700)), 0]
    final = [s + chunk * (steps + 1) for s in pre_start] + [c + steps for c in dec_ctx]
    need = [-(-c // bs) for c in final]
    perm = rng.permutation(sum(need))
    lists, off = [], 0
    for n in need:
        lists.append([int(x) for x in perm[off : off + n]])
        off += n
    nblocks = sum(need)
    gen = torch.Generator(device=device).manual_seed(3)

    def rand(*shape):
        return torch.randn(*shape, generator=gen, device=device).to(torch.bfloat16)

    key_cache = rand(layers, nblocks, bs, hkv, d)
    value_cache = rand(layers, nblocks, bs, hkv, d)
    width = max(len(x) for x in lists)
    table = torch.full((len(lists), width), -1, dtype=torch.int32)
    for i, blocks in enumerate(lists):
        table[i, : len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
    table = table.to(device)
    starts = pre_start + [c - 1 for c in dec_ctx]
    counts = [chunk, chunk] + [1] * n_dec
    t = sum(counts)
    step = ops.pack_step(table, starts, counts, bs, partition_size=part, num_kv_heads=hkv, num_query_heads=hq)
    assert step.num_prefill_items > 0 and step.num_merge_items > 0
    sizes = ops.work_counts(starts, counts, part, step.prefill_tile)
    sizes = sizes[:1] + sizes[2:]  # all but the context tokens, which grow

    q = [rand(1, hq, t, d) for _ in range(layers)]
    new_k = [rand(t, hkv, d) for _ in range(layers)]
    new_v = [rand(t, hkv, d) for _ in range(layers)]
    out = [torch.empty((t, hq, d), dtype=torch.bfloat16, device=device) for _ in range(layers)]
    scale = d ** -0.5

    def run_step(outs, rerun):
        if rerun:
            step.rerun()
        for l in range(layers):
            ops.attention(q[l], key_cache, value_cache, l, step, scale, out=outs[l], new_key=new_k[l],
                          new_value=new_v[l])

    run_step(out, True)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_step(out, True)

    for k in range(steps):
        starts = [s + chunk for s in starts[:2]] + [s + 1 for s in starts[2:]]
        step.repack(starts)
        now = ops.work_counts(starts, counts, part, step.prefill_tile)
        assert now[:1] + now[2:] == sizes
        for l in range(layers):
            q[l].copy_(rand(1, hq, t, d))
            new_k[l].copy_(rand(t, hkv, d))
            new_v[l].copy_(rand(t, hkv, d))
        graph.replay()
        torch.cuda.synchronize()
        replayed = [o.clone() for o in out]
        caches = (key_cache.clone(), value_cache.clone())
        eager = [torch.empty_like(o) for o in out]
        run_step(eager, False)  # the K/V write is idempotent: same slots, same rows
        torch.cuda.synchronize()
        for l in range(layers):
            assert torch.equal(replayed[l].view(torch.int16), eager[l].view(torch.int16)), (k, l)
        assert torch.equal(caches[0].view(torch.int16), key_cache.view(torch.int16)), k
        assert torch.equal(caches[1].view(torch.int16), value_cache.view(torch.int16)), k
