"""Paged-attention benchmark on one MI355X.

Headline workload: Llama-3-8B-shaped GQA decode, bf16 -- 256 sequences, 32
query / 8 KV heads, head_dim 128, block size 16, contexts
clip(round(lognormal(ln 1024, 1.0)), 32, 8192), random non-contiguous block
tables, N(0,1) synthetic values.  A "step" is one decode pass of one layer
over the batch (the HIP split-K partition kernel, which merges the split-K
partials in the same launch), with the batch already packed and resident in
HBM.

value    = algorithmic KV-read GB/s = decode bytes / mean step time, where
           decode bytes = sum_i ctx_i * 2 * H_kv * D * 2 (K+V read once per
           KV head) + q and out rows + block-table entries + context lengths;
tokens/s = sequences / mean step time (one token per sequence per layer).
roofline = the dominant kernel (the split-K partition kernel): its
           algorithmic bytes over its own launch time, measured with HIP
           events around each partition launch on its stream; traffic = its
           HBM bytes per launch from the committed rocprofv3 PMC summary.
Also on the line:
  full_step_ms   a whole step through the product path, host included: the
                 step context built on an HBM store (checks, plan, the
                 inputs handed over in pinned memory, the packing launch),
                 and the attention given the step's new K/V rows (written
                 inside the decode launches for a decode step);
                 full_vs_decode_step times it in alternation with the decode
                 step alone on the same pool and tables (the gap is what
                 the step's plumbing costs);
  host_step_us   the host time of building that step context (median), for
                 this workload and the mixed step;
  graph_step_ms  the decode step replayed from a HIP graph, timed in
                 alternation with the eager loop (graph_vs_eager);
  configs        the other workloads' lines: fp32 MHA decode and the K/V
                 write + packing step timed over rotated pool copies (their
                 data would otherwise sit in the 256 MB MALL), Llama-7B MHA
                 decode, and the mixed prefill + decode step (decode GB/s,
                 tokens/s, the prefill kernel's TFLOP/s against the nominal
                 bf16 MFMA peak and against the rate the device sustains on
                 MFMAs alone, pa_calibrate_mfma), each with its CPU baseline
                 on a bounded sample, each measured by this script in a
                 process of its own (its pool the first large allocation of
                 the process, as a server allocates its KV pool at start-up);
  cpu_baseline   the reference CPU kernel on a bounded sample of the same
                 workload on this host's cores.

--workload prefill_shapes prints one line of the prefill kernel alone on
prefill-only steps of four 512-token chunks (32/8 heads, D=128, bf16 and
fp32, and two small prompt steps), each against its dtype's dense MFMA peak,
the same launch writing the chunks' new K/V rows, and the whole step with
its write from HIP graphs, the cache-write kernel then the prefill against
the fused launch (--shape NAME: one of them).

--workload decode_layers prints, per layer, a model's 32-layer loop over one
bf16 decode step (16, 64 and 256 sequences; each layer writing its rows
inside the decode launch) from eager launches and from one HIP graph of the
32 layers, timed in alternation.

--workload decode_partitions prints, for latency-bound decode steps in a
32-layer loop, the per-layer time of every split-K partition from 64 to 4096
and the partition pa_plan_step picks.

--ab-library PATH [--ab-rounds N] times the workload's kernels and step in
alternation with another build of the library (csrc/build.py --rev REV
--out PATH builds one from a git revision) and prints one comparison line.

python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--no-configs] [--config-line] [--calibrate-mfma]
                [--calibrate-read] [--ab-library PATH [--ab-rounds N]]
                [--workload llama3_8b_gqa_decode|llama7b_mha_decode|mixed_step|fp32_mha_decode|kv_write_pack|
                            prefill_shapes|decode_layers|decode_partitions]
"""

from __future__ import annotations

import argparse
import contextlib
import importlib
import json
import os
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))
PACKAGE = "low-latency-distributed-llm-serving-infrastructure-custom-k8s-control-plane_amd"
METRIC = "paged-attn decode KV-read GB/s (% HBM peak) + decode tokens/s, 1 GPU"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_F32_PEAK_TFLOPS = 157.3
MALL_BYTES = 256 << 20


def pkg(sub):
    return importlib.import_module(PACKAGE + "." + sub)


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def host_desc() -> str:
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return f"host {cpu_model()}, nproc {os.cpu_count()}, OMP_NUM_THREADS {threads}"


def median(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2]


# ---------------------------------------------------------------------------
# CPU baselines (the reference kernel, or the oracle where it is not built)


def _kv_of(w, t, i):
    import numpy as np
    import torch

    blocks = torch.tensor(w.block_lists[i], dtype=torch.long, device=t.key_cache.device)
    k = t.key_cache[:, blocks].float().cpu().numpy()
    v = t.value_cache[:, blocks].float().cpu().numpy()
    slots = np.arange(len(w.block_lists[i]) * w.block_size, dtype=np.int64)[: w.context_lens[i]]
    return k, v, slots


# CPU baselines that take seconds run after every GPU measurement of the
# process, so that no GPU timing follows seconds of an idle GPU.
_DEFERRED = []


def defer_cpu(fn, into: dict, key: str) -> None:
    """Run ``fn`` after the GPU measurements; its result goes to into[key]."""
    _DEFERRED.append((fn, into, key))


def run_deferred() -> None:
    while _DEFERRED:
        fn, into, key = _DEFERRED.pop(0)
        into[key] = fn()


def cpu_baseline_per_sequence(w, t, budget_s: float, which: str = "decode"):
    """The reference kernel, one call per sequence (decode: T=1, all-ones
    mask; prefill chunk: causal-offset mask), on fp32 up-casts of the same
    values.  Sequences of the kind asked for are taken in order until about
    budget_s / 6 seconds of kernel time (a bounded sample), then the sample
    is timed once more as a warm-up plus five times; the median pass is
    reported, with GB/s over the same algorithmic bytes as the GPU's."""
    import numpy as np
    import torch

    from oracle import attention as oa

    kind = "reference" if oa.reference_available() else "port"
    q_all = t.query[0].transpose(0, 1)
    e = 2 if w.dtype != torch.float32 else 4
    qbase = np.concatenate([[0], np.cumsum(w.new_token_counts)])
    sample, spent = [], 0.0
    for i in range(w.num_seqs):
        n = w.new_token_counts[i]
        if (which == "decode") != (n == 1) or n == 0:
            continue
        k, v, slots = _kv_of(w, t, i)
        q = q_all[qbase[i] : qbase[i] + n].float().cpu().numpy().transpose(1, 0, 2)
        _, secs = oa.paged_attention_per_sequence(q, k, v, 0, [w.start_positions[i]], [n], slots, w.scaling,
                                                  kind=kind)
        sample.append((q, k, v, slots, w.start_positions[i], n))
        spent += secs
        if spent >= budget_s / 6:
            break
    passes = []
    for _ in range(5):
        total = 0.0
        for q, k, v, slots, start, n in sample:
            _, secs = oa.paged_attention_per_sequence(q, k, v, 0, [start], [n], slots, w.scaling, kind=kind)
            total += secs
        passes.append(total)
    med = median(passes)
    ctx_tokens = sum(s + n for *_, s, n in sample)
    nbytes = sum((s + n) * 2 * w.num_kv_heads * w.head_dim * e + n * w.num_query_heads * w.head_dim * 2 * e
                 for *_, s, n in sample)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    total_kind = sum(1 for c in w.new_token_counts if (which == "decode") == (c == 1) and c > 0)
    return {
        "value": round(nbytes / med / 1e9, 4),
        "unit": "GB/s",
        "tokens_per_s": round(sum(n for *_, n in sample) / med, 2),
        "cores": threads,
        "kind": kind,
        "sample": (f"first {len(sample)} of {total_kind} {which} sequences ({ctx_tokens} context tokens), one call "
                   f"per sequence ({'T=1, all-ones mask' if which == 'decode' else 'causal-offset mask'}; OpenMP "
                   f"parallelism capped at T*H_q rows), "
                   f"{'fp32 up-casts of the 16-bit' if e == 2 else 'the fp32'} values, median of 5 passes after a "
                   f"warm-up ({med:.3f} s/pass kernel time, steady_clock around the C call); {host_desc()}"),
    }


def cpu_baseline_flat(w, t):
    """The reference's native-backend call for the whole step: one flat call
    with the T x C uint8 mask (app/model/attention_backends.py:97-117)."""
    import numpy as np

    from oracle import attention as oa
    from oracle import packing as op

    kind = "reference" if oa.reference_available() else "port"
    q = t.query.float().cpu().numpy()
    k = t.key_cache.float().cpu().numpy()
    v = t.value_cache.float().cpu().numpy()
    slots = op.build_slot_mapping(w.block_lists, w.context_lens, w.block_size, [0] * w.num_seqs,
                                  w.context_lens).astype(np.int32)
    mask = op.attention_mask(w.start_positions, w.new_token_counts).astype(np.uint8)
    times = []
    for _ in range(6):
        t0 = time.perf_counter()
        oa.paged_attention(q, k, v, 0, slots, mask, w.scaling, kind=kind)
        times.append(time.perf_counter() - t0)
    med = median(times[1:])
    wl = pkg("workloads")
    nbytes = wl.decode_bytes(w)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": round(nbytes / med / 1e9, 4),
        "unit": "GB/s",
        "tokens_per_s": round(w.num_query_tokens / med, 2),
        "cores": threads,
        "kind": kind,
        "sample": (f"the whole step ({w.num_seqs} sequences, {w.num_context_tokens} context tokens): one flat call "
                   f"with the T x C mask, as the reference's native backend makes it; median of 5 after a warm-up "
                   f"({med * 1e3:.3f} ms, wall clock around the call); {host_desc()}"),
    }


# ---------------------------------------------------------------------------
# GPU timing helpers


def graph_ms(fn, reps, warmup, stream):
    """Per-call time of `reps` back-to-back calls captured in one HIP graph
    and replayed between two events: microsecond launches are timed without
    host launch gaps."""
    import torch

    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(reps):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def graph_vs_eager_ms(fn, steps, stream, rounds=3):
    """(eager ms, graph ms) per call: `steps` eager calls and a replay of the
    same `steps` calls captured in one HIP graph, alternated `rounds` times;
    medians.  Alternating matters: the GPU's clock drifts over a run, so a
    graph timed after the eager loop reads slower for reasons of its own."""
    import torch

    fn(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    eager, replay = [], []
    for _ in range(rounds):
        eager.append(timed_ms(lambda: fn(0), steps, 0, stream))
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        replay.append(a.elapsed_time(b) / steps)
    return median(eager), median(replay)


def paired_ms(fn_a, fn_b, steps, stream, rounds=5):
    """(a ms, b ms) per call: `steps` eager calls of each, alternated `rounds`
    times after one untimed pass of both; medians.  Two loops timed in
    alternation see the same clock, so their difference is the cost of what
    b adds, not clock drift."""
    a, b = [], []
    timed_ms(fn_a, steps, 0, stream)
    timed_ms(fn_b, steps, 0, stream)
    for _ in range(rounds):
        a.append(timed_ms(fn_a, steps, 0, stream))
        b.append(timed_ms(fn_b, steps, 0, stream))
    return median(a), median(b)


def timed_ms(fn, steps, warmup, stream):
    """Mean time of `steps` eager calls between two events after `warmup`."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def gpu_spacer():
    """A spin of about 80 us on the current stream, issued after a timed
    launch: the host prepares the next launch meanwhile, so that the next
    start event does not fire on an idle GPU before its launch is queued
    (for launches of tens of microseconds the host's own preparation would
    otherwise be counted in them)."""
    import torch

    torch.cuda._sleep(200_000)


def events_ms(launch, timed, steps, warmup, stream):
    """Average duration of the launches `timed()` issues, bracketed by HIP
    events on the launch stream, with `launch()` issued around them."""
    import torch

    pairs = []
    for i in range(warmup + steps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        timed()
        b.record(stream)
        launch()
        if i >= warmup:
            pairs.append((a, b))
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)


def measured_traffic(workload: str):
    """HBM bytes per launch of the dominant kernel on `workload`, from the
    committed rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE, each scaled
    by what the counter reads for a copy of known size); None if absent."""
    try:
        table = json.loads((REPO / "profiles" / "pmc_traffic.json").read_text())
    except (OSError, ValueError):
        return None
    entry = table.get(workload)
    return int(entry["traffic_bytes"]) if entry else None


def workload_config(w, **extra):
    cfg = {
        "workload": w.name,
        "num_seqs": w.num_seqs,
        "num_query_heads": w.num_query_heads,
        "num_kv_heads": w.num_kv_heads,
        "head_dim": w.head_dim,
        "block_size": w.block_size,
        "context_tokens": w.num_context_tokens,
        "query_tokens": w.num_query_tokens,
    }
    cfg.update(extra)
    return cfg


def calibrate_copy(device, nbytes: int = 1 << 30, reps: int = 5) -> None:
    """A plain device-to-device copy of known size (for scaling the PMC
    FETCH_SIZE / WRITE_SIZE counters of the profiled kernels)."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "reps": reps}), flush=True)


def sustained_mfma_tflops(device, iters: int = 4096, reps: int = 9, warmup: int = 20, valu_per_mfma: int = 0) -> float:
    """The bf16 matrix-core rate the device sustains (pa_calibrate_mfma: two
    independent 32x32x16 MFMA chains per wave on register operands, two
    workgroups of 8 waves per CU), median of `reps` launches timed with HIP
    events after `warmup` untimed ones (the clock settles under the load):
    the ceiling an MFMA kernel's TFLOP/s is read against beside the nominal
    peak."""
    import torch

    native = pkg("_native")
    lib = native.load_library()
    wgs = 2 * torch.cuda.get_device_properties(device).multi_processor_count
    out = torch.empty(wgs * 512, dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device)
    flops = lib.pa_calibrate_mfma_flops(wgs, iters)
    for _ in range(warmup):
        native.check(lib.pa_calibrate_mfma(out.data_ptr(), wgs, iters, valu_per_mfma, stream.cuda_stream),
                     "pa_calibrate_mfma")
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        native.check(lib.pa_calibrate_mfma(out.data_ptr(), wgs, iters, valu_per_mfma, stream.cuda_stream),
                     "pa_calibrate_mfma")
        b.record(stream)
        b.synchronize()
        times.append(a.elapsed_time(b))
    return flops / (median(times) * 1e-3) / 1e12


def sustained_read_gbs(device, nbytes: int, reps: int = 9, warmup: int = 5) -> float:
    """The read rate the device sustains for `nbytes` (pa_calibrate_read: one
    pass of 16-byte non-temporal loads over a fresh buffer of that size, 64
    workgroups of 256 threads per CU), median of `reps` launches timed with
    HIP events after `warmup` untimed ones: the ceiling an HBM-bound kernel's
    GB/s is read against beside the nominal peak.  Measured after the
    workload's own timings, so its pool stays the first large allocation of
    the process."""
    import torch

    native = pkg("_native")
    lib = native.load_library()
    nb = (int(nbytes) + 15) // 16 * 16
    buf = torch.empty(nb, dtype=torch.uint8, device=device)
    buf.fill_(1)
    out = torch.zeros(16, dtype=torch.uint8, device=device)
    wgs = 64 * torch.cuda.get_device_properties(device).multi_processor_count
    stream = torch.cuda.current_stream(device)

    def launch():
        native.check(lib.pa_calibrate_read(buf.data_ptr(), nb, out.data_ptr(), wgs, stream.cuda_stream),
                     "pa_calibrate_read")

    for _ in range(warmup):
        launch()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        launch()
        b.record(stream)
        b.synchronize()
        times.append(a.elapsed_time(b))
    del buf
    torch.cuda.empty_cache()
    return nb / (median(times) * 1e-3) / 1e9


# ---------------------------------------------------------------------------
# the product path's step: an HBM store, its row pool and the step context


def build_store(w, device, seed=0):
    """An HBM store holding the workload's sequences (blocks from the pool's
    own allocator), random cache contents, and the step's new K/V rows."""
    import torch

    mm = pkg("memory.manager")
    rq = pkg("engine.request")
    store = mm.PagedKVCacheManager(total_blocks=w.total_blocks, block_size=w.block_size, num_heads=w.num_kv_heads,
                                   head_dim=w.head_dim, dtype=w.dtype, num_layers=1, device=device)
    store.num_query_heads = w.num_query_heads
    seqs = []
    for i, ctx in enumerate(w.context_lens):
        seq = rq.Request(i + 1, [0] * ctx)
        store.allocate_prefix_blocks(seq)
        seqs.append(seq)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for cache in (store.key_cache, store.value_cache):
        cache.copy_(torch.randn(cache.shape, generator=gen, device=device).to(w.dtype))
    return store, seqs


def host_step_us(store, seqs, w, reps=200):
    """Median host time of building the step context (no device sync inside)."""
    import torch

    pa = pkg("model.paged_attention")
    starts, counts = list(w.start_positions), list(w.new_token_counts)
    for _ in range(5):
        pa.PagedStepContext(store, seqs, starts, counts)
    torch.cuda.synchronize()
    times = []
    for i in range(reps):
        t0 = time.perf_counter()
        pa.PagedStepContext(store, seqs, starts, counts)
        times.append(time.perf_counter() - t0)
        if i % 50 == 49:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return round(median(times) * 1e6, 1)


# ---------------------------------------------------------------------------
# workloads


def decode_main(args, w, t, device):
    """The headline decode line (Llama-3-8B GQA decode by default; another decode
    workload with --workload)."""
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    pa = pkg("model.paged_attention")
    table = torch.from_numpy(w.block_table_array()).to(device)
    tile = ops.prefill_tile_for(w.num_query_heads, w.num_kv_heads)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, prefill_tile=tile,
                         num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads, head_dim=w.head_dim,
                         dtype=w.dtype)
    out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
    stream = torch.cuda.current_stream(device)

    def decode_step():
        ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out)

    # The per-launch kernel timing runs first, after 500 untimed launches
    # (about 0.15 s): they bring the GPU from idle to its steady clock, which
    # a few warm-up steps alone do not.  The step is then timed after its W
    # warm-ups.
    kernel_ms = events_ms(
        lambda: None,
        lambda: ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out, phases=1),
        args.steps, max(args.warmup, 500), stream)
    ms = timed_ms(decode_step, args.steps, args.warmup, stream)
    eager_alt, graph_step = graph_vs_eager_ms(lambda i: decode_step(), args.steps, stream)

    # The whole step through the product path on an HBM store.
    store, seqs = build_store(w, device)
    new_k = t.new_keys
    new_v = t.new_values
    sout = torch.empty_like(out)

    def full_step():
        # as the layer hook runs it: the step context, then the attention
        # given the layer's new rows (written inside the decode launches)
        ctx = pa.PagedStepContext(store, seqs, w.start_positions, w.new_token_counts)
        ops.attention(t.query, store.key_cache, store.value_cache, 0, ctx.packed, w.scaling, out=sout,
                      new_key=new_k, new_value=new_v)

    # The decode step alone on the store's own pool and tables (packed once):
    # what the full step adds to it is the step's plumbing only.  (The
    # store's pool is a second allocation, and its tables come from the
    # allocator rather than the workload's random permutation; both move
    # the decode kernel's time.)
    ctx0 = pa.PagedStepContext(store, seqs, w.start_positions, w.new_token_counts)

    def store_decode_step():
        ops.attention(t.query, store.key_cache, store.value_cache, 0, ctx0.packed, w.scaling, out=sout)

    # The store was just built on the host with the GPU idle: like the kernel
    # timing above, the loop is timed after enough untimed steps (about
    # 0.1 s of GPU time) to bring the GPU back to its steady clock.
    full_ms = timed_ms(full_step, args.steps, max(args.warmup, 300), stream)
    dec_alt, full_alt = paired_ms(store_decode_step, full_step, args.steps, stream)
    host_us = host_step_us(store, seqs, w)
    del store, seqs

    kv_bytes = wl.decode_bytes(w)
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    kernel_gbs = kv_bytes / (kernel_ms * 1e-3) / 1e9
    read_gbs = sustained_read_gbs(device, kv_bytes)
    return {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == torch.bfloat16 else ("fp16" if w.dtype == torch.float16 else "fp32"),
        "data": "synthetic (seeded N(0,1) K/V/Q, random non-contiguous block tables)",
        "config": workload_config(w, partition=step.partition_size),
        "tokens_per_s": round(w.num_query_tokens / (ms * 1e-3), 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "full_step_ms": round(full_ms, 5),
        "full_step_gbs": round(kv_bytes / (full_ms * 1e-3) / 1e9, 2),
        "full_vs_decode_step": {"full_step_ms": round(full_alt, 5), "decode_step_ms": round(dec_alt, 5),
                                "gap_us": round((full_alt - dec_alt) * 1e3, 2),
                                "timing": "5 alternating rounds of the full-step loop and the decode-step loop "
                                          "(the latter on the store's pool and tables), medians"},
        "host_step_us": {w.name: host_us},
        "graph_step_ms": round(graph_step, 5),
        "graph_vs_eager": {"graph_ms": round(graph_step, 5), "eager_ms": round(eager_alt, 5),
                           "timing": "3 alternating rounds of the eager loop and a replay of it captured in a "
                                     "HIP graph, medians"},
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_partition_kernel",
            "achieved": round(kernel_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(w.name),
            "kernel_ms": round(kernel_ms, 5),
            "algorithmic_bytes": kv_bytes,
            "sustained_read_gbs": round(read_gbs, 1),
            "frac_of_sustained": round(kernel_gbs / read_gbs, 4),
        },
    }


def rotated_copies(nbytes_per_copy: int) -> int:
    """Copies of a working set that together exceed the MALL twice over."""
    return max(4, -(-2 * MALL_BYTES // max(nbytes_per_copy, 1)))


def decode_rotated(args, w, device):
    """A launch-bound decode (fp32 MHA, 8 sequences) timed from a HIP graph over R copies of
    the pool, one per launch, so no launch finds its K/V in the MALL."""
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    kv_bytes = wl.decode_bytes(w)
    copies = rotated_copies(kv_bytes)
    tensors = [wl.make_tensors(w, device, seed=s) for s in range(copies)]
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, num_kv_heads=w.num_kv_heads,
                         num_query_heads=w.num_query_heads, head_dim=w.head_dim, dtype=w.dtype)
    out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
    stream = torch.cuda.current_stream(device)

    def call(i):
        t = tensors[i % copies]
        ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out)

    reps = copies * max(1, args.steps // copies + 1)
    ms = graph_ms(call, reps, 3, stream)
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    line = {
        "value": round(gbs, 2), "unit": "GB/s", "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "ms_per_step": round(ms, 5), "tokens_per_s": round(w.num_query_tokens / (ms * 1e-3), 1),
        "dtype": "fp32", "partition": step.partition_size,
        "timing": f"HIP graph of {reps} decode steps over {copies} rotated pool copies (MALL 256 MB)",
        "config": workload_config(w),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_flat(w, tensors[0])
    return line


def kv_write_pack_line(args, w, device):
    """The K/V write + packing step: the packing kernels over the step's block tables plus the K/V
    write of its new tokens, timed from a HIP graph over R rotated copies of
    the new rows and the cache."""
    import numpy as np
    import torch

    from oracle import packing as op

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                         num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads)
    e = 2
    T, B = w.num_query_tokens, w.num_seqs
    write_bytes = 4 * T * w.num_kv_heads * w.head_dim * e + 8 * T
    pack_bytes = (8 * 2 + 8 * 2) * B + 16 * T + 4 * B + 4 * table.numel()
    total = write_bytes + pack_bytes
    copies = rotated_copies(write_bytes)
    tensors = [wl.make_tensors(w, device, seed=s) for s in range(copies)]
    stream = torch.cuda.current_stream(device)

    def write(i):
        t = tensors[i % copies]
        ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)

    def step_fn(i):
        ops._run_pack(step)
        write(i)

    reps = copies * max(1, args.steps // copies + 1)
    ms = graph_ms(step_fn, reps, 3, stream)
    kms = graph_ms(write, reps, 3, stream)
    line = {
        "metric": "paged KV write + ragged packing GB/s (% HBM peak), 1 GPU",
        "value": round(total / (ms * 1e-3) / 1e9, 2), "unit": "GB/s",
        "hbm_frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "ms_per_step": round(ms, 5), "tokens_per_s": round(T / (ms * 1e-3), 1), "dtype": "bf16",
        "timing": f"HIP graph of {reps} steps over {copies} rotated copies of the new K/V rows and the cache "
                  f"(MALL 256 MB)",
        "config": workload_config(w),
        "roofline": {
            "bound": "hbm", "kernel": "cache_write_vec_kernel",
            "achieved": round(write_bytes / (kms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(write_bytes / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "kernel_ms": round(kms, 5),
            "algorithmic_bytes": write_bytes,
        },
    }
    if not args.no_cpu_baseline:
        t = tensors[0]
        ctx = w.context_lens
        shape = (1, w.total_blocks, w.block_size, w.num_kv_heads, w.head_dim)
        kcache, vcache = np.zeros(shape, dtype=np.uint16), np.zeros(shape, dtype=np.uint16)
        krows = t.new_keys.view(torch.int16).cpu().numpy().view(np.uint16)
        vrows = t.new_values.view(torch.int16).cpu().numpy().view(np.uint16)
        passes = []
        for _ in range(6):
            t0 = time.perf_counter()
            slots = op.build_slot_mapping(w.block_lists, ctx, w.block_size, w.start_positions, w.new_token_counts)
            op.cumulative_offsets(w.new_token_counts)
            op.scatter_layer_kv(kcache, 0, krows, slots)
            op.scatter_layer_kv(vcache, 0, vrows, slots)
            passes.append(time.perf_counter() - t0)
        med = median(passes[1:])
        line["cpu_baseline"] = {
            "value": round(total / med / 1e9, 4), "unit": "GB/s", "tokens_per_s": round(T / med, 1),
            "cores": 1, "kind": "port",
            "sample": (f"the whole step ({T} new tokens of {B} sequences): NumPy slot mapping + cu_seqlens + K and V "
                       f"scatter into a host cache, median of 5 passes after a warm-up ({med * 1e3:.2f} ms/pass); "
                       f"{host_desc()}"),
        }
    return line


def decode_config_line(args, w, t, device):
    """Llama-7B MHA decode inside `configs`: the decode step, its partition kernel and the
    CPU baseline (the pool, 2.2 GB, is far larger than the MALL)."""
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, num_kv_heads=w.num_kv_heads,
                         num_query_heads=w.num_query_heads, head_dim=w.head_dim, dtype=w.dtype)
    out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
    stream = torch.cuda.current_stream(device)
    kernel_ms = events_ms(
        lambda: None,
        lambda: ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out, phases=1),
        args.steps, 100, stream)
    ms = timed_ms(lambda: ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out),
                  args.steps, args.warmup, stream)
    kv_bytes = wl.decode_bytes(w)
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    kernel_gbs = kv_bytes / (kernel_ms * 1e-3) / 1e9
    read_gbs = sustained_read_gbs(device, kv_bytes)
    line = {
        "value": round(gbs, 2), "unit": "GB/s", "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "ms_per_step": round(ms, 5), "tokens_per_s": round(w.num_query_tokens / (ms * 1e-3), 1), "dtype": "bf16",
        "partition": step.partition_size, "config": workload_config(w),
        "roofline": {"bound": "hbm", "kernel": "decode_partition_kernel",
                     "achieved": round(kernel_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(w.name),
                     "kernel_ms": round(kernel_ms, 5), "algorithmic_bytes": kv_bytes,
                     "sustained_read_gbs": round(read_gbs, 1), "frac_of_sustained": round(kernel_gbs / read_gbs, 4)},
    }
    if not args.no_cpu_baseline:
        defer_cpu(lambda: cpu_baseline_per_sequence(w, t, args.cpu_budget / 2), line, "cpu_baseline")
    return line


def mixed_line(args, w, t, device):
    """The mixed step: four 512-token prefill chunks + 128 long-context decodes in one
    flattened step: the attention step (prefill + split-K decode), the same
    step writing its new K/V rows (the product's default: the cache-write
    kernel ahead of the plain launches; and, paired, inside its launches),
    the whole step with packing, the decode kernel's GB/s, and the prefill
    kernel's TFLOP/s against the bf16 MFMA peak."""
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    table = torch.from_numpy(w.block_table_array()).to(device)
    tile = ops.prefill_tile_for(w.num_query_heads, w.num_kv_heads)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, prefill_tile=tile,
                         num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads, head_dim=w.head_dim,
                         dtype=w.dtype)
    out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
    stream = torch.cuda.current_stream(device)
    ms = timed_ms(lambda: ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out),
                  args.steps, args.warmup, stream)
    # 120 untimed launches (about 0.16 s) first: on a GPU that was idle the
    # first 20 launches averaged 4 % slower than the rest.
    decode_kernel_ms = events_ms(
        lambda: None,
        lambda: ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out, phases=1),
        args.steps, 120, stream)
    prefill_ms = events_ms(gpu_spacer,
                           lambda: ops.prefill(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out),
                           args.steps, 20, stream)

    def whole():
        s = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, prefill_tile=tile,
                          num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads, head_dim=w.head_dim,
                          dtype=w.dtype)
        ops.attention(t.query, t.key_cache, t.value_cache, 0, s, w.scaling, out=out, new_key=t.new_keys,
                      new_value=t.new_values)

    full_ms = timed_ms(whole, max(5, args.steps // 2), 2, stream)
    # The attention step writing the new K/V rows, on the packed step: as the
    # product does by default for a step with decodes (the cache-write
    # kernel, then the plain launches).
    write_ms = timed_ms(lambda: ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out,
                                              new_key=t.new_keys, new_value=t.new_values),
                        args.steps, args.warmup, stream)
    # What the K/V write and the packing add to the attention step, each
    # timed in alternation with it (the decode kernel's time drifts by about
    # 1 % between loops run seconds apart, more than the differences).
    def attention_only():
        ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out)

    def with_write():
        ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out, new_key=t.new_keys,
                      new_value=t.new_values)

    # The rows written inside the launches instead (pa_prefill_append +
    # pa_decode_append).
    def with_fused_write():
        ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out, new_key=t.new_keys,
                      new_value=t.new_values, fused_prefill_write=True)

    pair_steps = max(5, args.steps // 2)
    att1, wr1 = paired_ms(attention_only, with_write, pair_steps, stream)
    att3, fw3 = paired_ms(attention_only, with_fused_write, pair_steps, stream)
    if step.__dict__.get("_no_append"):
        raise RuntimeError("the mixed step did not take the fused K/V writes")
    att2, full2 = paired_ms(attention_only, whole, pair_steps, stream)
    sustained = sustained_mfma_tflops(device)
    kv_bytes = wl.decode_bytes(w)
    read_gbs = sustained_read_gbs(device, kv_bytes)
    pf = wl.prefill_flops(w)
    line = {
        "value": round(w.num_query_tokens / (ms * 1e-3), 1), "unit": "tokens/s",
        "ms_per_step": round(ms, 5), "with_kv_write_ms": round(write_ms, 5), "full_step_ms": round(full_ms, 5),
        "paired": {"kv_write_us": round((wr1 - att1) * 1e3, 2),
                   "fused_kv_write_us": round((fw3 - att3) * 1e3, 2),
                   "pack_and_kv_write_us": round((full2 - att2) * 1e3, 2),
                   "attention_ms": round(att1, 5), "with_kv_write_ms": round(wr1, 5), "full_step_ms": round(full2, 5)},
        "full_step_tokens_per_s": round(w.num_query_tokens / (full_ms * 1e-3), 1), "dtype": "bf16",
        "partition": step.partition_size, "config": workload_config(w),
        "decode": {"kernel": "decode_partition_kernel", "kernel_ms": round(decode_kernel_ms, 5),
                   "gbs": round(kv_bytes / (decode_kernel_ms * 1e-3) / 1e9, 2),
                   "hbm_frac": round(kv_bytes / (decode_kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "traffic": measured_traffic(w.name), "algorithmic_bytes": kv_bytes,
                   "sustained_read_gbs": round(read_gbs, 1),
                   "frac_of_sustained": round(kv_bytes / (decode_kernel_ms * 1e-3) / 1e9 / read_gbs, 4)},
        "prefill": {"kernel": "prefill_kernel", "gflop": round(pf / 1e9, 2), "kernel_ms": round(prefill_ms, 5),
                    "tflops": round(pf / (prefill_ms * 1e-3) / 1e12, 1),
                    "mfma_frac": round(pf / (prefill_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                    "traffic": measured_traffic("mixed_step_prefill"),
                    "mfma_sustained_tflops": round(sustained, 1),
                    "frac_of_sustained": round(pf / (prefill_ms * 1e-3) / 1e12 / sustained, 4)},
    }
    if not args.no_cpu_baseline:
        def both():
            dec = cpu_baseline_per_sequence(w, t, args.cpu_budget / 2, "decode")
            pre = cpu_baseline_per_sequence(w, t, args.cpu_budget / 2, "prefill")
            return {"decode": dec, "prefill": pre, "value": dec["value"], "unit": "GB/s", "cores": dec["cores"],
                    "kind": dec["kind"], "sample": "decode: " + dec["sample"] + " | prefill: " + pre["sample"]}

        defer_cpu(both, line, "cpu_baseline")
    return line


def prefill_shapes_line(args, device):
    """The prefill kernel alone on each prefill-only step of PREFILL_SHAPES:
    HIP-event time per launch, TFLOP/s (4 H_q D (n s + n(n+1)/2) per chunk)
    and the fraction of the dtype's dense MFMA peak."""
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    stream = torch.cuda.current_stream(device)
    shapes = {}
    for name, (starts, counts, dtype) in wl.PREFILL_SHAPES.items():
        if args.shape is not None and name != args.shape:
            continue
        w = wl.prefill_chunks(name, starts, counts, dtype, seed=args.seed)
        t = wl.make_tensors(w, device, seed=args.seed)
        table = torch.from_numpy(w.block_table_array()).to(device)
        step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                             prefill_tile=ops.prefill_tile_for(w.num_query_heads, w.num_kv_heads),
                             num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads,
                             head_dim=w.head_dim, dtype=w.dtype)
        out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
        ms = events_ms(gpu_spacer,
                       lambda: ops.prefill(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out),
                       args.steps, 20, stream)
        # The same launch writing the chunks' new K/V rows (pa_prefill_append).
        app_ms = events_ms(gpu_spacer,
                           lambda: ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out,
                                                 new_key=t.new_keys, new_value=t.new_values,
                                                 fused_prefill_write=True),
                           args.steps, 20, stream)
        if step.__dict__.get("_no_append"):
            raise RuntimeError(f"{name}: the prefill did not take the fused write")

        # The whole step with its K/V write from HIP graphs (no launch
        # gaps): the cache-write kernel then the prefill, against the fused
        # launch, alternated three times each.
        def separate(i=0):
            ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)
            ops.prefill(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out)

        def fused(i=0):
            ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out,
                          new_key=t.new_keys, new_value=t.new_values, fused_prefill_write=True)

        sep_g, fus_g = [], []
        for _ in range(3):
            sep_g.append(graph_ms(separate, 40, 3, stream))
            fus_g.append(graph_ms(fused, 40, 3, stream))
        pf = wl.prefill_flops(w)
        peak = MFMA_F32_PEAK_TFLOPS if dtype == torch.float32 else MFMA_BF16_PEAK_TFLOPS
        tf = pf / (ms * 1e-3) / 1e12
        shapes[name] = {"starts": list(starts), "counts": list(counts), "dtype": str(dtype).replace("torch.", ""),
                        "gflop": round(pf / 1e9, 2), "kernel_ms": round(ms, 5), "tflops": round(tf, 1),
                        "peak_tflops": peak, "mfma_frac": round(tf / peak, 4),
                        "append_kernel_ms": round(app_ms, 5),
                        "graph_step_us": {"write_then_prefill": round(median(sep_g) * 1e3, 2),
                                          "fused_write": round(median(fus_g) * 1e3, 2)}}
        del t, out, step, table
        torch.cuda.empty_cache()
    return {"workload": "prefill_shapes", "heads": [32, 8], "head_dim": 128, "block_size": wl.BLOCK_SIZE,
            "steps": args.steps, "shapes": shapes}


def decode_layers_line(args, device):
    """A model's layer loop over one decode step: 32 layers, each writing its
    new K/V rows inside the decode launch (pa_decode_append) and attending,
    from eager launches and from one HIP graph of the 32 layers replayed, in
    alternation (bf16 32/8 heads of 128, contexts of 256-1024 tokens, 16, 64
    and 256 sequences).  Per-layer microseconds."""
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    stream = torch.cuda.current_stream(device)
    lines = {}
    for n in (16, 64, 256):
        w = wl.decode_layers(n, seed=args.seed)
        t = wl.make_tensors(w, device, seed=args.seed)
        table = torch.from_numpy(w.block_table_array()).to(device)
        step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                             num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads, head_dim=w.head_dim,
                             dtype=w.dtype)
        out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)

        def layers(_i, t=t, step=step, out=out, w=w):
            for layer in range(w.num_layers):
                ops.attention(t.query, t.key_cache, t.value_cache, layer, step, w.scaling, out=out,
                              new_key=t.new_keys, new_value=t.new_values)

        eager, graph = graph_vs_eager_ms(layers, 20, stream, rounds=5)
        lines[str(n)] = {"eager_us_per_layer": round(eager * 1e3 / w.num_layers, 2),
                         "graph_us_per_layer": round(graph * 1e3 / w.num_layers, 2),
                         "partition": step.partition_size, "context_tokens": w.num_context_tokens}
        del t, step, out, table
        torch.cuda.empty_cache()
    return {"decode_layers": lines, "layers": 32, "unit": "us per layer", "data": "synthetic"}


def decode_partition_shapes(seed: int = 0):
    """Latency-bound decode steps (too small to fill the chip): (name, contexts,
    H_q, H_kv, D, dtype).  bf16 32/8 heads of 128 unless named otherwise."""
    import numpy as np
    import torch

    rng = np.random.Generator(np.random.PCG64(3 + seed))

    def draw(lo, hi, n):
        return [int(c) for c in rng.integers(lo, hi, size=n, endpoint=True)]

    bf = (32, 8, 128, torch.bfloat16)
    return [
        ("1x1024", [1024], *bf), ("4x1024", [1024] * 4, *bf), ("16x1024", [1024] * 16, *bf),
        ("24x1024", [1024] * 24, *bf), ("8x512", [512] * 8, *bf), ("2x2048", [2048] * 2, *bf),
        ("8x2048", [2048] * 8, *bf), ("64x2048", [2048] * 64, *bf), ("1x4096", [4096], *bf),
        ("4x4096", [4096] * 4, *bf), ("16x4096", [4096] * 16, *bf), ("2x8192", [8192] * 2, *bf),
        ("1x16384", [16384], *bf), ("4x16384", [16384] * 4, *bf),
        ("16x256-1024", draw(256, 1024, 16), *bf), ("64x256-1024", draw(256, 1024, 64), *bf),
        ("32x300-700", draw(300, 700, 32), *bf), ("32x512-4096", draw(512, 4096, 32), *bf),
        ("8x1000-8000", draw(1000, 8000, 8), *bf),
        ("8x16-512 fp32 8/8/64", draw(16, 512, 8), 8, 8, 64, torch.float32),
        ("4x2048 fp32 32/8/128", [2048] * 4, 32, 8, 128, torch.float32),
        ("8x1024 bf16 64/8/128", [1024] * 8, 64, 8, 128, torch.bfloat16),
    ]


def decode_partitions_line(args, device):
    """Latency-bound decode steps in a model's 32-layer loop (every layer's
    cache read cold, each layer writing its new rows inside the decode
    launch): per-layer time of each split-K partition from 64 to 4096 from
    one HIP graph of 10 passes, 7 alternated rounds, medians; beside it the
    partition pa_plan_step picks and how far it is from the fastest."""
    import numpy as np
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    stream = torch.cuda.current_stream(device)
    lines = {}
    for name, ctx, hq, hkv, d, dtype in decode_partition_shapes(args.seed):
        rng = np.random.Generator(np.random.PCG64(7))
        lists, total = wl._block_tables(rng, ctx, wl.BLOCK_SIZE)
        w = wl.StepWorkload(name, hq, hkv, d, wl.BLOCK_SIZE, dtype, 1.0, [c - 1 for c in ctx], [1] * len(ctx),
                            lists, total, 32)
        t = wl.make_tensors(w, device, seed=args.seed)
        table = torch.from_numpy(w.block_table_array()).to(device)
        out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
        graphs = {}  # partition -> (graph, step): the graph reads the step's buffers, so the step lives as long
        picked = None
        for part in [None, 64, 128, 256, 512, 1024, 2048, 4096]:
            if part is not None and (part > 2 * max(ctx) or part in graphs):
                continue
            step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, partition_size=part,
                                 num_kv_heads=hkv, num_query_heads=hq, head_dim=d, dtype=dtype)
            if part is None:
                picked = step.partition_size

            def layers(step=step):
                for layer in range(w.num_layers):
                    ops.attention(t.query, t.key_cache, t.value_cache, layer, step, w.scaling, out=out,
                                  new_key=t.new_keys, new_value=t.new_values)

            layers()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(10):
                    layers()
            g.replay()
            torch.cuda.synchronize()
            graphs[step.partition_size] = (g, step)
        times = {p: [] for p in graphs}
        for _ in range(7):
            for p, (g, _step) in graphs.items():
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                g.replay()
                b.record(stream)
                torch.cuda.synchronize()
                times[p].append(a.elapsed_time(b) * 1e3 / (10 * w.num_layers))
        us = {p: round(median(v), 2) for p, v in sorted(times.items())}
        fastest = min(us, key=us.get)
        lines[name] = {"us_per_layer": {str(p): v for p, v in us.items()}, "picked": picked, "fastest": fastest,
                       "picked_over_fastest": round(us[picked] / us[fastest], 4)}
        print(f"{name}: picked {picked} ({us[picked]} us), fastest {fastest} ({us[fastest]} us)", flush=True)
        del graphs, t, out, table
        torch.cuda.empty_cache()
    return {"decode_partitions": lines, "layers": 32, "unit": "us per layer", "data": "synthetic"}


def config_in_child(args, workload: str) -> dict:
    """One `configs` line, measured by this script in a process of its own.

    Each workload's pool is then the first large allocation of its process,
    as a server allocates its KV pool at start-up.  Measured on one box: the
    mixed step's 8.9 GB pool allocated a second time in one process (freed
    and allocated again, or after other workloads' tensors) made its decode
    kernel 1.376-1.379 ms against 1.322 ms for the first allocation; the
    random 32 KB block reads over the whole pool depend on how it is mapped."""
    cmd = [sys.executable, str(Path(__file__).resolve()), "--workload", workload, "--steps", str(args.steps),
           "--warmup", str(args.warmup), "--seed", str(args.seed), "--cpu-budget", str(args.cpu_budget),
           "--no-configs", "--config-line"]
    if args.no_cpu_baseline:
        cmd.append("--no-cpu-baseline")
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=900)
    if proc.returncode != 0:
        raise RuntimeError(f"bench.py --workload {workload} exited with {proc.returncode}")
    return json.loads([ln for ln in proc.stdout.splitlines() if ln.startswith("{")][-1])


def ab_line(args, device):
    """The workload's kernel and step times under the in-tree library ("a") and
    under another build of it ("b", --ab-library), in args.ab_rounds
    alternating rounds on the same tensors and packed step (each round:
    every measure under a, then under b).  Decode workloads: the partition
    kernel (HIP events), the decode step, and the step writing its new K/V
    rows; fp32_mha_decode: the step from
    a HIP graph over rotated pool copies; mixed_step: the attention step and
    its decode and prefill kernels; prefill_shapes (--shape, or all): the
    prefill kernel of each shape; decode_partitions (--shape, or all): a
    32-layer loop over each latency-bound decode step, per layer, from a
    HIP graph packed and captured under each library."""
    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    native = pkg("_native")
    stream = torch.cuda.current_stream(device)
    measures = {}  # name -> () -> ms

    def packed(w, **kw):
        table = torch.from_numpy(w.block_table_array()).to(device)
        return ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                             prefill_tile=ops.prefill_tile_for(w.num_query_heads, w.num_kv_heads),
                             num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads, head_dim=w.head_dim,
                             dtype=w.dtype, **kw)

    keep = []
    if args.workload == "prefill_shapes":
        for name, (starts, counts, dtype) in wl.PREFILL_SHAPES.items():
            if args.shape is not None and name != args.shape:
                continue
            w = wl.prefill_chunks(name, starts, counts, dtype, seed=args.seed)
            t = wl.make_tensors(w, device, seed=args.seed)
            step = packed(w)
            out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
            keep.append((t, step, out))
            measures[f"{name}.prefill_kernel_ms"] = (
                lambda t=t, step=step, out=out, w=w: events_ms(
                    gpu_spacer, lambda: ops.prefill(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out),
                    args.steps, 20, stream))
    elif args.workload == "fp32_mha_decode":
        w = wl.WORKLOADS[args.workload](seed=args.seed)
        args.no_cpu_baseline = True
        measures["step_ms"] = lambda: decode_rotated(args, w, device)["ms_per_step"]
    elif args.workload in ("llama3_8b_gqa_decode", "llama7b_mha_decode", "mixed_step"):
        w = wl.WORKLOADS[args.workload](seed=args.seed)
        t = wl.make_tensors(w, device, seed=args.seed)
        step = packed(w)
        out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
        keep.append((t, step, out))
        measures["decode_kernel_ms"] = lambda: events_ms(
            lambda: None, lambda: ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out,
                                             phases=1), args.steps, 100, stream)
        measures["step_ms"] = lambda: timed_ms(
            lambda: ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out),
            args.steps, args.warmup, stream)
        # The same step writing its new K/V rows (the product's default way).
        measures["step_with_kv_write_ms"] = lambda: timed_ms(
            lambda: ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out,
                                  new_key=t.new_keys, new_value=t.new_values),
            args.steps, args.warmup, stream)
        if args.workload == "mixed_step":
            measures["prefill_kernel_ms"] = lambda: events_ms(
                gpu_spacer, lambda: ops.prefill(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out),
                args.steps, 20, stream)
    elif args.workload == "decode_partitions":
        import numpy as np

        def layer_ms(w, t):
            # packed and captured under the library in use, replayed once, then timed
            step = packed(w)
            out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)

            def layers():
                for layer in range(w.num_layers):
                    ops.attention(t.query, t.key_cache, t.value_cache, layer, step, w.scaling, out=out,
                                  new_key=t.new_keys, new_value=t.new_values)

            layers()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(10):
                    layers()
            g.replay()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            g.replay()
            b.record(stream)
            torch.cuda.synchronize()
            ms = a.elapsed_time(b) / (10 * w.num_layers)
            del g  # before the step whose buffers it reads
            return ms

        for name, ctx, hq, hkv, d, dtype in decode_partition_shapes(args.seed):
            if args.shape is not None and name != args.shape:
                continue
            rng = np.random.Generator(np.random.PCG64(7))
            lists, total = wl._block_tables(rng, ctx, wl.BLOCK_SIZE)
            w = wl.StepWorkload(name, hq, hkv, d, wl.BLOCK_SIZE, dtype, 1.0, [c - 1 for c in ctx], [1] * len(ctx),
                                lists, total, 32)
            t = wl.make_tensors(w, device, seed=args.seed)
            keep.append(t)
            measures[f"{name}.layer_ms"] = lambda w=w, t=t: layer_ms(w, t)
    else:
        raise SystemExit(f"--ab-library does not cover {args.workload}")

    other = str(Path(args.ab_library).resolve())
    got = {name: {"a": [], "b": []} for name in measures}
    for _ in range(args.ab_rounds):
        for side in ("a", "b"):
            ctx = native.use_library(other) if side == "b" else contextlib.nullcontext()
            with ctx:
                for name, fn in measures.items():
                    got[name][side].append(round(fn(), 5))
    summary = {name: {"a_median": median(v["a"]), "b_median": median(v["b"]), "a": v["a"], "b": v["b"]}
               for name, v in got.items()}
    return {"ab": {"workload": args.workload, "a": str(native.LIBRARY_PATH), "b": other, "rounds": args.ab_rounds,
                   "steps": args.steps, "metrics": summary}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="llama3_8b_gqa_decode",
                    choices=["llama3_8b_gqa_decode", "llama7b_mha_decode", "mixed_step", "fp32_mha_decode",
                             "kv_write_pack", "prefill_shapes", "decode_layers", "decode_partitions"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--shape", default=None, help="prefill_shapes: measure only this shape")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="only the headline line, without `configs`")
    ap.add_argument("--config-line", action="store_true",
                    help="print the workload's `configs` line (how the headline run measures each config)")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device copy (reference for the PMC byte counters)")
    ap.add_argument("--calibrate-mfma", action="store_true",
                    help="only measure the sustained bf16 MFMA rate (pa_calibrate_mfma)")
    ap.add_argument("--calibrate-read", action="store_true",
                    help="only measure the sustained read rate for 1-8 GiB (pa_calibrate_read)")
    ap.add_argument("--ab-library", default=None,
                    help="time the workload's kernels in alternation with this other build of the library "
                         "(csrc/build.py --rev REV --out PATH) and print one comparison line")
    ap.add_argument("--ab-rounds", type=int, default=3)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path has no multi-GPU sharding "
              "(run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    wl = pkg("workloads")
    pkg("_native").load_library()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.calibrate_copy:
        calibrate_copy(device)
        return 0
    if args.calibrate_read:
        rates = {f"{gib}GiB": round(sustained_read_gbs(device, gib << 30), 1) for gib in (1, 2, 4, 8)}
        print(json.dumps({"read_gbs_sustained": rates, "nominal_gbs": HBM_PEAK_GBS}), flush=True)
        return 0
    if args.calibrate_mfma:
        tf = sustained_mfma_tflops(device)
        mixed = {str(nv): round(sustained_mfma_tflops(device, valu_per_mfma=nv), 1) for nv in (4, 8, 16)}
        print(json.dumps({"mfma_bf16_sustained_tflops": round(tf, 1), "nominal_tflops": MFMA_BF16_PEAK_TFLOPS,
                          "frac_of_nominal": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                          "mfma_tflops_with_fp32_fmas_per_mfma": mixed}), flush=True)
        return 0

    if args.ab_library is not None:
        print(json.dumps(ab_line(args, device)), flush=True)
        return 0
    if args.workload == "prefill_shapes":
        print(json.dumps(prefill_shapes_line(args, device)), flush=True)
        return 0
    if args.workload == "decode_layers":
        print(json.dumps(decode_layers_line(args, device)), flush=True)
        return 0
    if args.workload == "decode_partitions":
        print(json.dumps(decode_partitions_line(args, device)), flush=True)
        return 0
    w = wl.WORKLOADS[args.workload](seed=args.seed)
    if args.workload == "kv_write_pack":
        print(json.dumps(kv_write_pack_line(args, w, device)), flush=True)
        return 0
    if args.workload == "fp32_mha_decode":
        print(json.dumps(decode_rotated(args, w, device)), flush=True)
        return 0
    t = wl.make_tensors(w, device, seed=args.seed)
    if args.workload == "mixed_step":
        line = mixed_line(args, w, t, device)
        if args.config_line:
            del t
            torch.cuda.empty_cache()
            store, seqs = build_store(w, device)
            line["host_step_us"] = host_step_us(store, seqs, w)
            del store, seqs
        run_deferred()
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "llama7b_mha_decode" and args.config_line:
        line = decode_config_line(args, w, t, device)
        run_deferred()
        print(json.dumps(line), flush=True)
        return 0

    result = decode_main(args, w, t, device)
    if not args.no_cpu_baseline:
        defer_cpu(lambda t=t: cpu_baseline_per_sequence(w, t, args.cpu_budget), result, "cpu_baseline")
    del t
    if not args.no_configs and args.workload == "llama3_8b_gqa_decode":
        # The headline's own CPU baseline first (the children then run with
        # this process idle), then every config in a process of its own.
        run_deferred()
        configs = {name: config_in_child(args, name)
                   for name in ("fp32_mha_decode", "kv_write_pack", "llama7b_mha_decode", "mixed_step")}
        result["host_step_us"]["mixed_step"] = configs["mixed_step"].pop("host_step_us")
        result["configs"] = configs
    run_deferred()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
