"""Paged-attention decode benchmark on one MI355X.

Workload (default): Llama-3-8B-shaped GQA decode, bf16 -- 256 sequences,
32 query / 8 KV heads, head_dim 128, block size 16, contexts
clip(round(lognormal(ln 1024, 1.0)), 32, 8192), random non-contiguous block
tables, N(0,1) synthetic values.  A "step" is one decode pass of one layer
over the batch (the HIP split-K partition kernel + its merge kernel), with
the batch already packed and resident in HBM.

value   = algorithmic KV-read GB/s = decode bytes / mean step time, where
          decode bytes = sum_i ctx_i * 2 * H_kv * D * 2 (K+V read once per
          KV head) + q and out rows + block-table entries + context lengths;
tokens/s = sequences / mean step time (one token per sequence per layer).
roofline = the dominant kernel (the split-K partition kernel), its
          algorithmic bytes over its own launch time, measured with HIP
          events around each partition launch on its stream; traffic = its
          HBM bytes per launch from the committed rocprofv3 PMC summary.
Also reported: the full step time (GPU packing + K/V write of the step's
tokens + attention), the reference CPU kernel timed on a bounded sample of
the same workload on this host's cores, and for --workload mixed_step (prefill +
decode step) the prefill kernel's TFLOP/s against the bf16 MFMA peak.

python bench.py [--steps K] [--warmup W] [--no-cpu-baseline]
                [--workload llama3_8b_gqa_decode|llama7b_mha_decode|mixed_step]
"""

from __future__ import annotations

import argparse
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


def cpu_baseline(w, t, budget_s: float):
    """Reference kernel (oracle/_ref) per sequence on fp32 up-casts of the
    same values.  Sequences are taken in order until ~budget_s/6 seconds of
    kernel time (a bounded sample), then that sample is timed once more as a
    warm-up plus five times; the median pass is reported."""
    import numpy as np
    import torch

    from oracle import attention as oa

    kind = "reference" if oa.reference_available() else "port"
    q_all = t.query[0].transpose(0, 1)
    e = 2 if w.dtype == torch.bfloat16 else 4
    qbase = np.concatenate([[0], np.cumsum(w.new_token_counts)])  # first query token of each sequence
    sample, spent = [], 0.0
    for i in range(w.num_seqs):
        if w.new_token_counts[i] != 1:
            continue  # decode sequences only (a mixed step's prefill chunks are not decode work)
        blocks = torch.tensor(w.block_lists[i], dtype=torch.long, device=t.key_cache.device)
        k = t.key_cache[:, blocks].float().cpu().numpy()
        v = t.value_cache[:, blocks].float().cpu().numpy()
        ctx = w.context_lens[i]
        slots = np.arange(len(w.block_lists[i]) * w.block_size, dtype=np.int64)[:ctx]
        q = q_all[qbase[i] : qbase[i] + 1].float().cpu().numpy().transpose(1, 0, 2)
        _, secs = oa.paged_attention_per_sequence(q, k, v, 0, [w.start_positions[i]], [1], slots, w.scaling,
                                                  kind=kind)
        sample.append((q, k, v, slots, w.start_positions[i], ctx))
        spent += secs
        if spent >= budget_s / 6:
            break
    passes = []
    for _ in range(5):
        total = 0.0
        for q, k, v, slots, start, _ in sample:
            _, secs = oa.paged_attention_per_sequence(q, k, v, 0, [start], [1], slots, w.scaling, kind=kind)
            total += secs
        passes.append(total)
    med = sorted(passes)[len(passes) // 2]
    nbytes = sum(c * 2 * w.num_kv_heads * w.head_dim * e + w.num_query_heads * w.head_dim * 2 * e
                 for *_, c in sample)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": round(nbytes / med / 1e9, 4),
        "unit": "GB/s",
        "tokens_per_s": round(len(sample) / med, 2),
        "cores": threads,
        "kind": kind,
        "sample": (f"first {len(sample)} of {sum(1 for c in w.new_token_counts if c == 1)} decode sequences "
                   f"({sum(c for *_, c in sample)} context tokens), "
                   f"one call per sequence (T=1, all-ones mask; OpenMP parallelism capped at T*H_q="
                   f"{w.num_query_heads} rows), {'fp32 up-casts of the bf16' if e == 2 else 'the fp32'} values, "
                   f"median of 5 passes after a "
                   f"warm-up ({med:.2f} s/pass kernel time, steady_clock around the C call); "
                   f"host {cpu_model()}, nproc {os.cpu_count()}, OMP_NUM_THREADS {threads}"),
    }


def measured_traffic(workload: str):
    """HBM bytes per launch of the dominant kernel on `workload`, from the
    committed rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE, each scaled
    by what the counter reads for a copy of known size); None if absent."""
    path = REPO / "profiles" / "pmc_traffic.json"
    try:
        table = json.loads(path.read_text())
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


def bench_kv_write_pack(args, w, t, device):
    """The integer side of a step: the GPU packing kernel over the step's
    block tables plus the K/V write of its new tokens (32 sequences: 24
    decodes and 8 prompts of 64-256 tokens, 32 KV heads, D 128, bf16).

    value   = algorithmic GB/s of the step: new K and V rows read + cache
              rows written (4 * T * H_kv * D * 2 bytes) + the int64 slots
              read by the write and the packing outputs written;
    roofline = the K/V write kernel alone, timed with HIP events;
    cpu_baseline = the NumPy restatement (slot mapping + scatter) on the same
              step, one host thread."""
    import time

    import numpy as np
    import torch

    from oracle import packing as op

    ops = pkg("paged_ops")
    table = torch.from_numpy(w.block_table_array()).to(device)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size,
                         num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads)
    stream = torch.cuda.current_stream(device)
    e = t.new_keys.element_size()
    T, B = w.num_query_tokens, w.num_seqs
    write_bytes = 4 * T * w.num_kv_heads * w.head_dim * e + 8 * T
    pack_bytes = (8 * 2 + 8 * 2) * B + 16 * T + 4 * B + 4 * table.numel()
    total = write_bytes + pack_bytes

    def write():
        ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, step.scatter_slots, 0)

    def step_fn():
        ops._run_pack(step)
        write()

    ms = graph_ms(step_fn, args.steps, args.warmup, stream)
    kms = graph_ms(write, args.steps, args.warmup, stream)
    result = {
        "metric": "paged KV write + ragged packing GB/s (% HBM peak), 1 GPU",
        "value": round(total / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V, random non-contiguous block tables)",
        "config": workload_config(w),
        "timing": "HIP graph of back-to-back steps replayed between two events",
        "tokens_per_s": round(T / (ms * 1e-3), 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "cache_write_vec_kernel",
            "achieved": round(write_bytes / (kms * 1e-3) / 1e9, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(write_bytes / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel_ms": round(kms, 5),
            "algorithmic_bytes": write_bytes,
        },
    }
    if not args.no_cpu_baseline:
        ctx = [s + c for s, c in zip(w.start_positions, w.new_token_counts)]
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
        med = sorted(passes[1:])[2]
        result["cpu_baseline"] = {
            "value": round(total / med / 1e9, 4),
            "unit": "GB/s",
            "tokens_per_s": round(T / med, 1),
            "cores": 1,
            "kind": "port",
            "sample": (f"the whole step ({T} new tokens of {B} sequences): NumPy slot mapping + cu_seqlens + "
                       f"K and V scatter into a host cache, median of 5 passes after a warm-up "
                       f"({med * 1e3:.2f} ms/pass); host {cpu_model()}"),
        }
    return result


def graph_ms(fn, reps, warmup, stream):
    """Per-call time of `reps` back-to-back calls captured in one HIP graph
    and replayed between two events: microsecond launches are timed without
    host launch gaps."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="llama3_8b_gqa_decode",
                    choices=["llama3_8b_gqa_decode", "llama7b_mha_decode", "mixed_step", "fp32_mha_decode",
                             "kv_write_pack"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device copy (reference for the PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path has no multi-GPU sharding "
              "(run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    ops = pkg("paged_ops")
    wl = pkg("workloads")
    pkg("_native").load_library()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.calibrate_copy:
        calibrate_copy(device)
        return 0

    w = wl.WORKLOADS[args.workload](seed=args.seed)
    mixed = args.workload == "mixed_step"
    t = wl.make_tensors(w, device, seed=args.seed)
    if args.workload == "kv_write_pack":
        result = bench_kv_write_pack(args, w, t, device)
        print(json.dumps(result), flush=True)
        return 0
    table = torch.from_numpy(w.block_table_array()).to(device)
    tile = ops.prefill_tile_for(w.num_query_heads, w.num_kv_heads)
    step = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, prefill_tile=tile,
                         num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads,
                         head_dim=w.head_dim, dtype=w.dtype)
    out = torch.empty((w.num_query_tokens, w.num_query_heads, w.head_dim), dtype=w.dtype, device=device)
    stream = torch.cuda.current_stream(device)

    def decode_step():
        ops.attention(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out)

    def partition_kernel_ms(steps, warmup):
        """Average duration of the dominant kernel (the split-K partition
        kernel): the step is issued as pa_decode's two phases and HIP events
        on the launch stream bracket every partition launch."""
        pairs = []
        for i in range(warmup + steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out, phases=1)
            b.record(stream)
            ops.decode(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out, phases=2)
            if i >= warmup:
                pairs.append((a, b))
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)

    def prefill_kernel_ms(steps, warmup):
        """Average duration of the prefill kernel alone (HIP events on its stream)."""
        pairs = []
        for i in range(warmup + steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            ops.prefill(t.query, t.key_cache, t.value_cache, 0, step, w.scaling, out=out)
            b.record(stream)
            if i >= warmup:
                pairs.append((a, b))
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)

    def full_step():
        s = ops.pack_step(table, w.start_positions, w.new_token_counts, w.block_size, prefill_tile=tile,
                          num_kv_heads=w.num_kv_heads, num_query_heads=w.num_query_heads,
                          head_dim=w.head_dim, dtype=w.dtype)
        ops.reshape_and_cache(t.new_keys, t.new_values, t.key_cache, t.value_cache, s.scatter_slots, 0)
        ops.attention(t.query, t.key_cache, t.value_cache, 0, s, w.scaling, out=out)

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps  # ms

    # The per-launch kernel timing runs first, after 500 untimed launches
    # (about 0.15 s): they bring the GPU from idle to its steady clock, which
    # a few warm-up steps alone do not (the first timed loop after start-up
    # ran about 5 % slow).  The step is then timed after its W warm-ups.
    kernel_ms = partition_kernel_ms(args.steps, max(args.warmup, 500))
    ms = timed(decode_step, args.steps, args.warmup)
    full_ms = timed(full_step, max(5, args.steps // 5), 2)
    # The same step replayed from a HIP graph: for small steps the eager loop
    # above is bound by the host's launch rate, the graph shows the GPU's time.
    graph_step_ms = graph_ms(decode_step, args.steps, 2, stream)

    kv_bytes = wl.decode_bytes(w)
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    kernel_gbs = kv_bytes / (kernel_ms * 1e-3) / 1e9
    traffic = measured_traffic(w.name)
    tokens_per_s = w.num_query_tokens / (ms * 1e-3)
    result = {
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
        "dtype": "bf16" if w.dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded N(0,1) K/V/Q, random non-contiguous block tables)",
        "config": workload_config(w, partition=step.partition_size),
        "tokens_per_s": round(tokens_per_s, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "full_step_ms": round(full_ms, 5),
        "graph_step_ms": round(graph_step_ms, 5),
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_partition_kernel",
            "achieved": round(kernel_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel_ms": round(kernel_ms, 5),
            "algorithmic_bytes": kv_bytes,
        },
    }
    if mixed:
        pf = wl.prefill_flops(w)
        pms = prefill_kernel_ms(args.steps, args.warmup)
        result["prefill"] = {
            "kernel": "prefill_kernel",
            "gflop": round(pf / 1e9, 2),
            "kernel_ms": round(pms, 5),
            "tflops": round(pf / (pms * 1e-3) / 1e12, 1),
            "mfma_frac": round(pf / (pms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        }
        result["mixed_tokens_per_s"] = round(w.num_query_tokens / (ms * 1e-3), 1)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, t, args.cpu_budget)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
