"""ORACLE -- test infrastructure only (tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py; never the product path).

Python access to the CPU attention oracle:
  * ``liboracle_pa.so``: this directory's C restatement of the reference
    kernel (paged_attention_oracle.c, following
    csrc/src/paged_kernels.cpp:7-105);
  * ``_ref/libpaged_kernels_ref.so``: the reference kernel itself, compiled
    from its own source by ``make ref`` (when the reference tree was there);
  * :func:`attention_f64`: closed-form softmax attention in float64, used to
    pin the restatement independently of both.

:func:`paged_attention` mirrors the reference's pybind wrapper
(csrc/src/bindings.cpp:10-76): same validation, same dims derivation, same
output / scratch allocation, one flat call.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle_pa.so"
REF_LIB = HERE / "_ref" / "libpaged_kernels_ref.so"


class Dims(ctypes.Structure):
    _fields_ = [
        ("num_query_heads", ctypes.c_int32),
        ("num_query_tokens", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("total_blocks", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("num_context_tokens", ctypes.c_int32),
    ]


_KERNEL_ARGS = [
    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, Dims,
    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
]

_libs = {}


def build(reference: bool = True) -> None:
    """Compile the oracle (and, if the reference tree exists, the reference)."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    if reference and Path("/root/reference/csrc/src/paged_kernels.cpp").exists():
        subprocess.run(["make", "-s", "-B", "-C", str(HERE), "ref"], check=True)


def _load(kind: str):
    if kind in _libs:
        return _libs[kind]
    path = ORACLE_LIB if kind == "oracle" else REF_LIB
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built (make -C oracle{' ref' if kind == 'reference' else ''})")
    lib = ctypes.CDLL(str(path))
    fn = lib.oracle_paged_attention if kind == "oracle" else lib.paged_attention
    fn.restype = None
    fn.argtypes = _KERNEL_ARGS
    if kind == "oracle":
        drv = lib.oracle_paged_attention_per_sequence
        drv.restype = None
        drv.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, Dims,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_double),
        ]
    _libs[kind] = (lib, fn)
    return _libs[kind]


def reference_available() -> bool:
    return REF_LIB.exists()


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def paged_attention(query, key_cache, value_cache, layer_idx, gather_slots, attention_mask,
                    scaling, kind: str = "oracle") -> np.ndarray:
    """One flat call with the reference's pybind semantics (bindings.cpp:10-76).

    query [1, H_q, T, D], caches (L, N, bs, H_kv, D), gather_slots [C],
    attention_mask [1, 1, T, C] -> output [1, T, H_q, D] (all fp32).
    """
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(key_cache, dtype=np.float32)
    v = np.ascontiguousarray(value_cache, dtype=np.float32)
    s = np.ascontiguousarray(gather_slots, dtype=np.int32)
    m = np.ascontiguousarray(attention_mask, dtype=np.uint8)
    if q.ndim != 4:
        raise RuntimeError("query must be 4-D (1, heads, seq, dim)")
    if k.ndim != 5:
        raise RuntimeError("key_cache must be 5-D (layers, blocks, block_size, heads, dim)")
    if s.ndim != 1:
        raise RuntimeError("gather_slots must be 1-D")
    if m.ndim != 4:
        raise RuntimeError("attention_mask must be 4-D (1, 1, query, context)")
    dims = Dims(q.shape[1], q.shape[2], q.shape[3], k.shape[0], k.shape[1], k.shape[2], k.shape[3], s.shape[0])
    if dims.num_query_heads % dims.num_kv_heads != 0:
        raise RuntimeError("num_query_heads must be a multiple of num_kv_heads for GQA")
    if layer_idx < 0 or layer_idx >= dims.num_layers:
        raise RuntimeError("layer_idx out of range")
    out = np.empty((1, dims.num_query_tokens, dims.num_query_heads, dims.head_dim), dtype=np.float32)
    scratch = np.empty((dims.num_query_tokens, dims.num_query_heads, max(dims.num_context_tokens, 1)), dtype=np.float32)
    _, fn = _load(kind)
    fn(_p(q), _p(k), _p(v), int(layer_idx), dims, _p(s), _p(m), float(scaling), _p(out), _p(scratch), None)
    return out


def paged_attention_per_sequence(query_hm, key_cache, value_cache, layer_idx, starts, counts,
                                 gather_slots, scaling, kind: str = "oracle",
                                 seq_subset: Optional[Sequence[int]] = None):
    """Per-sequence calls (decode: all-ones mask; prefill: causal-offset mask).

    query_hm [H_q, T, D] head-major fp32; gather_slots int64 [C] in sequence
    order (prefix over start+count); returns (output [T, H_q, D] fp32,
    seconds spent inside the kernel calls).  With ``seq_subset`` only those
    sequences are run (their rows are filled, the rest are zero) and T is
    still the full token count.
    """
    lib, fn = _load("oracle")
    kernel = ctypes.cast(fn, ctypes.c_void_p) if kind == "oracle" else ctypes.cast(_load("reference")[1], ctypes.c_void_p)
    q = np.ascontiguousarray(query_hm, dtype=np.float32)
    k = np.ascontiguousarray(key_cache, dtype=np.float32)
    v = np.ascontiguousarray(value_cache, dtype=np.float32)
    starts = np.ascontiguousarray(starts, dtype=np.int64)
    counts = np.ascontiguousarray(counts, dtype=np.int64)
    slots = np.ascontiguousarray(gather_slots, dtype=np.int64)
    ctx = starts + counts
    offsets = np.zeros(len(ctx) + 1, dtype=np.int64)
    np.cumsum(ctx, out=offsets[1:])
    hq, t_total, d = q.shape
    dims = Dims(hq, t_total, d, k.shape[0], k.shape[1], k.shape[2], k.shape[3], 0)
    out = np.zeros((t_total, hq, d), dtype=np.float32)
    if seq_subset is None:
        run_counts = counts
    else:
        run_counts = np.zeros_like(counts)
        run_counts[list(seq_subset)] = counts[list(seq_subset)]
    # The driver walks query rows in sequence order; sequences skipped in
    # run_counts still own their rows, so drive one sequence at a time.
    max_n = int(counts.max()) if len(counts) else 0
    max_c = int(ctx.max()) if len(ctx) else 0
    mask = np.empty(max(max_n * max_c, 1), dtype=np.uint8)
    scratch = np.empty(max(max_n * hq * max_c, 1), dtype=np.float32)
    slot_buf = np.empty(max(max_c, 1), dtype=np.int32)
    q_buf = np.empty(max(max_n * hq * d, 1), dtype=np.float32)
    o_buf = np.empty(max(max_n * hq * d, 1), dtype=np.float32)
    seconds = 0.0
    qbase = np.zeros(len(counts) + 1, dtype=np.int64)
    np.cumsum(counts, out=qbase[1:])
    spent = ctypes.c_double(0.0)
    zero_offset = np.zeros(1, dtype=np.int64)
    for i in range(len(counts)):
        if run_counts[i] == 0:
            continue
        n = int(counts[i])
        sub_q = np.ascontiguousarray(q[:, qbase[i] : qbase[i] + n, :])
        sub_out = np.zeros((n, hq, d), dtype=np.float32)
        sd = Dims(hq, n, d, k.shape[0], k.shape[1], k.shape[2], k.shape[3], 0)
        lib.oracle_paged_attention_per_sequence(
            kernel, _p(sub_q), _p(k), _p(v), int(layer_idx), sd, 1,
            _p(starts[i : i + 1]), _p(counts[i : i + 1]), _p(slots[offsets[i] : offsets[i + 1]]),
            _p(zero_offset), float(scaling), _p(sub_out), _p(mask), _p(scratch),
            _p(slot_buf), _p(q_buf), _p(o_buf), ctypes.byref(spent))
        seconds += spent.value
        out[qbase[i] : qbase[i] + n] = sub_out
    return out, seconds


def attention_f64(query, keys, values, mask, scaling) -> np.ndarray:
    """Closed-form masked softmax attention in float64.

    query [H_q, T, D], keys / values [H_kv, C, D], mask bool [T, C] ->
    [T, H_q, D].  Rows with no attended context give zeros (the reference
    kernel's rule, csrc/src/paged_kernels.cpp:75-91).
    """
    q = np.asarray(query, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    v = np.asarray(values, dtype=np.float64)
    hq, t, d = q.shape
    hkv = k.shape[0]
    group = hq // hkv
    out = np.zeros((t, hq, d), dtype=np.float64)
    for h in range(hq):
        kh, vh = k[h // group], v[h // group]
        s = (q[h] @ kh.T) * scaling  # [T, C]
        s = np.where(mask, s, -np.inf)
        mx = np.max(s, axis=1, keepdims=True) if s.shape[1] else np.zeros((t, 1))
        mx = np.where(np.isfinite(mx), mx, 0.0)
        p = np.where(mask, np.exp(s - mx), 0.0)
        tot = p.sum(axis=1, keepdims=True)
        p = np.divide(p, tot, out=np.zeros_like(p), where=tot > 0)
        out[:, h, :] = p @ vh
    return out
