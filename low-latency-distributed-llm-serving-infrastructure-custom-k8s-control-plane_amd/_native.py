"""ctypes binding of libpaged_attention_amd.so (the C ABI in
include/paged_attention_amd.h).

The library is built in-tree by ``csrc/build.py`` and loaded from this
package directory only.  There is no fallback: if the library is missing or
does not export the expected symbols, :func:`load_library` raises, and every
GPU operation of the package raises with it.
"""

from __future__ import annotations

import contextlib
import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libpaged_attention_amd.so"
ABI_VERSION = 13

PA_OK = 0
PA_ERR_INVALID_ARGUMENT = 1
PA_ERR_UNSUPPORTED = 2
PA_ERR_WORKSPACE = 3
PA_ERR_LAUNCH = 4

PA_DTYPE_F32 = 0
PA_DTYPE_BF16 = 1
PA_DTYPE_F16 = 2

PA_DECODE_PARTITION = 2048
PA_DECODE_MAX_PARTITION = 4096
PA_DECODE_PHASE_PARTITIONS = 1
PA_DECODE_PHASE_MERGE = 2
PA_DECODE_SCRATCH_BYTES = 64 << 20
PA_DECODE_SCRATCH_STATE_BYTES = 1 << 20
PA_SWAP_OUT = 0
PA_SWAP_IN = 1

#: Every symbol the header declares; tests check the library exports them all.
EXPORTED_SYMBOLS = (
    "paged_attention",
    "pa_last_error",
    "pa_pack_workspace_size",
    "pa_pack",
    "pa_plan_step",
    "pa_reshape_and_cache",
    "pa_copy_blocks",
    "pa_swap_blocks",
    "pa_decode_workspace_size",
    "pa_decode_merge_state_size",
    "pa_decode_workgroups_per_item",
    "pa_decode_workgroups_per_cu",
    "pa_prefill_tile",
    "pa_decode",
    "pa_decode_phases",
    "pa_decode_no_alloc",
    "pa_decode_append",
    "pa_prefill",
    "pa_prefill_append",
    "pa_map_host_memory",
    "pa_calibrate_mfma",
    "pa_calibrate_mfma_flops",
    "pa_calibrate_read",
    "pa_error_string",
    "pa_last_error_message",
    "pa_abi_version",
)


class PagedAttentionDims(ctypes.Structure):
    """Mirror of the reference PagedAttentionDims (csrc/include/paged_kernels.h:11-20)."""

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


class PaStepDims(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_query_tokens", ctypes.c_int32),
        ("num_query_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("total_blocks", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("partition_size", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("num_table_rows", ctypes.c_int32),
        ("q_token_stride", ctypes.c_int64),
        ("q_head_stride", ctypes.c_int64),
        ("block_table_rows", ctypes.c_void_p),
    ]


class PaNewRows(ctypes.Structure):
    _fields_ = [
        ("key", ctypes.c_void_p),
        ("value", ctypes.c_void_p),
        ("key_token_stride", ctypes.c_int64),
        ("key_head_stride", ctypes.c_int64),
        ("value_token_stride", ctypes.c_int64),
        ("value_head_stride", ctypes.c_int64),
    ]


class PaPackDims(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("partition_size", ctypes.c_int32),
        ("prefill_tile", ctypes.c_int32),
        ("num_table_rows", ctypes.c_int32),
        ("num_updates", ctypes.c_int32),
        ("step_table_width", ctypes.c_int32),
        ("max_new_tokens", ctypes.c_int32),
        ("max_context", ctypes.c_int32),
        ("max_query_tokens", ctypes.c_int64),
        ("max_context_tokens", ctypes.c_int64),
        ("max_decode_items", ctypes.c_int64),
        ("max_merge_items", ctypes.c_int64),
        ("max_prefill_items", ctypes.c_int64),
    ]


class PaPlanParams(ctypes.Structure):
    _fields_ = [
        ("block_size", ctypes.c_int32),
        ("prefill_tile", ctypes.c_int32),
        ("partition_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("num_query_heads", ctypes.c_int32),
        ("workgroups_per_item", ctypes.c_int32),
        ("workgroups_per_cu", ctypes.c_int32),
        ("compute_units", ctypes.c_int32),
    ]


class PaStepPlan(ctypes.Structure):
    _fields_ = [
        ("num_query_tokens", ctypes.c_int64),
        ("num_context_tokens", ctypes.c_int64),
        ("num_decode_items", ctypes.c_int64),
        ("num_merge_items", ctypes.c_int64),
        ("num_prefill_items", ctypes.c_int64),
        ("max_context", ctypes.c_int64),
        ("num_decode_seqs", ctypes.c_int32),
        ("num_prefill_seqs", ctypes.c_int32),
        ("partition_size", ctypes.c_int32),
        ("max_blocks", ctypes.c_int32),
        ("bad_seq", ctypes.c_int32),
        ("max_new_tokens", ctypes.c_int32),
    ]


_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

_SIGNATURES = {
    "paged_attention": (None, [_vp, _vp, _vp, _i32, PagedAttentionDims, _vp, _vp, _f32, _vp, _vp, _vp]),
    "pa_last_error": (ctypes.c_int, []),
    "pa_pack_workspace_size": (_sz, [_i32]),
    "pa_pack": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _vp, PaPackDims, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
         _vp, _sz, _vp, _sz, _vp],
    ),
    "pa_plan_step": (ctypes.c_int, [_vp, _vp, _vp, _i32, PaPlanParams, ctypes.POINTER(PaStepPlan)]),
    "pa_calibrate_mfma": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp]),
    "pa_calibrate_mfma_flops": (ctypes.c_int64, [_i32, _i32]),
    "pa_calibrate_read": (ctypes.c_int, [_vp, _i64, _vp, _i32, _vp]),
    "pa_reshape_and_cache": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "pa_copy_blocks": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _vp]),
    "pa_swap_blocks": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _i32, _vp]),
    "pa_decode_workspace_size": (_sz, [PaStepDims, _i64]),
    "pa_decode_merge_state_size": (_sz, [PaStepDims, _i64]),
    "pa_decode_workgroups_per_item": (_i32, [_i32, _i32, _i32, _i32]),
    "pa_decode_workgroups_per_cu": (_i32, [_i32, _i32, _i32, _i32]),
    "pa_prefill_tile": (_i32, [_i32, _i32]),
    "pa_decode": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, PaStepDims, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _f32, _vp, _vp, _sz, _vp],
    ),
    "pa_decode_phases": (
        ctypes.c_int,
        [_i32, _vp, _vp, _vp, _i32, PaStepDims, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _f32, _vp, _vp, _sz, _vp],
    ),
    "pa_decode_no_alloc": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, PaStepDims, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _f32, _vp, _vp],
    ),
    "pa_decode_append": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, PaStepDims, PaNewRows, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _f32, _vp, _vp, _sz,
         _vp],
    ),
    "pa_prefill": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, PaStepDims, _vp, _vp, _vp, _vp, _i64, _i32, _f32, _vp, _vp],
    ),
    "pa_prefill_append": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i32, PaStepDims, PaNewRows, _vp, _vp, _vp, _vp, _i64, _i32, _f32, _vp, _vp],
    ),
    "pa_map_host_memory": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_void_p)]),
    "pa_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "pa_last_error_message": (ctypes.c_char_p, []),
    "pa_abi_version": (ctypes.c_int, []),
}

_lock = threading.Lock()
_lib = None
_others: dict = {}  # other builds opened by use_library, by path


def library_built() -> bool:
    return LIBRARY_PATH.exists()


def load_library():
    """Open the in-tree HIP library (once) and type its entry points."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise RuntimeError(
                f"HIP extension {LIBRARY_PATH.name} is not built; run __graft_entry__.build() "
                "(or csrc/build.py) before using the GPU paged-attention path"
            )
        _lib = _open(LIBRARY_PATH)
        return _lib


def _open(path: Path):
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.pa_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    return lib


@contextlib.contextmanager
def use_library(path):
    """A measurement aid: inside the block, :func:`load_library` returns the
    build of the library at ``path`` (same ABI version) instead of the
    in-tree one, so that two builds (``csrc/build.py --rev``) can be timed
    in alternation in one process (``bench.py --ab-library``).  Values the
    package caches from the library (launch-shape queries) stay those of the
    in-tree build, so both builds run the same launch shapes."""
    global _lib
    key = str(Path(path).resolve())
    load_library()
    with _lock:
        other = _others.get(key)
        if other is None:
            other = _others[key] = _open(Path(key))
        saved, _lib = _lib, other
    try:
        yield other
    finally:
        with _lock:
            _lib = saved


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status returned by the library."""
    if status == PA_OK:
        return
    lib = load_library()
    detail = lib.pa_last_error_message().decode(errors="replace")
    kind = lib.pa_error_string(status).decode(errors="replace")
    raise RuntimeError(f"{what} failed ({kind}): {detail}")
