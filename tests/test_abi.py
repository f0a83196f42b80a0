"""The C-ABI library loads and exports every entry point the header declares.

No kernel is launched here (no GPU needed): only symbol presence, the ABI
version and argument checks that return before any HIP call."""

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from helpers import pkg

HEADER = Path(__file__).resolve().parent.parent / "include" / "paged_attention_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "while", "sizeof")))


def test_header_declarations_match_binding_table():
    native = pkg("_native")
    assert declared_functions() == sorted(native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    native = pkg("_native")
    lib = native.load_library()
    raw = ctypes.CDLL(str(native.LIBRARY_PATH))
    for name in declared_functions():
        assert hasattr(raw, name), name
    assert lib.pa_abi_version() == native.ABI_VERSION


def test_use_library_swaps_and_restores(tmp_path):
    """The A/B measurement aid: inside use_library(path), load_library()
    returns the build at path (here a copy of the in-tree one), typed and
    version-checked; outside, the in-tree library again."""
    native = pkg("_native")
    lib = native.load_library()
    other_path = tmp_path / "libpaged_attention_amd_copy.so"
    shutil.copy2(native.LIBRARY_PATH, other_path)
    with native.use_library(other_path) as other:
        assert native.load_library() is other and other is not lib
        assert other.pa_abi_version() == native.ABI_VERSION
        assert other.pa_decode_workspace_size.argtypes == lib.pa_decode_workspace_size.argtypes
    assert native.load_library() is lib


def test_struct_layouts(tmp_path):
    """The ctypes mirrors match the header's structs field by field: a C
    program built against the header prints every offset and size."""
    native = pkg("_native")
    structs = {name: getattr(native, name) for name in
               ("PagedAttentionDims", "PaStepDims", "PaPackDims", "PaPlanParams", "PaStepPlan", "PaNewRows")}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "paged_attention_amd.h"', "int main(void) {"]
    for name, st in structs.items():
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for field, _ in st._fields_:
            lines.append(f'printf("{name}.{field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    for name, st in structs.items():
        assert int(got[name]) == ctypes.sizeof(st), name
        for field, _ in st._fields_:
            assert int(got[f"{name}.{field}"]) == getattr(st, field).offset, f"{name}.{field}"


def test_error_strings():
    lib = pkg("_native").load_library()
    assert lib.pa_error_string(0) == b"ok"
    assert lib.pa_error_string(3) == b"workspace missing or too small"


def test_invalid_arguments_rejected_before_launch():
    native = pkg("_native")
    lib = native.load_library()
    dims = native.PaStepDims(num_seqs=1, num_query_tokens=1, num_query_heads=6, num_kv_heads=4, head_dim=64,
                             block_size=16, total_blocks=8, num_layers=1, max_blocks_per_seq=1,
                             partition_size=512, dtype=native.PA_DTYPE_BF16, q_token_stride=384, q_head_stride=64)
    rc = lib.pa_decode(None, None, None, 0, dims, None, None, None, None, 1, None, 0, 1.0, None, None, 0, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT
    assert b"multiple of num_kv_heads" in lib.pa_last_error_message()
    dims.num_query_heads = 8
    rc = lib.pa_prefill(None, None, None, 3, dims, None, None, None, None, 1, 32, 1.0, None, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT
    assert b"Layer index 3 out of range" in lib.pa_last_error_message()
    rc = lib.pa_reshape_and_cache(None, None, 0, 0, 0, 0, None, None, None, 4, 2, 8, 4, 4, 1, 0, 7, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT
    for phases in (0, 4, -1):
        rc = lib.pa_decode_phases(phases, None, None, None, 0, dims, None, None, None, None, 1, None, 0, 1.0,
                                  None, None, 0, None)
        assert rc == native.PA_ERR_INVALID_ARGUMENT
        assert b"phases must be" in lib.pa_last_error_message()
    rc = lib.pa_copy_blocks(None, None, None, -1, 1, 1, 1, 16, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT
    rc = lib.pa_copy_blocks(None, None, None, 1, 1, 1, 1, 16, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT and b"missing" in lib.pa_last_error_message()
    assert lib.pa_copy_blocks(None, None, None, 0, 1, 1, 1, 16, None) == native.PA_OK
    pdims = native.PaPackDims(num_seqs=1, block_size=0, max_blocks_per_seq=1, partition_size=512, prefill_tile=32)
    args = [None] * 5 + [pdims] + [None] * 11 + [None, 0] + [None, 0, None]
    assert lib.pa_pack(*args) == native.PA_ERR_INVALID_ARGUMENT
    pdims.block_size = 16
    pdims.step_table_width = 4
    fake = [0x1000 * (i + 1) for i in range(17)]
    for clear, nbytes in ((None, 16), (fake[0] + 8, 16), (fake[0], 24)):  # a clear region of whole aligned words
        args = fake[:5] + [pdims] + fake[5:16] + [clear, nbytes] + [fake[16], 4096, None]
        assert lib.pa_pack(*args) == native.PA_ERR_INVALID_ARGUMENT
        assert b"clear must be" in lib.pa_last_error_message()
    args = fake[:5] + [pdims] + fake[5:16] + [None, 0] + [None, 0, None]
    rc = lib.pa_pack(*args)
    assert rc == native.PA_ERR_WORKSPACE and b"workspace of 544 bytes" in lib.pa_last_error_message()
    assert lib.pa_pack_workspace_size(1) == 544 and lib.pa_pack_workspace_size(0) == 512
    args = fake[:3] + [None, fake[4], pdims] + fake[5:16] + [None, 0] + [fake[16], 4096, None]
    assert lib.pa_pack(*args) == native.PA_ERR_INVALID_ARGUMENT
    assert b"both NULL" in lib.pa_last_error_message()
    pdims.num_updates = 2
    args = [fake[0], fake[1], None] + fake[3:5] + [pdims] + fake[5:16] + [None, 0] + [fake[16], 4096, None]
    assert lib.pa_pack(*args) == native.PA_ERR_INVALID_ARGUMENT
    assert b"2 updates" in lib.pa_last_error_message()
    rows = native.PaNewRows(None, 0x1000, 128, 1024, 128, 1024)
    rc = lib.pa_decode_append(*([None] * 3), 0, native.PaStepDims(), rows, *([None] * 4), 1, None, 0, 1.0,
                              None, None, 0, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT and b"new_rows.key" in lib.pa_last_error_message()
    rows = native.PaNewRows(0x1000, None, 128, 1024, 128, 1024)
    rc = lib.pa_prefill_append(*([None] * 3), 0, native.PaStepDims(), rows, *([None] * 4), 1, 32, 1.0,
                               None, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT and b"new_rows.value" in lib.pa_last_error_message()
    assert lib.pa_calibrate_mfma(None, 1, 1, 0, None) == native.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_calibrate_mfma(0x1000, 0, 1, 0, None) == native.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_calibrate_mfma(0x1000, 1, 1, 3, None) == native.PA_ERR_INVALID_ARGUMENT
    assert b"valu_per_mfma" in lib.pa_last_error_message()
    assert lib.pa_calibrate_mfma_flops(512, 4096) == 512 * 8 * 4096 * 2 * 32768
    assert lib.pa_calibrate_mfma_flops(0, 4096) == 0
    for data, nbytes, out, wgs in ((None, 64, 0x1000, 4), (0x1000, 24, 0x1000, 4), (0x1008, 64, 0x1000, 4),
                                   (0x1000, 64, None, 4), (0x1000, 64, 0x1000, 0)):
        assert lib.pa_calibrate_read(data, nbytes, out, wgs, None) == native.PA_ERR_INVALID_ARGUMENT
    assert b"pa_calibrate_read" in lib.pa_last_error_message()
    for direction in (-1, 2):
        rc = lib.pa_swap_blocks(None, None, None, 1, 1, 1, 1, 16, direction, None)
        assert rc == native.PA_ERR_INVALID_ARGUMENT and b"direction" in lib.pa_last_error_message()
    rc = lib.pa_swap_blocks(None, None, None, 1, 1, 1, 1, 16, native.PA_SWAP_OUT, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT and b"device_cache must not be NULL" in lib.pa_last_error_message()
    assert lib.pa_swap_blocks(None, None, None, 0, 1, 1, 1, 16, native.PA_SWAP_IN, None) == native.PA_OK


DECODE_POINTERS = ["query", "key_cache", "value_cache", "output", "block_tables", "context_lens", "cu_seqlens",
                   "decode_items"]


@pytest.mark.parametrize("missing", DECODE_POINTERS)
def test_decode_and_prefill_reject_null_pointers(missing):
    """With work to do, every required device pointer is checked before any
    launch: a NULL gives PA_ERR_INVALID_ARGUMENT and a message naming it."""
    native = pkg("_native")
    lib = native.load_library()
    dims = native.PaStepDims(num_seqs=1, num_query_tokens=1, num_query_heads=8, num_kv_heads=4, head_dim=64,
                             block_size=16, total_blocks=8, num_layers=1, max_blocks_per_seq=1,
                             partition_size=512, dtype=native.PA_DTYPE_BF16, q_token_stride=512, q_head_stride=64)
    fake = {name: 0x1000 * (i + 1) for i, name in enumerate(DECODE_POINTERS)}
    fake[missing] = None
    p = fake
    rc = lib.pa_decode(p["query"], p["key_cache"], p["value_cache"], 0, dims, p["block_tables"],
                       p["context_lens"], p["cu_seqlens"], p["decode_items"], 1, None, 0, 1.0, p["output"],
                       None, 0, None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_last_error_message() == f"pa_decode: {missing} must not be NULL".encode()
    name = "prefill_items" if missing == "decode_items" else missing
    rc = lib.pa_prefill(p["query"], p["key_cache"], p["value_cache"], 0, dims, p["block_tables"],
                        p["context_lens"], p["cu_seqlens"], p["decode_items"], 1, 16, 1.0, p["output"], None)
    assert rc == native.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_last_error_message() == f"pa_prefill: {name} must not be NULL".encode()


def test_reference_abi_latches_errors():
    native = pkg("_native")
    lib = native.load_library()
    dims = native.PagedAttentionDims(num_query_heads=3, num_query_tokens=1, head_dim=8, num_layers=1,
                                     total_blocks=1, block_size=4, num_kv_heads=2, num_context_tokens=1)
    lib.paged_attention(None, None, None, 0, dims, None, None, 1.0, None, None, None)
    assert lib.pa_last_error() == native.PA_ERR_INVALID_ARGUMENT
    dims.num_query_heads = 4
    lib.paged_attention(None, None, None, 1, dims, None, None, 1.0, None, None, None)
    assert lib.pa_last_error() == native.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_last_error_message() == b"layer_idx out of range"


def test_workspace_size():
    native = pkg("_native")
    lib = native.load_library()
    ops = pkg("paged_ops")
    dims = native.PaStepDims(num_query_heads=32, num_kv_heads=8, head_dim=128)
    assert lib.pa_decode_workspace_size(dims, 925) == ops.decode_workspace_bytes(925, 32, 128)
    assert lib.pa_decode_workspace_size(dims, 0) == 0
    # paired heads keep the real partial layout
    dims = native.PaStepDims(num_query_heads=16, num_kv_heads=4, head_dim=64, dtype=native.PA_DTYPE_BF16)
    assert lib.pa_decode_workspace_size(dims, 77) == ops.decode_workspace_bytes(77, 16, 64)
    assert lib.pa_decode_merge_state_size(dims, 77) == 0  # no sequences: no merge records


@pytest.mark.parametrize("hq,hkv,d,dtype,units", [
    (32, 8, 128, "PA_DTYPE_BF16", 4),    # paired KV heads: one record per pair
    (32, 8, 128, "PA_DTYPE_F32", 8),     # one per KV head
    (64, 2, 128, "PA_DTYPE_BF16", 2 * 4),  # a group of 32 runs as 4 sub-groups of 8 per KV head
    (8, 8, 64, "PA_DTYPE_F32", 8),
])
def test_merge_state_size(hq, hkv, d, dtype, units):
    """8 bytes of merge records per (sequence, decode workgroup of an item),
    rounded up to 256, after the partials; none without decode items."""
    native = pkg("_native")
    lib = native.load_library()
    ops = pkg("paged_ops")
    for b in (1, 37, 256):
        dims = native.PaStepDims(num_seqs=b, num_query_heads=hq, num_kv_heads=hkv, head_dim=d,
                                 dtype=getattr(native, dtype))
        assert lib.pa_decode_workgroups_per_item(dims.dtype, d, hkv, hq) == units
        state = -(-8 * b * units // 256) * 256
        assert lib.pa_decode_merge_state_size(dims, 50) == state
        assert lib.pa_decode_workspace_size(dims, 50) == ops.decode_workspace_bytes(50, hq, d) + state
        assert lib.pa_decode_workspace_size(dims, 0) == lib.pa_decode_merge_state_size(dims, 0) == 0


def test_workgroups_per_item():
    native = pkg("_native")
    lib = native.load_library()
    bf16, f32 = native.PA_DTYPE_BF16, native.PA_DTYPE_F32
    # (dtype, head_dim, H_kv, H_q) -> decode partition workgroups per work item
    cases = {
        # pairs of adjacent KV heads: half the KV heads
        (bf16, 64, 8, 8): 4, (bf16, 64, 8, 16): 4, (bf16, 64, 8, 24): 4, (bf16, 64, 8, 32): 4,
        (bf16, 128, 8, 8): 4, (bf16, 128, 32, 32): 16, (bf16, 128, 8, 16): 4, (bf16, 128, 8, 32): 4,
        # one per KV head: groups of 5-8, an odd KV head count, fp32
        (bf16, 64, 8, 40): 8, (bf16, 128, 8, 48): 8, (bf16, 64, 3, 9): 3,
        (f32, 64, 8, 8): 8, (f32, 128, 8, 16): 8,
        # groups above 8: the fewest equal sub-groups of at most 8 heads
        (bf16, 128, 8, 128): 16, (bf16, 128, 4, 48): 8, (f32, 64, 2, 22): 22, (bf16, 128, 1, 64): 8,
        (bf16, 64, 2, 18): 6,
        # fp16 pairs like bf16
        (native.PA_DTYPE_F16, 64, 8, 8): 4, (native.PA_DTYPE_F16, 128, 2, 8): 1,
        # heads of 96 and 256 are never paired
        (bf16, 96, 8, 8): 8, (bf16, 256, 8, 16): 8,
        # no tuned kernel (the generic one runs a workgroup per KV head's rows)
        (bf16, 112, 8, 8): 8, (bf16, 128, 1, 72): 1,
        # rejected head counts
        (bf16, 64, 0, 8): 0, (bf16, 64, 8, 12): 0, (bf16, 64, 8, 0): 0,
    }
    for (dtype, d, hkv, hq), want in cases.items():
        assert lib.pa_decode_workgroups_per_item(dtype, d, hkv, hq) == want, (dtype, d, hkv, hq)


def test_prefill_tile():
    lib = pkg("_native").load_library()
    ops = pkg("paged_ops")
    # 128 query rows over one workgroup's heads; groups above 8 split into the
    # fewest equal sub-groups of at most 8 heads
    cases = {(8, 8): 128, (32, 8): 32, (24, 8): 42, (64, 8): 16, (9, 3): 42, (7, 1): 18,
             (96, 8): 21, (128, 8): 16, (9, 1): 42, (64, 1): 16, (11, 1): 128,
             (0, 8): 0, (12, 8): 0, (8, 0): 0}
    for (hq, hkv), want in cases.items():
        assert lib.pa_prefill_tile(hq, hkv) == want, (hq, hkv)
    assert ops.prefill_tile_for(128, 8) == 16
    assert ops.prefill_tile_for(12, 8) == 128  # rejected counts: one workgroup row of tokens


def test_product_path_fails_loudly_without_library(monkeypatch, tmp_path):
    native = pkg("_native")
    monkeypatch.setattr(native, "LIBRARY_PATH", tmp_path / "missing.so")
    monkeypatch.setattr(native, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        native.load_library()


def test_map_host_memory_rejects_unpinned_and_null():
    native = pkg("_native")
    lib = native.load_library()
    out = ctypes.c_void_p()
    assert lib.pa_map_host_memory(None, ctypes.byref(out)) == native.PA_ERR_INVALID_ARGUMENT
    assert b"NULL" in lib.pa_last_error_message()
