// extern "C" entry points of libpaged_attention_amd.so (declared in
// include/paged_attention_amd.h).  Validation lives here; the kernels trust
// what passes it.  Nothing in this file allocates, frees or synchronises.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <initializer_list>
#include <mutex>

#include "pa_common.hpp"
#include "pa_error.hpp"
#include "pa_launch.hpp"

namespace {

thread_local char g_msg[512] = "";
thread_local int g_ref_abi_status = PA_OK;

int vfail(int code, const char* fmt, va_list ap) {
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  return code;
}

__attribute__((format(printf, 2, 3))) int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vfail(code, fmt, ap);
  va_end(ap);
  return code;
}

int from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return PA_OK;
  if (e == hipErrorNotSupported) return fail(PA_ERR_UNSUPPORTED, "%s: shape not supported", what);
  return fail(PA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

int elem_bytes(int dtype) {
  switch (dtype) {
    case PA_DTYPE_F32: return 4;
    case PA_DTYPE_BF16: return 2;
    case PA_DTYPE_F16: return 2;
    default: return 0;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int log2_exact(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return (1 << r) == v ? r : -1;
}

int check_step(const PaStepDims& d, const char* who) {
  if (elem_bytes(d.dtype) == 0) return fail(PA_ERR_INVALID_ARGUMENT, "%s: unknown dtype %d", who, d.dtype);
  if (d.num_seqs < 0 || d.num_query_tokens < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: negative batch size", who);
  if (d.num_query_heads <= 0 || d.num_kv_heads <= 0 || d.head_dim <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: heads and head_dim must be positive", who);
  if (d.num_query_heads % d.num_kv_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "%s: num_query_heads must be a multiple of num_kv_heads for GQA", who);
  if (d.block_size <= 0 || d.total_blocks <= 0 || d.num_layers <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: cache geometry must be positive", who);
  if (d.max_blocks_per_seq < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: negative block-table stride", who);
  return PA_OK;
}

// PA_ERR_INVALID_ARGUMENT naming the first pointer of `list` that is NULL.
struct Required {
  const void* ptr;
  const char* name;
};
int require(const char* who, std::initializer_list<Required> list) {
  for (const Required& r : list)
    if (r.ptr == nullptr) return fail(PA_ERR_INVALID_ARGUMENT, "%s: %s must not be NULL", who, r.name);
  return PA_OK;
}

const char* layer_base(const void* cache, const PaStepDims& d, int32_t layer_idx) {
  const int64_t span = static_cast<int64_t>(d.total_blocks) * d.block_size * d.num_kv_heads *
                       d.head_dim * elem_bytes(d.dtype);
  return reinterpret_cast<const char*>(cache) + span * layer_idx;
}

}  // namespace

int pa::set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vfail(code, fmt, ap);
  va_end(ap);
  return code;
}

const char* pa::last_error_message() { return g_msg; }

// Split-K partials of pa_decode_no_alloc: a file-scope array every device
// the library runs on holds once, from the load of this code object until
// the process ends.  In host code `scratch` is only a stand-in for the
// symbol; kernels get the device address that hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[PA_DECODE_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up with
// hipGetSymbolAddress on the first call per device and kept.
int scratch_address(void** out, const char* who) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PA_ERR_LAUNCH, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(PA_ERR_UNSUPPORTED, "%s: device %d is beyond the %d the scratch table holds", who, dev,
                kMaxScratchDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr) {
        (void)hipGetLastError();  // leave no stale error for the next launch check
        return fail(PA_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                    hipGetErrorString(e));
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return PA_OK;
}

}  // namespace

extern "C" {

int pa_abi_version(void) { return 13; }

const char* pa_error_string(int code) {
  switch (code) {
    case PA_OK: return "ok";
    case PA_ERR_INVALID_ARGUMENT: return "invalid argument";
    case PA_ERR_UNSUPPORTED: return "unsupported shape";
    case PA_ERR_WORKSPACE: return "workspace missing or too small";
    case PA_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown error";
  }
}

const char* pa_last_error_message(void) { return g_msg; }

int pa_map_host_memory(const void* host_ptr, void** device_ptr) {
  if (host_ptr == nullptr || device_ptr == nullptr)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_map_host_memory: NULL pointer");
  *device_ptr = nullptr;
  const hipError_t e = hipHostGetDevicePointer(device_ptr, const_cast<void*>(host_ptr), 0);
  if (e != hipSuccess || *device_ptr == nullptr) {
    (void)hipGetLastError();  // leave no stale error for the next launch check
    *device_ptr = nullptr;
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_map_host_memory: not pinned host memory (%s)",
                hipGetErrorString(e));
  }
  return PA_OK;
}

int pa_last_error(void) { return g_ref_abi_status; }

void paged_attention(const float* query, const float* key_cache, const float* value_cache,
                     int32_t layer_idx, PagedAttentionDims dims, const int32_t* gather_slots,
                     const uint8_t* attention_mask, float scaling, float* output, float* scratch,
                     void* stream) {
  (void)scratch;
  g_ref_abi_status = PA_OK;
  // Checks of csrc/src/bindings.cpp:25-48.
  if (dims.num_kv_heads <= 0 || dims.num_query_heads % dims.num_kv_heads != 0) {
    g_ref_abi_status = fail(PA_ERR_INVALID_ARGUMENT,
                            "num_query_heads must be a multiple of num_kv_heads for GQA");
    return;
  }
  if (layer_idx < 0 || layer_idx >= dims.num_layers) {
    g_ref_abi_status = fail(PA_ERR_INVALID_ARGUMENT, "layer_idx out of range");
    return;
  }
  if (dims.num_query_tokens < 0 || dims.num_context_tokens < 0 || dims.head_dim <= 0 ||
      dims.block_size <= 0 || dims.total_blocks < 0) {
    g_ref_abi_status = fail(PA_ERR_INVALID_ARGUMENT, "negative dimension");
    return;
  }
  if (!pa::generic_supported(PA_DTYPE_F32, dims.head_dim)) {
    g_ref_abi_status = fail(PA_ERR_UNSUPPORTED, "head_dim %d not supported", dims.head_dim);
    return;
  }
  pa::GenericArgs a{};
  a.query = query;
  a.q_token_stride = dims.head_dim;
  a.q_head_stride = static_cast<int64_t>(dims.num_query_tokens) * dims.head_dim;
  const int64_t span = static_cast<int64_t>(dims.total_blocks) * dims.block_size *
                       dims.num_kv_heads * dims.head_dim;
  a.key_cache = key_cache + span * layer_idx;
  a.value_cache = value_cache + span * layer_idx;
  a.gather_slots = gather_slots;
  a.mask = attention_mask;
  a.total_blocks = dims.total_blocks;  // out-of-pool slots are skipped
  a.block_size = dims.block_size;
  a.num_context_tokens = dims.num_context_tokens;
  a.output = output;
  a.num_query_tokens = dims.num_query_tokens;
  a.num_query_heads = dims.num_query_heads;
  a.num_kv_heads = dims.num_kv_heads;
  a.head_dim = dims.head_dim;
  a.scale_log2e = scaling * pa::kLog2e;
  g_ref_abi_status = from_hip(
      pa::launch_generic(a, PA_DTYPE_F32, true, static_cast<hipStream_t>(stream)), "paged_attention");
}

size_t pa_pack_workspace_size(int32_t num_seqs) { return pa::pack_workspace_size(num_seqs); }

int pa_pack(int32_t* block_tables, const int32_t* rows, const int32_t* updates,
            const int64_t* start_positions, const int64_t* new_token_counts, PaPackDims dims,
            int32_t* step_block_tables, int32_t* step_rows, int64_t* cu_seqlens, int64_t* cu_context_offsets,
            int32_t* context_lens, int64_t* scatter_slots, int64_t* position_ids,
            int64_t* gather_slots, int32_t* decode_items, int32_t* merge_items,
            int32_t* prefill_items, void* clear, size_t clear_bytes, void* workspace,
            size_t workspace_bytes, void* stream) {
  if (dims.num_seqs < 0) return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: negative num_seqs");
  if (clear_bytes > 0 && (clear == nullptr || !aligned16(clear) || clear_bytes % 16 != 0))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_pack: clear must be a 16-byte aligned region of whole 16-byte words (%zu bytes given)",
                clear_bytes);
  if (dims.block_size <= 0) return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: block_size must be positive");
  if (dims.max_blocks_per_seq < 0 || dims.num_table_rows < 0 || dims.num_updates < 0 ||
      dims.step_table_width < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: negative table geometry or update count");
  if (dims.partition_size <= 0 || dims.prefill_tile <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: partition and prefill tile must be positive");
  if (cu_seqlens == nullptr || cu_context_offsets == nullptr)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: cu_seqlens and cu_context_offsets are required");
  // A re-run reads each sequence's row from the workspace: the table's row
  // count is the caller's in every mode.
  const int32_t table_rows = dims.num_table_rows > 0 ? dims.num_table_rows : dims.num_seqs;
  if ((start_positions == nullptr) != (new_token_counts == nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_pack: start_positions and new_token_counts are given together or both NULL (re-run)");
  if (dims.num_seqs > 0) {
    int rc = require("pa_pack", {{context_lens, "context_lens"},
                                 {scatter_slots, "scatter_slots"},
                                 {position_ids, "position_ids"}});
    if (rc != PA_OK) return rc;
  }
  if (block_tables == nullptr && dims.max_blocks_per_seq > 0 && table_rows > 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: block_tables must not be NULL");
  if (dims.num_updates > 0 && (updates == nullptr || block_tables == nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: %d updates given without updates or block_tables",
                dims.num_updates);
  if (step_block_tables != nullptr && dims.step_table_width == 0 && dims.num_seqs > 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: step_block_tables given with step_table_width 0");
  if (!aligned16(merge_items))
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_pack: merge_items must be 16-byte aligned");
  const size_t need = pa::pack_workspace_size(dims.num_seqs);
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return fail(PA_ERR_WORKSPACE, "pa_pack: a 16-byte aligned workspace of %zu bytes is needed, %zu given",
                need, workspace == nullptr ? size_t(0) : workspace_bytes);
  pa::PackArgs a{};
  a.block_tables = block_tables;
  a.rows = rows;
  a.updates = updates;
  a.start_positions = start_positions;
  a.new_token_counts = new_token_counts;
  a.step_block_tables = step_block_tables;
  a.step_rows = step_rows;
  a.cu_seqlens = cu_seqlens;
  a.cu_context_offsets = cu_context_offsets;
  a.context_lens = context_lens;
  a.scatter_slots = scatter_slots;
  a.position_ids = position_ids;
  a.gather_slots = gather_slots;
  a.decode_items = decode_items;
  a.merge_items = merge_items;
  a.prefill_items = prefill_items;
  a.ws_header = reinterpret_cast<int32_t*>(workspace);
  a.ws_seq = reinterpret_cast<int4*>(reinterpret_cast<char*>(workspace) + pa::kPackHeaderBytes);
  a.num_seqs = dims.num_seqs;
  a.num_table_rows = block_tables != nullptr ? table_rows : 0;
  a.num_updates = dims.num_updates;
  a.step_table_width = step_block_tables != nullptr ? dims.step_table_width : 0;
  a.block_size = dims.block_size;
  a.block_table_stride = dims.max_blocks_per_seq;
  a.partition = dims.partition_size;
  a.prefill_tile = dims.prefill_tile;
  a.max_query_tokens = dims.max_query_tokens;
  a.max_context_tokens = gather_slots ? dims.max_context_tokens : 0;
  a.max_decode_items = decode_items ? dims.max_decode_items : 0;
  a.max_merge_items = merge_items ? dims.max_merge_items : 0;
  a.max_prefill_items = prefill_items ? dims.max_prefill_items : 0;
  a.clear = static_cast<uint4*>(clear);
  a.clear_words = static_cast<int64_t>(clear_bytes / 16);
  a.fused = pa::pack_fusable(a, dims.max_new_tokens, dims.max_context) ? 1 : 0;
  return from_hip(pa::launch_pack(a, static_cast<hipStream_t>(stream)), "pa_pack");
}

int pa_reshape_and_cache(const void* key, const void* value, int64_t key_token_stride,
                         int64_t key_head_stride, int64_t value_token_stride,
                         int64_t value_head_stride, void* key_cache, void* value_cache,
                         const int64_t* slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
                         int32_t head_dim, int32_t block_size, int32_t total_blocks,
                         int32_t num_layers, int32_t layer_idx, int32_t dtype, void* stream) {
  const int eb = elem_bytes(dtype);
  if (eb == 0) return fail(PA_ERR_INVALID_ARGUMENT, "pa_reshape_and_cache: unknown dtype %d", dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || total_blocks < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_reshape_and_cache: bad geometry");
  if (layer_idx < 0 || layer_idx >= num_layers)
    return fail(PA_ERR_INVALID_ARGUMENT, "Layer index %d out of range (num_layers=%d)", layer_idx,
                num_layers);
  if (num_tokens == 0) return PA_OK;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_reshape_and_cache: null buffer");
  pa::CacheWriteArgs a{};
  const int64_t span = static_cast<int64_t>(total_blocks) * block_size * num_kv_heads * head_dim * eb;
  a.key = key;
  a.value = value;
  a.key_token_stride = key_token_stride;
  a.key_head_stride = key_head_stride;
  a.value_token_stride = value_token_stride;
  a.value_head_stride = value_head_stride;
  a.key_cache = reinterpret_cast<char*>(key_cache) + span * layer_idx;
  a.value_cache = reinterpret_cast<char*>(value_cache) + span * layer_idx;
  a.slot_mapping = slot_mapping;
  a.num_slots = static_cast<int64_t>(total_blocks) * block_size;
  a.num_tokens = num_tokens;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  return from_hip(pa::launch_cache_write(a, dtype, static_cast<hipStream_t>(stream)),
                  "pa_reshape_and_cache");
}

int pa_copy_blocks(const void* src_cache, void* dst_cache, const int64_t* block_mapping,
                   int64_t num_pairs, int32_t num_layers, int64_t src_total_blocks,
                   int64_t dst_total_blocks, int64_t block_bytes, void* stream) {
  if (num_pairs < 0 || num_layers < 0 || src_total_blocks < 0 || dst_total_blocks < 0 ||
      block_bytes < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_copy_blocks: negative size");
  if (num_pairs == 0 || num_layers == 0 || block_bytes == 0) return PA_OK;
  if (src_cache == nullptr || dst_cache == nullptr || block_mapping == nullptr)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_copy_blocks: missing cache or block mapping");
  if (block_bytes % 4 != 0 || (reinterpret_cast<uintptr_t>(src_cache) & 3u) != 0 ||
      (reinterpret_cast<uintptr_t>(dst_cache) & 3u) != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_copy_blocks: caches and block size must be 4-byte aligned");
  if (num_pairs * static_cast<int64_t>(num_layers) > 0x7fffffffLL)
    return fail(PA_ERR_UNSUPPORTED, "pa_copy_blocks: too many blocks in one call");
  pa::CopyBlocksArgs a{};
  a.src = src_cache;
  a.dst = dst_cache;
  a.block_mapping = block_mapping;
  a.num_pairs = num_pairs;
  a.src_total_blocks = src_total_blocks;
  a.dst_total_blocks = dst_total_blocks;
  a.block_bytes = block_bytes;
  a.num_layers = num_layers;
  const bool vec16 = block_bytes % 16 == 0 && aligned16(src_cache) && aligned16(dst_cache);
  return from_hip(pa::launch_copy_blocks(a, vec16, static_cast<hipStream_t>(stream)),
                  "pa_copy_blocks");
}

int pa_swap_blocks(void* device_cache, void* host_cache, const int64_t* block_mapping,
                   int64_t num_pairs, int32_t num_layers, int64_t device_total_blocks,
                   int64_t host_total_blocks, int64_t block_bytes, int32_t direction,
                   void* stream) {
  if (direction != PA_SWAP_OUT && direction != PA_SWAP_IN)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_swap_blocks: direction must be PA_SWAP_OUT or PA_SWAP_IN, got %d",
                direction);
  if (num_pairs < 0 || num_layers < 0 || device_total_blocks < 0 || host_total_blocks < 0 ||
      block_bytes < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_swap_blocks: negative size");
  if (num_pairs == 0 || num_layers == 0 || block_bytes == 0) return PA_OK;
  int rc = require("pa_swap_blocks", {{device_cache, "device_cache"}, {host_cache, "host_cache"},
                                      {block_mapping, "block_mapping"}});
  if (rc != PA_OK) return rc;
  void* host_view = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&host_view, host_cache, 0);
  if (e != hipSuccess || host_view == nullptr) {
    (void)hipGetLastError();  // leave no stale error for the next launch check
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_swap_blocks: host_cache is not pinned host memory (%s)",
                hipGetErrorString(e));
  }
  const bool out = direction == PA_SWAP_OUT;
  return pa_copy_blocks(out ? device_cache : host_view, out ? host_view : device_cache, block_mapping,
                        num_pairs, num_layers, out ? device_total_blocks : host_total_blocks,
                        out ? host_total_blocks : device_total_blocks, block_bytes, stream);
}

namespace {
// Two adjacent KV heads run as one workgroup reading one row of twice the
// length per token (pa::decode_pairs_heads has the shapes).
bool decode_pairs(const PaStepDims& d) {
  const int group = d.num_kv_heads > 0 ? d.num_query_heads / d.num_kv_heads : 0;
  return pa::decode_pairs_heads(d.dtype, d.head_dim, d.num_kv_heads, group);
}
// Bytes of merge records of a step: 8 per (sequence, decode unit,
// sub-group), rounded up to 256 bytes.
size_t merge_state_bytes(const PaStepDims& d) {
  if (d.num_seqs <= 0 || d.num_kv_heads <= 0 || d.num_query_heads < d.num_kv_heads) return 0;
  const int group = d.num_query_heads / d.num_kv_heads;
  const bool pair = decode_pairs(d);
  const int64_t units = (pair ? d.num_kv_heads / 2 : d.num_kv_heads) *
                        static_cast<int64_t>(pair ? 1 : pa::decode_sub_groups(group));
  return (static_cast<size_t>(d.num_seqs) * units * 8 + 255) & ~size_t(255);
}
struct DecodeWorkspaceLayout {
  size_t acc, ml, state, total;
};
// part_acc [items, H_q, D] fp32 | part_ml [items, H_q, 2] fp32 | merge
// records (merge_state_bytes), each rounded up to 256 bytes.
DecodeWorkspaceLayout decode_workspace_layout(const PaStepDims& dims, int64_t items) {
  DecodeWorkspaceLayout w{0, 0, 0, 0};
  if (items <= 0 || dims.num_query_heads <= 0 || dims.head_dim <= 0) return w;
  const size_t rows = static_cast<size_t>(items) * dims.num_query_heads;
  w.acc = (rows * dims.head_dim * sizeof(float) + 255) & ~size_t(255);
  w.ml = (rows * 2 * sizeof(float) + 255) & ~size_t(255);
  w.state = merge_state_bytes(dims);
  w.total = w.acc + w.ml + w.state;
  return w;
}
}  // namespace

size_t pa_decode_workspace_size(PaStepDims dims, int64_t num_decode_items) {
  return decode_workspace_layout(dims, num_decode_items).total;
}

size_t pa_decode_merge_state_size(PaStepDims dims, int64_t num_decode_items) {
  return decode_workspace_layout(dims, num_decode_items).state;
}

int32_t pa_decode_workgroups_per_item(int32_t dtype, int32_t head_dim, int32_t num_kv_heads,
                                      int32_t num_query_heads) {
  if (num_kv_heads <= 0 || num_query_heads <= 0 || num_query_heads % num_kv_heads != 0) return 0;
  const int group = num_query_heads / num_kv_heads;
  if (pa::decode_pairs_heads(dtype, head_dim, num_kv_heads, group)) return num_kv_heads / 2;
  if (!pa::decode_fast_path_supported(dtype, head_dim, group, 16, 32)) return num_kv_heads;
  return num_kv_heads * pa::decode_sub_groups(group);
}

int32_t pa_prefill_tile(int32_t num_query_heads, int32_t num_kv_heads) {
  if (num_kv_heads <= 0 || num_query_heads <= 0 || num_query_heads % num_kv_heads != 0) return 0;
  return pa::prefill_tile_for(num_query_heads / num_kv_heads);
}

int32_t pa_decode_workgroups_per_cu(int32_t dtype, int32_t head_dim, int32_t num_kv_heads,
                                    int32_t num_query_heads) {
  if (pa_decode_workgroups_per_item(dtype, head_dim, num_kv_heads, num_query_heads) == 0) {
    fail(PA_ERR_INVALID_ARGUMENT, "pa_decode_workgroups_per_cu: bad head counts %d / %d",
         num_query_heads, num_kv_heads);
    return 0;
  }
  const int group = num_query_heads / num_kv_heads;
  if (!pa::decode_fast_path_supported(dtype, head_dim, group, 16, 32)) {
    fail(PA_ERR_UNSUPPORTED, "pa_decode_workgroups_per_cu: no tuned decode kernel for dtype %d, "
         "head_dim %d, %d query heads per KV head", dtype, head_dim, group);
    return 0;
  }
  const bool pair = pa::decode_pairs_heads(dtype, head_dim, num_kv_heads, group);
  int per_cu = 0;
  const hipError_t err = pa::decode_workgroups_per_cu(dtype, head_dim, group, pair, &per_cu);
  if (err != hipSuccess) {
    from_hip(err, "pa_decode_workgroups_per_cu");
    return 0;
  }
  return per_cu;
}

int pa_decode(const void* query, const void* key_cache, const void* value_cache,
              int32_t layer_idx, PaStepDims dims, const int32_t* block_tables,
              const int32_t* context_lens, const int64_t* cu_seqlens,
              const int32_t* decode_items, int64_t num_decode_items,
              const int32_t* merge_items, int64_t num_merge_items, float scaling,
              void* output, void* workspace, size_t workspace_bytes, void* stream) {
  return pa_decode_phases(PA_DECODE_PHASE_PARTITIONS | PA_DECODE_PHASE_MERGE, query, key_cache,
                          value_cache, layer_idx, dims, block_tables, context_lens, cu_seqlens,
                          decode_items, num_decode_items, merge_items, num_merge_items, scaling,
                          output, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace {

// pa_decode_phases with the split-K partials in `workspace`, or, when
// `use_scratch`, in this device's `scratch` array (workspace ignored).
int decode_phases(const char* who, bool use_scratch, int32_t phases, const void* query,
                  const void* key_cache, const void* value_cache, int32_t layer_idx,
                  PaStepDims dims, const int32_t* block_tables, const int32_t* context_lens,
                  const int64_t* cu_seqlens, const int32_t* decode_items,
                  int64_t num_decode_items, const int32_t* merge_items, int64_t num_merge_items,
                  float scaling, void* output, void* workspace, size_t workspace_bytes,
                  void* stream, const PaNewRows* new_rows = nullptr) {
  if (phases <= 0 || (phases & ~(PA_DECODE_PHASE_PARTITIONS | PA_DECODE_PHASE_MERGE)) != 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: phases must be a non-empty mask of "
                "PA_DECODE_PHASE_PARTITIONS and PA_DECODE_PHASE_MERGE, got %d", who, phases);
  int rc = check_step(dims, who);
  if (rc != PA_OK) return rc;
  if (layer_idx < 0 || layer_idx >= dims.num_layers)
    return fail(PA_ERR_INVALID_ARGUMENT, "Layer index %d out of range (num_layers=%d)", layer_idx,
                dims.num_layers);
  if (num_decode_items <= 0 || dims.num_seqs == 0) return PA_OK;
  if (num_decode_items * static_cast<int64_t>(dims.num_kv_heads) *
          pa::decode_sub_groups(dims.num_query_heads / dims.num_kv_heads) > 0x7fffffffLL)
    return fail(PA_ERR_UNSUPPORTED, "%s: too many work items", who);
  rc = require(who, {{query, "query"}, {key_cache, "key_cache"}, {value_cache, "value_cache"},
                    {output, "output"}, {block_tables, "block_tables"},
                    {context_lens, "context_lens"}, {cu_seqlens, "cu_seqlens"},
                    {decode_items, "decode_items"}});
  if (rc != PA_OK) return rc;
  if (num_merge_items < 0 || (num_merge_items > 0 && merge_items == nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: merge_items is required when num_merge_items > 0", who);
  if (!aligned16(merge_items))
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: merge_items must be 16-byte aligned", who);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int group = dims.num_query_heads / dims.num_kv_heads;
  const int eb = elem_bytes(dims.dtype);
  const int log2_bs = log2_exact(dims.block_size);
  const bool pair = decode_pairs(dims);
  const bool fast =
      pa::decode_fast_path_supported(dims.dtype, dims.head_dim, group, dims.block_size,
                                     dims.partition_size) &&
      aligned16(query) && aligned16(key_cache) && aligned16(value_cache) &&
      (dims.q_token_stride * eb) % 16 == 0 && (dims.q_head_stride * eb) % 16 == 0;
  if (new_rows != nullptr) {
    // The fused write moves 16-byte pieces of whole heads.
    const bool fused = fast && aligned16(new_rows->key) && aligned16(new_rows->value) &&
                       (dims.head_dim * eb) % 16 == 0 && (new_rows->key_token_stride * eb) % 16 == 0 &&
                       (new_rows->key_head_stride * eb) % 16 == 0 &&
                       (new_rows->value_token_stride * eb) % 16 == 0 &&
                       (new_rows->value_head_stride * eb) % 16 == 0;
    if (!fused)
      return fail(PA_ERR_UNSUPPORTED, "%s: this shape or alignment takes pa_reshape_and_cache + pa_decode", who);
  }
  if (fast) {
    const DecodeWorkspaceLayout wl = decode_workspace_layout(dims, num_decode_items);
    int32_t* merge_state = nullptr;
    if (use_scratch) {
      // Partials from the start of the array; merge records in its fixed
      // last PA_DECODE_SCRATCH_STATE_BYTES (zero from the load of the code
      // object on, and left zero by every launch), so what a call of another
      // shape left in the partials never reads as a record.
      const size_t partials = wl.acc + wl.ml;
      if (partials > PA_DECODE_SCRATCH_BYTES - PA_DECODE_SCRATCH_STATE_BYTES)
        return fail(PA_ERR_WORKSPACE,
                    "%s: %lld decode items need %zu bytes of split-K partials, more than the %zu "
                    "bytes of scratch; use pa_decode with a workspace",
                    who, static_cast<long long>(num_decode_items), partials,
                    static_cast<size_t>(PA_DECODE_SCRATCH_BYTES - PA_DECODE_SCRATCH_STATE_BYTES));
      rc = scratch_address(&workspace, who);
      if (rc != PA_OK) return rc;
      workspace_bytes = PA_DECODE_SCRATCH_BYTES;
      // More records than the region holds: the merge kernel combines the
      // partials instead.
      if (wl.state <= PA_DECODE_SCRATCH_STATE_BYTES)
        merge_state = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + PA_DECODE_SCRATCH_BYTES -
                                                 PA_DECODE_SCRATCH_STATE_BYTES);
    } else {
      if (workspace == nullptr || workspace_bytes < wl.total)
        return fail(PA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who, wl.total,
                    workspace_bytes);
      if (wl.state > 0) merge_state = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + wl.acc + wl.ml);
    }
    pa::DecodeArgs a{};
    a.query = query;
    a.q_token_stride = dims.q_token_stride;
    a.q_head_stride = dims.q_head_stride;
    a.key_cache = layer_base(key_cache, dims, layer_idx);
    a.value_cache = layer_base(value_cache, dims, layer_idx);
    a.block_tables = block_tables;
    a.rows = dims.block_table_rows;
    a.num_table_rows = dims.num_table_rows > 0 ? dims.num_table_rows : dims.num_seqs;
    a.context_lens = context_lens;
    a.cu_seqlens = cu_seqlens;
    a.items = decode_items;
    a.num_items = num_decode_items;
    a.output = output;
    a.part_acc = reinterpret_cast<float*>(workspace);
    a.part_ml = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + wl.acc);
    a.merge_items = merge_items;
    a.num_merge = merge_items != nullptr ? num_merge_items : 0;
    a.block_table_stride = dims.max_blocks_per_seq;
    a.num_kv_heads = pair ? dims.num_kv_heads / 2 : dims.num_kv_heads;
    a.total_blocks = dims.total_blocks;
    a.log2_block_size = log2_bs;
    a.partition = dims.partition_size;
    a.scale_log2e = scaling * pa::kLog2e;
    a.pair = pair ? 1 : 0;
    a.group = pair ? 2 * group : group;
    a.sub_groups = pair ? 1 : pa::decode_sub_groups(group);
    a.head_dim = dims.head_dim;
    // A record's fields hold counts and items below 65535.
    a.merge_state = num_decode_items < 65535 ? merge_state : nullptr;
    a.num_seqs = dims.num_seqs;
    if (new_rows != nullptr) {
      a.new_key = new_rows->key;
      a.new_value = new_rows->value;
      a.new_key_token_stride = new_rows->key_token_stride;
      a.new_key_head_stride = new_rows->key_head_stride;
      a.new_value_token_stride = new_rows->value_token_stride;
      a.new_value_head_stride = new_rows->value_head_stride;
    }
    return from_hip(
        pa::launch_decode(a, dims.dtype, dims.head_dim, group, num_decode_items, phases, s), who);
  }
  if (!pa::generic_supported(dims.dtype, dims.head_dim))
    return fail(PA_ERR_UNSUPPORTED, "%s: head_dim %d / dtype %d not supported", who,
                dims.head_dim, dims.dtype);
  // The generic kernel finishes every row in one pass: it is the partition
  // phase, and the merge phase has nothing to do.
  if (!(phases & PA_DECODE_PHASE_PARTITIONS)) return PA_OK;
  pa::GenericArgs a{};
  a.query = query;
  a.q_token_stride = dims.q_token_stride;
  a.q_head_stride = dims.q_head_stride;
  a.key_cache = layer_base(key_cache, dims, layer_idx);
  a.value_cache = layer_base(value_cache, dims, layer_idx);
  a.block_tables = block_tables;
  a.rows = dims.block_table_rows;
  a.num_table_rows = dims.num_table_rows > 0 ? dims.num_table_rows : dims.num_seqs;
  a.context_lens = context_lens;
  a.cu_seqlens = cu_seqlens;
  a.num_seqs = dims.num_seqs;
  a.block_table_stride = dims.max_blocks_per_seq;
  a.block_size = dims.block_size;
  a.total_blocks = dims.total_blocks;
  a.filter = 1;
  a.output = output;
  a.num_query_tokens = dims.num_query_tokens;
  a.num_query_heads = dims.num_query_heads;
  a.num_kv_heads = dims.num_kv_heads;
  a.head_dim = dims.head_dim;
  a.scale_log2e = scaling * pa::kLog2e;
  return from_hip(pa::launch_generic(a, dims.dtype, false, s), who);
}

}  // namespace

extern "C" {

int pa_decode_phases(int32_t phases, const void* query, const void* key_cache,
                     const void* value_cache, int32_t layer_idx, PaStepDims dims,
                     const int32_t* block_tables, const int32_t* context_lens,
                     const int64_t* cu_seqlens, const int32_t* decode_items,
                     int64_t num_decode_items, const int32_t* merge_items,
                     int64_t num_merge_items, float scaling, void* output, void* workspace,
                     size_t workspace_bytes, void* stream) {
  return decode_phases("pa_decode", false, phases, query, key_cache, value_cache, layer_idx, dims,
                       block_tables, context_lens, cu_seqlens, decode_items, num_decode_items,
                       merge_items, num_merge_items, scaling, output, workspace, workspace_bytes,
                       stream);
}

int pa_decode_append(const void* query, void* key_cache, void* value_cache, int32_t layer_idx,
                     PaStepDims dims, PaNewRows new_rows, const int32_t* block_tables,
                     const int32_t* context_lens, const int64_t* cu_seqlens,
                     const int32_t* decode_items, int64_t num_decode_items,
                     const int32_t* merge_items, int64_t num_merge_items, float scaling,
                     void* output, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = require("pa_decode_append", {{new_rows.key, "new_rows.key"}, {new_rows.value, "new_rows.value"}});
  if (rc != PA_OK) return rc;
  return decode_phases("pa_decode_append", false, PA_DECODE_PHASE_PARTITIONS | PA_DECODE_PHASE_MERGE, query,
                       key_cache, value_cache, layer_idx, dims, block_tables, context_lens, cu_seqlens,
                       decode_items, num_decode_items, merge_items, num_merge_items, scaling, output,
                       workspace, workspace_bytes, stream, &new_rows);
}

int pa_decode_no_alloc(const void* query, const void* key_cache, const void* value_cache,
                       int32_t layer_idx, PaStepDims dims, const int32_t* block_tables,
                       const int32_t* context_lens, const int64_t* cu_seqlens,
                       const int32_t* decode_items, int64_t num_decode_items,
                       const int32_t* merge_items, int64_t num_merge_items, float scaling,
                       void* output, void* stream) {
  return decode_phases("pa_decode_no_alloc", true,
                       PA_DECODE_PHASE_PARTITIONS | PA_DECODE_PHASE_MERGE, query, key_cache,
                       value_cache, layer_idx, dims, block_tables, context_lens, cu_seqlens,
                       decode_items, num_decode_items, merge_items, num_merge_items, scaling,
                       output, nullptr, 0, stream);
}

}  // extern "C"

namespace {

// pa_prefill, and with new_rows pa_prefill_append (the fast path only).
int prefill_impl(const char* who, const void* query, const void* key_cache, const void* value_cache,
                 int32_t layer_idx, PaStepDims dims, const int32_t* block_tables,
                 const int32_t* context_lens, const int64_t* cu_seqlens, const int32_t* prefill_items,
                 int64_t num_prefill_items, int32_t prefill_tile, float scaling, void* output,
                 void* stream, const PaNewRows* new_rows) {
  int rc = check_step(dims, who);
  if (rc != PA_OK) return rc;
  if (layer_idx < 0 || layer_idx >= dims.num_layers)
    return fail(PA_ERR_INVALID_ARGUMENT, "Layer index %d out of range (num_layers=%d)", layer_idx,
                dims.num_layers);
  if (num_prefill_items <= 0 || dims.num_seqs == 0) return PA_OK;
  rc = require(who, {{query, "query"}, {key_cache, "key_cache"}, {value_cache, "value_cache"},
                     {output, "output"}, {block_tables, "block_tables"},
                     {context_lens, "context_lens"}, {cu_seqlens, "cu_seqlens"},
                     {prefill_items, "prefill_items"}});
  if (rc != PA_OK) return rc;
  if (num_prefill_items * static_cast<int64_t>(dims.num_kv_heads) *
          pa::decode_sub_groups(dims.num_query_heads / dims.num_kv_heads) > 0x7fffffffLL)
    return fail(PA_ERR_UNSUPPORTED, "%s: too many work items", who);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int group = dims.num_query_heads / dims.num_kv_heads;
  const int eb = elem_bytes(dims.dtype);
  const bool fast =
      pa::prefill_fast_path_supported(dims.dtype, dims.head_dim, group, dims.block_size) &&
      prefill_tile == pa::prefill_tile_for(group) && dims.max_blocks_per_seq > 0 &&
      static_cast<int64_t>(dims.block_size) * dims.num_kv_heads * dims.head_dim * eb <= 0xffffffffLL &&
      aligned16(query) && aligned16(key_cache) &&
      aligned16(value_cache) && aligned16(output) && (dims.q_token_stride * eb) % 16 == 0 &&
      (dims.q_head_stride * eb) % 16 == 0;
  if (new_rows != nullptr) {
    // The kernels copy and store 16-byte pieces of whole heads; a copy's rows
    // sit at 32-bit offsets of at most 16 token strides from its base.
    const auto stride_ok = [&](int64_t st) { return st >= 0 && (st * eb) % 16 == 0; };
    const bool fused = fast && pa::prefill_append_supported(dims.dtype, dims.head_dim) &&
                       aligned16(new_rows->key) && aligned16(new_rows->value) &&
                       stride_ok(new_rows->key_token_stride) && stride_ok(new_rows->key_head_stride) &&
                       stride_ok(new_rows->value_token_stride) && stride_ok(new_rows->value_head_stride) &&
                       new_rows->key_token_stride * eb < (int64_t{1} << 24) &&
                       new_rows->value_token_stride * eb < (int64_t{1} << 24);
    if (!fused)
      return fail(PA_ERR_UNSUPPORTED, "%s: shape or alignment not taken by the fused write "
                  "(write the rows with pa_reshape_and_cache, then call pa_prefill)", who);
  }
  if (fast) {
    pa::PrefillArgs a{};
    a.query = query;
    a.q_token_stride = dims.q_token_stride;
    a.q_head_stride = dims.q_head_stride;
    a.key_cache = layer_base(key_cache, dims, layer_idx);
    a.value_cache = layer_base(value_cache, dims, layer_idx);
    a.block_tables = block_tables;
    a.rows = dims.block_table_rows;
    a.num_table_rows = dims.num_table_rows > 0 ? dims.num_table_rows : dims.num_seqs;
    a.context_lens = context_lens;
    a.cu_seqlens = cu_seqlens;
    a.items = prefill_items;
    a.output = output;
    a.block_table_stride = dims.max_blocks_per_seq;
    a.num_kv_heads = dims.num_kv_heads;
    a.total_blocks = dims.total_blocks;
    a.log2_block_size = log2_exact(dims.block_size);
    a.scale_log2e = scaling * pa::kLog2e;
    a.group = group;
    a.sub_groups = pa::decode_sub_groups(group);
    if (new_rows != nullptr) {
      a.new_key = new_rows->key;
      a.new_value = new_rows->value;
      a.new_key_token_stride = new_rows->key_token_stride;
      a.new_key_head_stride = new_rows->key_head_stride;
      a.new_value_token_stride = new_rows->value_token_stride;
      a.new_value_head_stride = new_rows->value_head_stride;
    }
    return from_hip(pa::launch_prefill(a, dims.dtype, dims.head_dim, group, num_prefill_items, s), who);
  }
  if (!pa::generic_supported(dims.dtype, dims.head_dim))
    return fail(PA_ERR_UNSUPPORTED, "pa_prefill: head_dim %d / dtype %d not supported",
                dims.head_dim, dims.dtype);
  pa::GenericArgs a{};
  a.query = query;
  a.q_token_stride = dims.q_token_stride;
  a.q_head_stride = dims.q_head_stride;
  a.key_cache = layer_base(key_cache, dims, layer_idx);
  a.value_cache = layer_base(value_cache, dims, layer_idx);
  a.block_tables = block_tables;
  a.rows = dims.block_table_rows;
  a.num_table_rows = dims.num_table_rows > 0 ? dims.num_table_rows : dims.num_seqs;
  a.context_lens = context_lens;
  a.cu_seqlens = cu_seqlens;
  a.num_seqs = dims.num_seqs;
  a.block_table_stride = dims.max_blocks_per_seq;
  a.block_size = dims.block_size;
  a.total_blocks = dims.total_blocks;
  a.filter = 2;
  a.output = output;
  a.num_query_tokens = dims.num_query_tokens;
  a.num_query_heads = dims.num_query_heads;
  a.num_kv_heads = dims.num_kv_heads;
  a.head_dim = dims.head_dim;
  a.scale_log2e = scaling * pa::kLog2e;
  return from_hip(pa::launch_generic(a, dims.dtype, false, s), who);
}

}  // namespace

extern "C" {

int pa_prefill(const void* query, const void* key_cache, const void* value_cache,
               int32_t layer_idx, PaStepDims dims, const int32_t* block_tables,
               const int32_t* context_lens, const int64_t* cu_seqlens,
               const int32_t* prefill_items, int64_t num_prefill_items, int32_t prefill_tile,
               float scaling, void* output, void* stream) {
  return prefill_impl("pa_prefill", query, key_cache, value_cache, layer_idx, dims, block_tables,
                      context_lens, cu_seqlens, prefill_items, num_prefill_items, prefill_tile, scaling,
                      output, stream, nullptr);
}

int pa_prefill_append(const void* query, void* key_cache, void* value_cache, int32_t layer_idx,
                      PaStepDims dims, PaNewRows new_rows, const int32_t* block_tables,
                      const int32_t* context_lens, const int64_t* cu_seqlens,
                      const int32_t* prefill_items, int64_t num_prefill_items, int32_t prefill_tile,
                      float scaling, void* output, void* stream) {
  int rc = require("pa_prefill_append", {{new_rows.key, "new_rows.key"}, {new_rows.value, "new_rows.value"}});
  if (rc != PA_OK) return rc;
  return prefill_impl("pa_prefill_append", query, key_cache, value_cache, layer_idx, dims, block_tables,
                      context_lens, cu_seqlens, prefill_items, num_prefill_items, prefill_tile, scaling,
                      output, stream, &new_rows);
}

}  // extern "C"
