// Kernel argument blocks and host-side launchers shared between the kernel
// sources and the C-ABI layer (abi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

// Decode (split-K) over block tables.
struct DecodeArgs {
  const void* query;
  int64_t q_token_stride;
  int64_t q_head_stride;
  const void* key_cache;    // base of the layer
  const void* value_cache;  // base of the layer
  const int32_t* block_tables;
  const int32_t* rows;      // row of block_tables per sequence, or null (row = seq)
  int32_t num_table_rows;   // rows of block_tables (a row outside reads as no blocks)
  const int32_t* context_lens;
  const int64_t* cu_seqlens;
  const int32_t* items;     // (seq, partition) pairs
  int64_t num_items;
  void* output;             // [T, H_q, D]
  float* part_acc;          // [items, H_q, D]
  float* part_ml;           // [items, H_q, 2]
  const int32_t* merge_items;  // first item of every multi-partition sequence
  int64_t num_merge;
  int32_t block_table_stride;
  int32_t num_kv_heads;
  int32_t total_blocks;
  int32_t log2_block_size;
  int32_t partition;
  float scale_log2e;
  // 1: two adjacent real KV heads of D/2 run as one of D (G counts the query
  // heads of both).  Every query head reads only its own half of the rows;
  // outputs and partials use the real layout [.., H_q, D/2].
  int32_t pair;
  // Query heads per num_kv_heads unit (for a pair, those of both heads) and
  // the workgroups that share them (1 unless the group is split because it
  // exceeds the largest kernel group; each then re-reads the unit's K/V).
  int32_t group;
  int32_t sub_groups;
  // pa_decode_append: the step's new K/V rows ([T, H_kv, head_dim], element
  // strides), written into the cache slot of position context_len - 1 by the
  // workgroups of each sequence's last partition before they read it; null
  // for the other entry points.
  const void* new_key;
  const void* new_value;
  int64_t new_key_token_stride;
  int64_t new_key_head_stride;
  int64_t new_value_token_stride;
  int64_t new_value_head_stride;
  int32_t head_dim;  // real head dim (the pair's unit row holds two heads)
  // Merge records of the in-launch split-K merge, 8 bytes per (sequence,
  // unit, sub-group): arrivals, first full-partition item, partial item.
  // Zero before the launch and left zero by it; null (always for 65535 or
  // more items): the partition phase stores partials only and the merge
  // kernel combines them.
  int32_t* merge_state;
  int32_t num_seqs;  // sequences the records cover
};

// Generic one-wave-per-(query token, head) attention: any head_dim <= 256,
// any GQA ratio, any block size.  Two context sources:
//   masked = 0: block tables + causal limit (flat ragged batch),
//   masked = 1: the reference ABI's flat gather list + dense uint8 mask.
struct GenericArgs {
  const void* query;
  int64_t q_token_stride;
  int64_t q_head_stride;
  const void* key_cache;   // base of the layer
  const void* value_cache;
  // block-table source
  const int32_t* block_tables;
  const int32_t* rows;  // row of block_tables per sequence, or null (row = seq)
  int32_t num_table_rows;
  const int32_t* context_lens;
  const int64_t* cu_seqlens;
  int32_t num_seqs;
  int32_t block_table_stride;
  int32_t block_size;
  int32_t total_blocks;
  int32_t filter;  // 0 = every token, 1 = decode sequences only, 2 = multi-token only
  // gather/mask source
  const int32_t* gather_slots;
  const uint8_t* mask;
  int32_t num_context_tokens;
  // common
  void* output;  // [T, H_q, D] contiguous
  int32_t num_query_tokens;
  int32_t num_query_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  float scale_log2e;
};

// Packing of one step (pack.hip): a one-workgroup scan and a per-sequence
// fill sharing a small workspace, or the scan alone for a small decode step.
constexpr int kPackBuckets = 64;          // length buckets of the partial partitions
constexpr size_t kPackHeaderBytes = 512;  // workspace header: full count + bucket bases

struct PackArgs {
  int32_t* block_tables;          // the step's table, or a pool of rows
  const int32_t* rows;            // row of each sequence in block_tables, or null (row = seq)
  const int32_t* updates;         // (row, col, block) triples applied first
  const int64_t* start_positions;
  const int64_t* new_token_counts;
  int32_t* step_block_tables;     // [B, step_table_width] copy of the rows, or null
  int32_t* step_rows;             // [B] the sequences' rows, or null
  int64_t* cu_seqlens;
  int64_t* cu_context_offsets;
  int32_t* context_lens;
  int64_t* scatter_slots;
  int64_t* position_ids;
  int64_t* gather_slots;
  int32_t* decode_items;
  int32_t* merge_items;
  int32_t* prefill_items;
  int32_t* ws_header;             // [0] full partitions, [1 + b] base of bucket b
  int4* ws_seq;                   // per sequence: (full, merge and prefill offsets, partial
                                  // rank), (start, count, table row, 0)
  int32_t num_seqs;
  int32_t num_table_rows;
  int32_t num_updates;
  int32_t step_table_width;
  int32_t fused;                  // the scan kernel writes every output (one launch)
  int32_t block_size;
  int32_t block_table_stride;
  int32_t partition;
  int32_t prefill_tile;
  int64_t max_query_tokens;
  int64_t max_context_tokens;
  int64_t max_decode_items;
  int64_t max_merge_items;
  int64_t max_prefill_items;
  uint4* clear;                   // 16-byte words zeroed by the scan kernel (the decode merge records)
  int64_t clear_words;
};

struct CacheWriteArgs {
  const void* key;
  const void* value;
  int64_t key_token_stride;
  int64_t key_head_stride;
  int64_t value_token_stride;
  int64_t value_head_stride;
  void* key_cache;    // base of the layer
  void* value_cache;  // base of the layer
  const int64_t* slot_mapping;
  int64_t num_slots;  // total_blocks * block_size
  int32_t num_tokens;
  int32_t num_kv_heads;
  int32_t head_dim;
};

// KV block copy (copy_blocks).
struct CopyBlocksArgs {
  const void* src;              // cache (L, N_src, bs, H_kv, D)
  void* dst;                    // cache (L, N_dst, bs, H_kv, D)
  const int64_t* block_mapping;  // [num_pairs, 2]: (src block, dst block)
  int64_t num_pairs;
  int64_t src_total_blocks;
  int64_t dst_total_blocks;
  int64_t block_bytes;          // bs * H_kv * D * element bytes
  int32_t num_layers;
};

// Causal chunked prefill over block tables (MFMA tiles).
struct PrefillArgs {
  const void* query;
  int64_t q_token_stride;
  int64_t q_head_stride;
  const void* key_cache;
  const void* value_cache;
  const int32_t* block_tables;
  const int32_t* rows;   // row of block_tables per sequence, or null (row = seq)
  int32_t num_table_rows;
  const int32_t* context_lens;
  const int64_t* cu_seqlens;
  const int32_t* items;  // (seq, query tile) pairs
  void* output;
  int32_t block_table_stride;
  int32_t num_kv_heads;
  int32_t total_blocks;
  int32_t log2_block_size;
  float scale_log2e;
  // Query heads per KV head and the workgroups that share them (1 unless
  // the group exceeds the largest kernel group; each serves group /
  // sub_groups heads and walks the context itself).
  int32_t group;
  int32_t sub_groups;
  // Work units of the launch (items x KV heads x sub-groups): the MFMA
  // prefill runs fewer workgroups than units, each looping over its share.
  int64_t num_units;
  // pa_prefill_append (null otherwise): the step's new K and V rows
  // ([T, H_kv, D], element strides).  Context positions at or after a
  // sequence's chunk start are read from them, and sub-group 0 of each
  // unit writes its own tile's rows into the (writable) caches.
  const void* new_key;
  const void* new_value;
  int64_t new_key_token_stride;
  int64_t new_key_head_stride;
  int64_t new_value_token_stride;
  int64_t new_value_head_stride;
};

bool decode_fast_path_supported(int dtype, int head_dim, int group, int block_size,
                                int partition);
// Largest query-head group the decode serves (split into sub-groups of at
// most 8 heads above 8).
constexpr int kMaxDecodeQueryGroup = 64;
// Workgroups sharing one KV head's query heads: the fewest equal sub-groups
// of at most 8 heads.
int decode_sub_groups(int group);
// Whether two adjacent KV heads of this shape run as one workgroup
// (DecodeArgs::pair; the KV head count must then be even).
bool decode_pairs_heads(int dtype, int head_dim, int num_kv_heads, int group);
// phases: PA_DECODE_PHASE_PARTITIONS and/or PA_DECODE_PHASE_MERGE.  head_dim
// and group are the real ones; a.num_kv_heads counts pairs when a.pair.
hipError_t launch_decode(const DecodeArgs& a, int dtype, int head_dim, int group,
                         int64_t num_items, int phases, hipStream_t stream);
// Resident partition workgroups per CU of the kernel launch_decode runs for
// a shape (the HIP occupancy calculator on the current device).
hipError_t decode_workgroups_per_cu(int dtype, int head_dim, int group, bool pair, int* per_cu);

bool generic_supported(int dtype, int head_dim);
hipError_t launch_generic(const GenericArgs& a, int dtype, bool masked, hipStream_t stream);

size_t pack_workspace_size(int64_t num_seqs);
// Whether one launch can pack the step: a single scan chunk, no gather or
// step table, and per-sequence work (new tokens, full partitions) bounded
// by the hints.
bool pack_fusable(const PackArgs& a, int32_t max_new_tokens, int32_t max_context);
hipError_t launch_pack(const PackArgs& a, hipStream_t stream);

hipError_t launch_cache_write(const CacheWriteArgs& a, int dtype, hipStream_t stream);
hipError_t launch_copy_blocks(const CopyBlocksArgs& a, bool vec16, hipStream_t stream);

bool prefill_fast_path_supported(int dtype, int head_dim, int group, int block_size);
// Whether the fast path of this shape also takes new rows (PrefillArgs::new_key).
bool prefill_append_supported(int dtype, int head_dim);
// Compute units of the current device (cached per device; 0 if unknown): the
// width of the persistent prefill launches.
int device_compute_units();
int prefill_tile_for(int group);
hipError_t launch_prefill(const PrefillArgs& a, int dtype, int head_dim, int group,
                          int64_t num_items, hipStream_t stream);
hipError_t launch_prefill256(const PrefillArgs& a, int dtype, int group, int64_t num_items, hipStream_t stream);
// fp32 caches: the fp32 MFMA kernel of prefill_f32.hip (same units and rows).
hipError_t launch_prefill_f32(const PrefillArgs& a, int head_dim, int group, int64_t num_items,
                              hipStream_t stream);

}  // namespace pa
