/*
 * paged_attention_amd.h -- C ABI of the MI355X (gfx950) paged-attention path.
 *
 * Every pointer argument is a DEVICE pointer (HBM) unless stated otherwise;
 * `stream` is a hipStream_t passed as void* (NULL = the null stream).  No
 * entry point allocates, frees or synchronises: outputs and workspaces are
 * caller-owned, every launch is asynchronous on `stream`, and the library
 * keeps no device-side state between calls (reentrant), apart from the
 * scratch array of pa_decode_no_alloc (see there).
 *
 * Entry points returning int return 0 (PA_OK) on success or a PA_ERR_* code;
 * pa_error_string() turns a code into text and pa_last_error_message()
 * returns the detailed message of the calling thread's last failure.
 *
 * Cache layout (fixed by the reference, app/memory/strategies.py:73-97):
 *   key_cache / value_cache : (num_layers, total_blocks, block_size,
 *                              num_kv_heads, head_dim), contiguous
 *   slot s of layer l, kv head h  ->  element
 *       ((l * total_blocks * block_size) + s) * num_kv_heads * head_dim
 *       + h * head_dim
 */
#ifndef PAGED_ATTENTION_AMD_H
#define PAGED_ATTENTION_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
    PA_OK = 0,
    PA_ERR_INVALID_ARGUMENT = 1, /* shape / stride / dtype rejected        */
    PA_ERR_UNSUPPORTED = 2,      /* valid but not implemented on this path */
    PA_ERR_WORKSPACE = 3,        /* workspace missing or too small         */
    PA_ERR_LAUNCH = 4            /* the HIP runtime refused a launch       */
};

/* Element type tags for K/V/query/output buffers. */
enum { PA_DTYPE_F32 = 0, PA_DTYPE_BF16 = 1, PA_DTYPE_F16 = 2 };

/* Default split-K partition of the decode kernel, in context tokens, and the
 * largest one its fast path takes (larger or non-multiple-of-32 partitions
 * run on the generic kernel). */
#define PA_DECODE_PARTITION 2048
#define PA_DECODE_MAX_PARTITION 4096

/* ---- (0) reference ABI, device pointers -------------------------------- */

/* Same fields, same order as the reference's PagedAttentionDims
 * (csrc/include/paged_kernels.h:11-20). */
typedef struct {
    int32_t num_query_heads;
    int32_t num_query_tokens;
    int32_t head_dim;
    int32_t num_layers;
    int32_t total_blocks;
    int32_t block_size;
    int32_t num_kv_heads;
    int32_t num_context_tokens;
} PagedAttentionDims;

/*
 * Replaces: paged_attention(), csrc/include/paged_kernels.h:22-34 and
 * csrc/src/paged_kernels.cpp:7-105 (bound by csrc/src/bindings.cpp:56-71).
 * Same signature and semantics, fp32, over device pointers:
 *   query  [1, H_q, T, D] head-major, caches as above (fp32),
 *   gather_slots int32 [C], attention_mask uint8 [T, C] (nonzero = attend),
 *   output [T, H_q, D]; a fully masked row and C == 0 give zeros.
 * `scratch` is accepted for ABI compatibility and not touched (may be NULL).
 * The reference returns void; so does this.  Failures are latched per
 * thread: read them with pa_last_error().
 */
void paged_attention(const float *query, const float *key_cache,
                     const float *value_cache, int32_t layer_idx,
                     PagedAttentionDims dims, const int32_t *gather_slots,
                     const uint8_t *attention_mask, float scaling,
                     float *output, float *scratch, void *stream);

/* Status of the calling thread's last paged_attention() call. */
int pa_last_error(void);

/* ---- shared step description ------------------------------------------ */

/*
 * One engine step over the flattened ragged batch (the layout of
 * app/model/paged_attention.py:37-118): B sequences, sequence i owns query
 * tokens [cu_seqlens[i], cu_seqlens[i+1]) of the flat buffer, its new tokens
 * sit at positions [start_i, start_i + count_i), and its context is
 * positions [0, context_lens[i]) with context_lens[i] = start_i + count_i.
 * The query token at position start_i + j attends context positions
 * [0, start_i + j] of its own sequence only (paged_attention.py:101-117).
 */
typedef struct {
    int32_t num_seqs;           /* B                                        */
    int32_t num_query_tokens;   /* T = sum of new-token counts              */
    int32_t num_query_heads;    /* H_q                                      */
    int32_t num_kv_heads;       /* H_kv (H_q % H_kv == 0)                   */
    int32_t head_dim;           /* D                                        */
    int32_t block_size;         /* bs, tokens per KV block                  */
    int32_t total_blocks;       /* N, blocks per layer in the pool          */
    int32_t num_layers;         /* L                                        */
    int32_t max_blocks_per_seq; /* row stride of block_tables (elements)    */
    int32_t partition_size;     /* decode split-K partition, tokens         */
    int32_t dtype;              /* PA_DTYPE_* of query, caches and output   */
    int32_t num_table_rows;     /* rows of block_tables (0: num_seqs)       */
    int64_t q_token_stride;     /* query element stride between tokens      */
    int64_t q_head_stride;      /* query element stride between heads       */
    /* Row of block_tables per sequence (int32 [num_seqs], device), or NULL:
     * row i is sequence i.  With it, block_tables can be a pool of rows kept
     * on the device across steps (pa_pack's table), read in place.  A row
     * outside [0, num_table_rows) reads as a sequence without blocks. */
    const int32_t *block_table_rows;
} PaStepDims;

/* ---- (a) ragged-batch packing ------------------------------------------ */

typedef struct {
    int32_t num_seqs;           /* B                                        */
    int32_t block_size;         /* bs                                       */
    int32_t max_blocks_per_seq; /* row stride of block_tables               */
    int32_t partition_size;     /* decode split-K partition, tokens         */
    int32_t prefill_tile;       /* query tokens per prefill work item       */
    int32_t num_table_rows;     /* rows of block_tables (0 = num_seqs)      */
    int32_t num_updates;        /* (row, col, block) triples in `updates`   */
    int32_t step_table_width;   /* columns of step_block_tables             */
    int32_t max_new_tokens;     /* hint: most new tokens of one sequence    */
    int32_t max_context;        /* hint: longest context (0: no hints)      */
    int64_t max_query_tokens;   /* capacity of scatter_slots / position_ids */
    int64_t max_context_tokens; /* capacity of gather_slots                 */
    int64_t max_decode_items;   /* capacity of decode_items (pairs)         */
    int64_t max_merge_items;    /* capacity of merge_items                  */
    int64_t max_prefill_items;  /* capacity of prefill_items (pairs)        */
} PaPackDims;

/* Bytes of workspace pa_pack needs for `num_seqs` sequences (a 512-byte
 * header + 32 bytes per sequence).  No counterpart in the reference. */
size_t pa_pack_workspace_size(int32_t num_seqs);

/*
 * Replaces, on the GPU: _cumulative_offsets (app/model/paged_attention.py:
 * 121-125), PagedKVCacheManager.build_slot_mapping / _sequence_slots
 * (app/memory/manager.py:104-128, 301-333) for both the scatter slots and
 * the gather slots (paged_attention.py:64-69), PagedStepContext.
 * position_ids (paged_attention.py:81-90), and build_block_tables
 * (manager.py:236-271) from a device-resident pool of table rows.
 *
 * block_tables: int32 [num_table_rows, max_blocks_per_seq], -1 padded.
 * With rows == NULL it is the step's own table (row i = sequence i); with
 * rows (int32 [B]) it is a pool of rows kept on the device across steps and
 * sequence i reads row rows[i] (a row outside the pool reads as all -1).
 * updates (int32 [num_updates, 3], may be NULL when num_updates is 0):
 * (row, col, block id) entries written into block_tables before anything
 * reads it (entries outside the table are skipped) -- how a host appends
 * the blocks it allocated since the last step.  The entries are stored in
 * no fixed order: each (row, col) may appear at most once (a host that
 * queued several values for one entry passes only the last).
 * start_positions / new_token_counts: int64 [B].
 * rows, updates, start_positions and new_token_counts are read once, by
 * the first launch, and may sit in pinned host memory (the device address
 * pa_map_host_memory gives): a host hands a step over without a copy.  The
 * first launch keeps a copy of the starts, counts and rows in the workspace:
 * with start_positions and new_token_counts both NULL, a call re-runs the
 * step the last call on this workspace described (rows then ignored), e.g.
 * from a captured HIP graph.
 * Positions and counts must stay below 2^31 (context_lens is int32).
 * Outputs (all int64 unless noted, bit-exact with the reference):
 *   step_block_tables int32 [B, step_table_width] (may be NULL): the rows
 *   of the step's sequences, -1 past max_blocks_per_seq;
 *   step_rows int32 [B] (may be NULL): the row of every sequence (rows[i],
 *   or i without rows) -- with it, the attention entry points read the
 *   pool in place (PaStepDims.block_table_rows) and no step table is built;
 *   cu_seqlens [B+1], cu_context_offsets [B+1], context_lens int32 [B],
 *   scatter_slots [T], position_ids [T], gather_slots [C] (may be NULL),
 *   decode_items int32 pairs (seq, partition) for every sequence with one
 *   new token: all full partitions first (by sequence, then partition),
 *   then the partial last partitions by decreasing length bucket (bucket =
 *   (length - 1) * 64 / partition_size; ties by sequence), so short work
 *   ends the launch (may be NULL),
 *   merge_items int32 [., 4]: (index in decode_items of the sequence's first
 *   full partition, number of full partitions, sequence, index of its
 *   partial partition or -1) for every single-token sequence whose context
 *   spans more than one partition, ordered by sequence (may be NULL;
 *   16-byte aligned),
 *   prefill_items int32 pairs (seq, query tile) for every sequence with more
 *   than one new token (may be NULL).
 * clear / clear_bytes (may be NULL / 0): a 16-byte aligned region of whole
 * 16-byte words the first launch sets to zero -- the merge records of the
 * step's decode workspace (pa_decode_merge_state_size), so the step needs
 * no separate memset.
 * Writes past a capacity in PaPackDims are dropped, never performed.
 * A block-table entry that is negative or past its row yields slot -1.
 * workspace: pa_pack_workspace_size(B) bytes, 16-byte aligned; calls that
 * share one must not overlap in time.  Two launches, each linear in B; one
 * launch when B <= 1024, neither gather_slots nor step_block_tables is
 * asked for, and the hints bound every sequence's new tokens and full
 * partitions by 32 (hints that understate only slow that launch down).
 */
int pa_pack(int32_t *block_tables, const int32_t *rows, const int32_t *updates,
            const int64_t *start_positions, const int64_t *new_token_counts,
            PaPackDims dims, int32_t *step_block_tables, int32_t *step_rows,
            int64_t *cu_seqlens,
            int64_t *cu_context_offsets, int32_t *context_lens,
            int64_t *scatter_slots, int64_t *position_ids,
            int64_t *gather_slots, int32_t *decode_items,
            int32_t *merge_items, int32_t *prefill_items, void *clear,
            size_t clear_bytes, void *workspace, size_t workspace_bytes,
            void *stream);

/* ---- host-side step planning ------------------------------------------- */

typedef struct {
    int32_t block_size;          /* bs                                       */
    int32_t prefill_tile;        /* query tokens per prefill work item       */
    int32_t partition_size;      /* > 0: use it; 0: choose (see below)       */
    int32_t num_kv_heads;        /* H_kv                                     */
    int32_t num_query_heads;     /* H_q (0: 4 x H_kv)                        */
    int32_t workgroups_per_item; /* decode launch width per item (0: H_kv)   */
    int32_t workgroups_per_cu;   /* resident decode workgroups per CU (0:
                                    5 for one query head per KV head, else 4) */
    int32_t compute_units;       /* CUs of the device (0: 256)               */
} PaPlanParams;

typedef struct {
    int64_t num_query_tokens;    /* T                                        */
    int64_t num_context_tokens;  /* C                                        */
    int64_t num_decode_items;    /* sizes of pa_pack's work lists            */
    int64_t num_merge_items;
    int64_t num_prefill_items;
    int64_t max_context;         /* longest context of the step              */
    int32_t num_decode_seqs;     /* sequences with one new token             */
    int32_t num_prefill_seqs;    /* sequences with more than one             */
    int32_t partition_size;      /* the split-K partition of the step        */
    int32_t max_blocks;          /* max over sequences of ceil(ctx / bs)     */
    int32_t bad_seq;             /* first sequence failing a check, or -1    */
    int32_t max_new_tokens;      /* most new tokens of one sequence          */
} PaStepPlan;

/*
 * Host code, no GPU call: sizes a step from the HOST arrays of its start
 * positions and new-token counts (int64 [num_seqs]) -- what pa_pack will
 * emit, so buffers are sized without reading the device -- and chooses the
 * decode split-K partition when params.partition_size is 0: the largest of
 * 4096 ... 256 tokens whose decode launch (items x workgroups_per_item)
 * gives every resident workgroup slot (compute_units x workgroups_per_cu)
 * one and a half workgroups; failing that (a latency-bound step) the one of
 * 64 ... 4096 with the least modelled time: the longest workgroup's read at
 * 0.049 us per token, slowed by its share of HBM when more than 310
 * workgroups run at once and multiplied by the waves of workgroups, plus
 * 2 us per batch of 8 split-K partials of the longest sequence (ties to
 * the shorter partition; 64 for a step without decodes).
 * allocated_tokens (int64 [num_seqs], may be NULL): tokens each sequence has
 * slots for; a sequence with start + count above it, or a negative start or
 * count, fails the call with PA_ERR_INVALID_ARGUMENT and plan->bad_seq set
 * (the checks of app/memory/manager.py:104-128, 301-315).
 * No counterpart in the reference (whose step has no work lists).
 */
int pa_plan_step(const int64_t *start_positions, const int64_t *new_token_counts,
                 const int64_t *allocated_tokens, int32_t num_seqs,
                 PaPlanParams params, PaStepPlan *plan);

/* ---- (b) K/V cache write ------------------------------------------------ */

/*
 * Replaces: PagedKVCacheManager.scatter_layer_kv (app/memory/manager.py:
 * 150-168), i.e. key_cache[layer].view(N*bs, H_kv, D)[slot_mapping] = key,
 * and the same for value, called from paged_attention.py:152-154.
 * key / value: [num_tokens, H_kv, D] with arbitrary token / head strides
 * (elements) and unit stride along D, so the model's transposed
 * [1, H_kv, T, D] projections are consumed without a copy.
 * slot_mapping int64 [num_tokens].  Slots outside [0, N*bs) are skipped
 * (never written).  A bit-exact copy: no arithmetic on the values.
 */
int pa_reshape_and_cache(const void *key, const void *value,
                         int64_t key_token_stride, int64_t key_head_stride,
                         int64_t value_token_stride, int64_t value_head_stride,
                         void *key_cache, void *value_cache,
                         const int64_t *slot_mapping, int32_t num_tokens,
                         int32_t num_kv_heads, int32_t head_dim,
                         int32_t block_size, int32_t total_blocks,
                         int32_t num_layers, int32_t layer_idx, int32_t dtype,
                         void *stream);

/*
 * Replaces: KVCacheMemoryStrategy.copy_blocks (app/memory/strategies.py:
 * 50-56; CPU 88-90, CUDA 117-122: one torch copy per block).  For every
 * (src block, dst block) pair of block_mapping (int64 [num_pairs, 2]) and
 * every layer, copies the block (block_bytes = bs * H_kv * D * element
 * bytes) of src_cache (L, src_total_blocks, bs, H_kv, D) into dst_cache
 * (L, dst_total_blocks, bs, H_kv, D); call once for the keys and once for
 * the values.  Both caches must be device-accessible; pairs with an index
 * outside its cache are skipped.  When the two caches are one, no pair's
 * destination may be another pair's source.  (The reference indexes
 * dim 0 of its caches with the block id, which selects a layer; this copies
 * the named physical block of every layer.)
 */
int pa_copy_blocks(const void *src_cache, void *dst_cache,
                   const int64_t *block_mapping, int64_t num_pairs,
                   int32_t num_layers, int64_t src_total_blocks,
                   int64_t dst_total_blocks, int64_t block_bytes,
                   void *stream);

/* Directions of pa_swap_blocks. */
enum { PA_SWAP_OUT = 0, PA_SWAP_IN = 1 };

/*
 * Replaces: the data movement behind PageAllocator::swap_out / swap_in
 * (csrc/include/page_allocator.hpp:179-247), which only keeps the
 * bookkeeping, and KVCacheMemoryStrategy.copy_blocks (app/memory/
 * strategies.py:50-56, 117-122).  Copies blocks between a device cache
 * (L, device_total_blocks, bs, H_kv, D) in HBM and a host pool of the same
 * block shape (L, host_total_blocks, bs, H_kv, D) in pinned host memory
 * (hipHostMalloc'd, e.g. a torch pin_memory tensor), every layer, in one
 * launch: PA_SWAP_OUT copies device block -> host block for each (device
 * block, host block) pair of block_mapping, PA_SWAP_IN host block -> device
 * block for each (host block, device block) pair.  block_mapping: int64
 * [num_pairs, 2] in device memory; pairs outside a cache are skipped.
 * host_cache is a HOST pointer: the library maps it with
 * hipHostGetDevicePointer and refuses memory that is not pinned host
 * memory (PA_ERR_INVALID_ARGUMENT).  Call once for the keys and once for
 * the values; the copy is asynchronous on `stream` (the host pool is only
 * complete, or free to reuse, once the stream reaches that point).
 */
int pa_swap_blocks(void *device_cache, void *host_cache,
                   const int64_t *block_mapping, int64_t num_pairs,
                   int32_t num_layers, int64_t device_total_blocks,
                   int64_t host_total_blocks, int64_t block_bytes,
                   int32_t direction, void *stream);

/* ---- (c) paged-attention decode (split-K) ------------------------------ */

/* Bytes of workspace pa_decode needs for `num_decode_items` work items: the
 * split-K partials, then the merge records (pa_decode_merge_state_size
 * bytes at the end of the workspace).  Calls that share a workspace must
 * not overlap in time. */
size_t pa_decode_workspace_size(PaStepDims dims, int64_t num_decode_items);

/* Bytes of merge records at the end of a pa_decode workspace of this size
 * (8 per sequence and decode workgroup of an item; 0 when the workspace is
 * 0).  They must be zero when a workspace is first used -- pa_pack clears
 * them when passed as its `clear` region -- and every pa_decode call leaves
 * them zero.  The rest of the workspace needs no initial value.  (No
 * counterpart in the reference.) */
size_t pa_decode_merge_state_size(PaStepDims dims, int64_t num_decode_items);

/* Partition workgroups pa_decode launches per decode work item:
 *  - num_kv_heads / 2 when two adjacent KV heads run as one workgroup
 *    (bf16 or fp16, an even KV head count, head_dim 64 or 128 and groups of up to 4
 *    query heads: each token's rows of the two heads are read as one row of
 *    twice the length);
 *  - num_kv_heads x the sub-groups of a group of more than 8 query heads
 *    (the fewest equal sub-groups of at most 8; each reads the K/V again,
 *    ordered so that the re-reads of one KV head's rows meet one L2);
 *  - num_kv_heads otherwise; 0 for head counts pa_decode rejects.
 * A host choosing the split-K partition size from the launch width uses it.
 * (No counterpart in the reference, whose CPU kernel has no workgroups.) */
int32_t pa_decode_workgroups_per_item(int32_t dtype, int32_t head_dim,
                                      int32_t num_kv_heads, int32_t num_query_heads);

/* Query tokens per pa_prefill work item (the `prefill_tile` given to pa_pack
 * and pa_prefill) that the MFMA prefill kernel takes for these head counts:
 * 128 query rows over the query heads of one workgroup, i.e. 128 / group,
 * or 128 / (sub-group) for groups above 8; 0 for bad head counts.  Another
 * tile is still correct but runs the generic kernel.  (No counterpart in
 * the reference.) */
int32_t pa_prefill_tile(int32_t num_query_heads, int32_t num_kv_heads);

/* Decode workgroups of this shape that one compute unit of the current
 * device holds at once (the HIP occupancy calculator on the kernel pa_decode
 * launches for it), or 0 for a shape without a tuned kernel or on a HIP
 * error (pa_last_error_message then says which).  With the CU count it gives
 * the resident width a host's split-K partition choice aims to fill.  (No
 * counterpart in the reference.) */
int32_t pa_decode_workgroups_per_cu(int32_t dtype, int32_t head_dim,
                                    int32_t num_kv_heads, int32_t num_query_heads);

/*
 * Replaces: NativePagedBackend.attend for decode steps
 * (app/model/attention_backends.py:88-117) and the paged_attention kernel
 * it calls, over block tables instead of a dense mask.
 * Runs every (sequence, partition) item of `decode_items` (from pa_pack) for
 * every KV head in one launch; the split-K partials of a multi-partition
 * sequence are combined in the same launch by whichever of its partition
 * workgroups finishes last (counted in the workspace's merge records), or,
 * for a step of 65535 or more items, by a second launch.
 * decode_items must list each partition of a sequence once, its full
 * partitions as consecutive items (as pa_pack writes them).  merge_items
 * (from pa_pack) serve the separate merge phase; they may be NULL only when
 * num_merge_items is 0.  The single query token
 * of decode sequence i is flat token cu_seqlens[i]; it attends positions
 * [0, context_lens[i]).  query: [T, H_q, D] through PaStepDims strides;
 * output: [T, H_q, D] contiguous, dtype of the caches; rows of tokens that
 * are not decode tokens are not written.  Tuned kernels serve head_dim 64,
 * 80, 96 and 128 (every dtype) and 256 (bf16, fp16) with groups of up to
 * 64 query heads, power-of-two block sizes and partitions that are
 * multiples of 32 up to 4096; other shapes run a generic kernel with the
 * same results.
 */
int pa_decode(const void *query, const void *key_cache,
              const void *value_cache, int32_t layer_idx, PaStepDims dims,
              const int32_t *block_tables, const int32_t *context_lens,
              const int64_t *cu_seqlens, const int32_t *decode_items,
              int64_t num_decode_items, const int32_t *merge_items,
              int64_t num_merge_items, float scaling, void *output,
              void *workspace, size_t workspace_bytes, void *stream);

/* Phases of pa_decode, for callers that launch them separately. */
enum { PA_DECODE_PHASE_PARTITIONS = 1, PA_DECODE_PHASE_MERGE = 2 };

/*
 * pa_decode's two phases (same arguments and rules).  The partition phase
 * writes the final rows of single-partition sequences and the split-K
 * partials of the others into `workspace`, and merges those partials in the
 * same launch; the merge phase alone runs the merge kernel over merge_items,
 * which combines the partials the last partition phase left (a no-op when
 * every sequence fits one partition or the step runs on the generic
 * kernel).  Both merges run the same arithmetic: pa_decode(...) equals
 * pa_decode_phases(PA_DECODE_PHASE_PARTITIONS | PA_DECODE_PHASE_MERGE, ...),
 * which launches the partition kernel only, and a partition call followed
 * by a merge call on one stream gives the same bits.  No reference
 * counterpart: the reference's decode is one CPU call.
 */
int pa_decode_phases(int32_t phases, const void *query, const void *key_cache,
                     const void *value_cache, int32_t layer_idx, PaStepDims dims,
                     const int32_t *block_tables, const int32_t *context_lens,
                     const int64_t *cu_seqlens, const int32_t *decode_items,
                     int64_t num_decode_items, const int32_t *merge_items,
                     int64_t num_merge_items, float scaling, void *output,
                     void *workspace, size_t workspace_bytes, void *stream);

/* The step's new K and V rows ([T, H_kv, head_dim], any token / head element
 * strides, unit stride along head_dim), as pa_reshape_and_cache takes them. */
typedef struct {
    const void *key;
    const void *value;
    int64_t key_token_stride;
    int64_t key_head_stride;
    int64_t value_token_stride;
    int64_t value_head_stride;
} PaNewRows;

/*
 * Replaces, for the single-token sequences of a step:
 * scatter_layer_kv (app/memory/manager.py:150-168, called at
 * app/model/paged_attention.py:152-154) followed by the decode attention
 * (attention_backends.py:88-117) -- pa_reshape_and_cache + pa_decode in the
 * decode launches.  The workgroups that attend a sequence's last partition
 * first write its new K and V rows into the cache at the slot its block
 * table gives position context_len - 1 (bit-exact, as pa_reshape_and_cache
 * writes them; an out-of-pool block id writes nothing), then attend; no
 * other workgroup reads that position.  Rows of sequences with more than
 * one new token are NOT written: for a step with prefill tokens,
 * pa_prefill_append writes those (or pa_reshape_and_cache writes every
 * row first).  Arguments as pa_decode, with writable caches.
 * PA_ERR_UNSUPPORTED (nothing launched) for a shape or alignment the fused
 * path does not take (16-byte aligned rows and strides, the tuned decode's
 * shapes): the caller then writes with pa_reshape_and_cache and calls
 * pa_decode.
 */
int pa_decode_append(const void *query, void *key_cache, void *value_cache,
                     int32_t layer_idx, PaStepDims dims, PaNewRows new_rows,
                     const int32_t *block_tables, const int32_t *context_lens,
                     const int64_t *cu_seqlens, const int32_t *decode_items,
                     int64_t num_decode_items, const int32_t *merge_items,
                     int64_t num_merge_items, float scaling, void *output,
                     void *workspace, size_t workspace_bytes, void *stream);

/* Bytes of the file-scope device array behind pa_decode_no_alloc (64 MiB:
 * the split-K partials of about 4000 decode work items of 32 query heads of
 * 128 -- pa_decode_workspace_size less pa_decode_merge_state_size gives the
 * need of a step -- in the first 63 MiB, and the merge records in the last
 * PA_DECODE_SCRATCH_STATE_BYTES). */
#define PA_DECODE_SCRATCH_BYTES ((size_t)64 << 20)
#define PA_DECODE_SCRATCH_STATE_BYTES ((size_t)1 << 20)

/*
 * No counterpart in the reference: pa_decode for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * pa_decode without the workspace: the split-K partials go into a
 * file-scope device array of PA_DECODE_SCRATCH_BYTES that each device the
 * library runs on holds from its first use until the process ends.  The
 * first call on a device (with that device current) looks up the array's
 * address with hipGetSymbolAddress; no call allocates or frees anything.
 * A step whose partials exceed the first PA_DECODE_SCRATCH_BYTES -
 * PA_DECODE_SCRATCH_STATE_BYTES bytes of the array is rejected with
 * PA_ERR_WORKSPACE and nothing is launched.  The array keeps the last call's
 * contents.  Its partials need no initial value (the partition phase writes
 * every partial a merge reads); its merge records sit at a fixed place, the
 * last PA_DECODE_SCRATCH_STATE_BYTES, which hold zeros from the load of the
 * code object on and which every call leaves zero.  A step with more
 * records than that region holds merges in a second launch instead.  Every
 * call on one device shares that device's array, so calls that overlap in
 * time on one device (two streams, two threads) race; serialise them on
 * one stream.
 */
int pa_decode_no_alloc(const void *query, const void *key_cache,
                       const void *value_cache, int32_t layer_idx,
                       PaStepDims dims, const int32_t *block_tables,
                       const int32_t *context_lens, const int64_t *cu_seqlens,
                       const int32_t *decode_items, int64_t num_decode_items,
                       const int32_t *merge_items, int64_t num_merge_items,
                       float scaling, void *output, void *stream);

/* ---- (d) causal chunked prefill ----------------------------------------- */

/*
 * Replaces: the SDPA path for multi-token steps (paged_attention.py:165-180,
 * attention_backends.py:55-78) over the block-diagonal causal mask.
 * Runs every (sequence, query tile) item of `prefill_items` (from pa_pack):
 * query token j of sequence i (flat index cu_seqlens[i] + j, position
 * context_lens[i] - count_i + j) attends positions [0, that position].
 * K/V are read from the paged cache, so the new tokens must already have
 * been written with pa_reshape_and_cache.  A launch takes at most 2^30
 * (item, KV head, query-head sub-group) units (PA_ERR_LAUNCH beyond).
 */
int pa_prefill(const void *query, const void *key_cache,
               const void *value_cache, int32_t layer_idx, PaStepDims dims,
               const int32_t *block_tables, const int32_t *context_lens,
               const int64_t *cu_seqlens, const int32_t *prefill_items,
               int64_t num_prefill_items, int32_t prefill_tile, float scaling,
               void *output, void *stream);

/*
 * Replaces, for the multi-token sequences of a step: scatter_layer_kv
 * (app/memory/manager.py:150-168, called at app/model/paged_attention.py:
 * 152-154) followed by the prefill attention (paged_attention.py:165-180)
 * -- pa_reshape_and_cache of those sequences' rows + pa_prefill in one
 * launch.  Each (item, KV head) unit of query-head sub-group 0 writes the
 * rows of its own tile's tokens for its KV head into the cache at the slots
 * their block table gives (bit-exact, as pa_reshape_and_cache writes them;
 * a position without a table column or in a block outside the pool writes
 * nothing), and every unit reads the positions at or after its sequence's
 * chunk start (context_len - count) from new_rows rather than the cache,
 * so no unit reads a row that another one writes.  The rows of the other
 * sequences of the step (single-token ones: pa_decode_append writes those)
 * are NOT written, nor those of tokens whose tiles are not in
 * prefill_items.  A slot is assumed to be written by at most one position
 * of the step and read by no other sequence of it (the allocator's
 * copy-on-write keeps shared blocks full and read-only).  Arguments as
 * pa_prefill, with writable caches.  PA_ERR_UNSUPPORTED (nothing launched)
 * for a shape the fused path does not take (heads of 256, the generic
 * kernel's shapes, rows or strides that are not 16-byte multiples, token
 * strides of 16 MiB or more): the caller then writes with
 * pa_reshape_and_cache and calls pa_prefill.
 */
int pa_prefill_append(const void *query, void *key_cache, void *value_cache,
                      int32_t layer_idx, PaStepDims dims, PaNewRows new_rows,
                      const int32_t *block_tables, const int32_t *context_lens,
                      const int64_t *cu_seqlens, const int32_t *prefill_items,
                      int64_t num_prefill_items, int32_t prefill_tile,
                      float scaling, void *output, void *stream);

/* ---- utilities ------------------------------------------------------------ */

/* The device address of pinned host memory (hipHostMalloc'd, e.g. a torch
 * pin_memory tensor), for passing host-resident inputs to pa_pack, or
 * PA_ERR_INVALID_ARGUMENT for memory that is not pinned.  No counterpart in
 * the reference. */
int pa_map_host_memory(const void *host_ptr, void **device_ptr);

/* Measurement aid, no counterpart in the reference: `workgroups` x 8 waves
 * each run `iters` x 2 independent bf16 32x32x16 MFMAs on register operands,
 * with `valu_per_mfma` (0, 4, 8 or 16) independent fp32 FMAs after each, and
 * write one float per lane to `out` (workgroups x 512 floats, device).
 * Timing the launch gives the matrix-core rate the device sustains (0) and
 * how much vector work it overlaps with it; pa_calibrate_mfma_flops gives
 * the MFMA flops of such a launch. */
int pa_calibrate_mfma(float *out, int32_t workgroups, int32_t iters, int32_t valu_per_mfma,
                      void *stream);
int64_t pa_calibrate_mfma_flops(int32_t workgroups, int32_t iters);

/* Measurement aid, no counterpart in the reference: `workgroups` x 256
 * threads read `bytes` (a multiple of 16) of device memory at `data` once,
 * with 16-byte non-temporal loads.  `out` (16 bytes, device) is written only
 * when the XOR of everything read equals 0x9e3779b9.  Timing the launch
 * gives the read rate the device sustains, against which an HBM-bound
 * kernel's rate can be read besides the nominal peak. */
int pa_calibrate_read(const void *data, int64_t bytes, void *out, int32_t workgroups, void *stream);

const char *pa_error_string(int code);
const char *pa_last_error_message(void);
/* ABI version: bumped whenever a signature or a struct above changes. */
int pa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PAGED_ATTENTION_AMD_H */
