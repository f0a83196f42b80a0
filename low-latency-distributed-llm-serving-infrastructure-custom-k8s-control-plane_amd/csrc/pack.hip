// Ragged-batch packing on the GPU, in two launches that are linear in the
// batch (one for a small decode step, below):
//
//   pack_scan_kernel   one workgroup of 1024 threads.  Applies the queued
//                      block-table updates, then walks the sequences in
//                      chunks of 1024 with block-wide exclusive scans:
//                      cu_seqlens, cu_context_offsets, context_lens, and per
//                      sequence (into the workspace) the offsets of its
//                      full decode partitions, merge entry and prefill tiles,
//                      the rank of its partial partition, and its start,
//                      count and table row.  It is the only reader of the
//                      step's host inputs, which may sit in pinned host
//                      memory (read once, over PCIe, with no copy launch).
//   pack_fill_kernel   one workgroup per sequence.  Copies the sequence's
//                      block-table row into the step table, writes its
//                      scatter slots, positions, gather slots and work items
//                      at the offsets the scan left.
//
// A small step (one chunk of sequences, no gather slots or step table, and
// little work per sequence: a decode batch) is packed in ONE launch: the
// scan kernel keeps each thread's sequence in registers and, once the bucket
// bases are known, every thread fills its own sequence.  The two launches
// would cost a second dispatch on the step's critical path.
//
// Reference semantics (all int64, bit-exact):
//   cu_seqlens / cu_context_offsets: exclusive prefix sums over the new-token
//     counts and over context_len = start + count
//     (app/model/paged_attention.py:57-62, 121-125);
//   slot of position p of a sequence = block_table[p // bs] * bs + p % bs,
//     concatenated in sequence order (app/memory/manager.py:104-128,
//     301-333), for the new tokens (scatter) and for the whole context
//     (gather, paged_attention.py:64-69);
//   position_ids restart at every sequence: start .. start+count-1
//     (paged_attention.py:81-90).
//
// Work lists of the attention kernels (no reference counterpart): decode
// items (seq, partition) for sequences with exactly one new token -- every
// full partition first (by sequence), then the partial last partitions in
// decreasing length bucket (bucket = (length - 1) * 64 / partition, ties by
// sequence) so short work ends the launch; the merge list (first full item,
// number of full partitions, sequence, item of the partial one or -1) of
// every such sequence with more than one partition, by sequence; prefill
// items (seq, query tile) for the multi-token sequences, by sequence.
//
// The partial-partition rank is a stable counting sort over the 64 buckets:
// within a chunk, each wave finds every lane's bucket-mates with six ballots
// (one per bucket bit), ranks it among them with mbcnt and counts each
// bucket, the 16 waves' counts are scanned per bucket, and a per-bucket carry
// crosses the chunks; bucket bases (largest bucket first) follow once every
// chunk is counted.  In-chunk sums are 32-bit: a step's context tokens stay
// below 2^31 (pa_plan_step checks it).
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kScanThreads = 1024;
constexpr int kScanWaves = kScanThreads / kWave;
constexpr int kFillThreads = 256;
// Per-sequence work (new tokens, full partitions) one thread of the fused
// launch takes on.
constexpr int kFusedMaxWork = 32;

__device__ __forceinline__ int64_t nonneg(int64_t v) { return v < 0 ? 0 : v; }

// Five per-sequence counts scanned together (one shuffle chain, one pair of
// barriers for all five).
struct Counts {
  int32_t tok, ctx, full, merge, tiles;
};

__device__ __forceinline__ Counts add(Counts x, Counts y) {
  return {x.tok + y.tok, x.ctx + y.ctx, x.full + y.full, x.merge + y.merge, x.tiles + y.tiles};
}

// Inclusive scan over the 64 lanes of a wave with DPP moves, no LDS: sums
// within rows of 16 lanes (row_shr 1, 2, 4, 8; lanes without a source add
// 0), then the last lane of row 0 and of row 2 into rows 1 and 3
// (row_bcast:15) and the last lane of row 1 into rows 2 and 3
// (row_bcast:31).
template <int Ctrl, int RowMask>
__device__ __forceinline__ int32_t dpp_in(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, Ctrl, RowMask, 0xF, false);
}

__device__ __forceinline__ int32_t wave_inclusive_sum(int32_t v) {
  v += dpp_in<0x111, 0xF>(v);  // row_shr:1
  v += dpp_in<0x112, 0xF>(v);  // row_shr:2
  v += dpp_in<0x114, 0xF>(v);  // row_shr:4
  v += dpp_in<0x118, 0xF>(v);  // row_shr:8
  v += dpp_in<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_in<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

__device__ __forceinline__ Counts wave_inclusive_sum(Counts v) {
  return {wave_inclusive_sum(v.tok), wave_inclusive_sum(v.ctx), wave_inclusive_sum(v.full),
          wave_inclusive_sum(v.merge), wave_inclusive_sum(v.tiles)};
}

// A workgroup barrier that orders LDS only: the scan kernel never reads back
// its global stores, so they are not waited for at every chunk.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct SeqInput {
  uint32_t start, count;
  int32_t row;
};

// Sequence `seq`'s start, count and table row: from the caller's inputs, or
// without them, from the copies the previous call left in the workspace.
__device__ __forceinline__ SeqInput load_input(const PackArgs& a, int seq) {
  SeqInput in{0u, 0u, -1};
  if (seq >= a.num_seqs) return in;
  if (a.start_positions != nullptr) {
    // Positions and counts are below 2^31 (context_lens is int32).
    in.start = static_cast<uint32_t>(nonneg(a.start_positions[seq]));
    in.count = static_cast<uint32_t>(nonneg(a.new_token_counts[seq]));
    in.row = a.rows != nullptr ? a.rows[seq] : seq;
  } else {
    const int4 w = a.ws_seq[2 * seq + 1];
    in.start = static_cast<uint32_t>(w.x);
    in.count = static_cast<uint32_t>(w.y);
    in.row = w.z;
  }
  return in;
}

// One sequence's scatter slots, positions, gather slots and work items, at
// the offsets the scan found (e: full, merge and prefill offsets and the
// partial partition's rank in its bucket; in: start, count, table row; tok,
// ctx: its first query and context token; bases: the buckets' first item).
// `stride` threads share the loops, thread `first` of them calling.
__device__ __forceinline__ void fill_sequence(const PackArgs& a, int seq, int4 e, int4 in, int64_t tok,
                                              int64_t ctx, const int32_t* bases, int first, int stride) {
  const int64_t start = in.x;
  const int64_t count = in.y;
  const int64_t clen = start + count;
  const int32_t row = in.z;
  const int32_t* bt = row >= 0 && row < a.num_table_rows
                          ? a.block_tables + static_cast<int64_t>(row) * a.block_table_stride
                          : nullptr;
  const int64_t stride_bt = bt != nullptr ? a.block_table_stride : 0;
  const int64_t bs = a.block_size;

  // The sequence's row of the step's own block table (-1 past its row).
  if (a.step_block_tables != nullptr) {
    int32_t* out = a.step_block_tables + static_cast<int64_t>(seq) * a.step_table_width;
    for (int j = first; j < a.step_table_width; j += stride) out[j] = j < stride_bt ? bt[j] : -1;
  }

  // New tokens: scatter slots + positions.
  for (int64_t j = first; j < count; j += stride) {
    const int64_t idx = tok + j;
    if (idx >= a.max_query_tokens) break;
    const int64_t p = start + j;
    const int64_t col = p / bs;
    int64_t slot = -1;
    if (col < stride_bt) {
      const int32_t b = bt[col];
      if (b >= 0) slot = static_cast<int64_t>(b) * bs + (p - col * bs);
    }
    a.scatter_slots[idx] = slot;
    a.position_ids[idx] = p;
  }

  // Whole context: gather slots.
  if (a.gather_slots != nullptr) {
    for (int64_t c = first; c < clen; c += stride) {
      const int64_t idx = ctx + c;
      if (idx >= a.max_context_tokens) break;
      const int64_t col = c / bs;
      int64_t slot = -1;
      if (col < stride_bt) {
        const int32_t b = bt[col];
        if (b >= 0) slot = static_cast<int64_t>(b) * bs + (c - col * bs);
      }
      a.gather_slots[idx] = slot;
    }
  }

  // Attention work lists.
  const int64_t P = a.partition;
  const int64_t nfull = count == 1 ? clen / P : 0;
  const int64_t rem_idx = e.w >= 0 ? static_cast<int64_t>(bases[((clen % P - 1) * kPackBuckets) / P]) + e.w : -1;
  if (count == 1 && a.merge_items != nullptr && first == 0 && e.y < a.max_merge_items &&
      nfull + (rem_idx >= 0 ? 1 : 0) > 1) {
    int4 m;
    m.x = e.x;
    m.y = static_cast<int32_t>(nfull);
    m.z = seq;
    m.w = static_cast<int32_t>(rem_idx);
    reinterpret_cast<int4*>(a.merge_items)[e.y] = m;
  }
  if (count == 1 && a.decode_items != nullptr) {
    for (int64_t p = first; p < nfull; p += stride) {
      const int64_t idx = e.x + p;
      if (idx >= a.max_decode_items) break;
      a.decode_items[2 * idx] = seq;
      a.decode_items[2 * idx + 1] = static_cast<int32_t>(p);
    }
    if (first == 0 && rem_idx >= 0 && rem_idx < a.max_decode_items) {
      a.decode_items[2 * rem_idx] = seq;
      a.decode_items[2 * rem_idx + 1] = static_cast<int32_t>(nfull);
    }
  } else if (count > 1 && a.prefill_items != nullptr) {
    const int64_t ntiles = (count + a.prefill_tile - 1) / a.prefill_tile;
    for (int64_t q = first; q < ntiles; q += stride) {
      const int64_t idx = e.z + q;
      if (idx >= a.max_prefill_items) break;
      a.prefill_items[2 * idx] = seq;
      a.prefill_items[2 * idx + 1] = static_cast<int32_t>(q);
    }
  }
}

template <bool kFused>
__global__ __launch_bounds__(kScanThreads) void pack_scan_kernel(PackArgs a) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  // The first chunk's inputs are loaded before the updates are applied (both
  // may come over PCIe from pinned host memory: the two round trips overlap;
  // the compiler would not move these loads above the updates' stores).
  SeqInput next = load_input(a, tid);
  // Queued block-table updates land before anything reads the table (the
  // fill kernel runs after this launch on the same stream; the fused fill
  // after a barrier).
  for (int u = tid; u < a.num_updates; u += kScanThreads) {
    const int32_t row = a.updates[3 * u];
    const int32_t col = a.updates[3 * u + 1];
    if (row >= 0 && row < a.num_table_rows && col >= 0 && col < a.block_table_stride)
      a.block_tables[static_cast<int64_t>(row) * a.block_table_stride + col] = a.updates[3 * u + 2];
  }
  // The region the step's later launches need zeroed (the decode's merge
  // records); nothing in this launch reads it.
  for (int64_t w = tid; w < a.clear_words; w += kScanThreads) a.clear[w] = make_uint4(0, 0, 0, 0);

  __shared__ Counts s_wave[kScanWaves];
  __shared__ int32_t s_bucket_wave[kScanWaves][kPackBuckets];  // per-chunk counts, then offsets
  __shared__ int32_t s_bucket_carry[kPackBuckets];
  __shared__ int32_t s_bases[kFused ? kPackBuckets : 1];
  if (tid < kPackBuckets) s_bucket_carry[tid] = 0;
  if (tid == 0) {
    a.cu_seqlens[0] = 0;
    a.cu_context_offsets[0] = 0;
  }

  const uint32_t P = static_cast<uint32_t>(a.partition);
  // Partitions are powers of two in practice: shifts instead of divisions.
  const int log2_p = (P & (P - 1)) == 0 ? __builtin_ctz(P) : -1;
  int64_t tok_carry = 0, ctx_carry = 0;
  int32_t full_carry = 0, merge_carry = 0, tiles_carry = 0;
  // One chunk when fused: the thread's sequence, kept for the fill below.
  int4 f_e = {0, 0, 0, -1}, f_in = {0, 0, -1, 0};
  int64_t f_tok = 0, f_ctx = 0;
  for (int base = 0; base < a.num_seqs; base += kScanThreads) {
    const int seq = base + tid;
    const bool valid = seq < a.num_seqs;
    const SeqInput cur = next;
    // The next chunk's loads are in flight while this chunk is scanned.
    next = load_input(a, seq + kScanThreads);
    const uint32_t start = cur.start, count = cur.count;
    const int32_t row = cur.row;
    const uint32_t clen = start + count;
    const uint32_t nfull = count == 1 ? (log2_p >= 0 ? clen >> log2_p : clen / P) : 0u;
    const uint32_t rlen = count == 1 ? clen - nfull * P : 0u;
    Counts v;
    v.tok = static_cast<int32_t>(count);
    v.ctx = static_cast<int32_t>(clen);
    v.full = static_cast<int32_t>(nfull);
    v.merge = count == 1 && nfull + (rlen > 0 ? 1u : 0u) > 1u ? 1 : 0;
    v.tiles = count > 1 ? static_cast<int32_t>((count + a.prefill_tile - 1) / a.prefill_tile) : 0;
    const int bucket = rlen == 0 ? -1
                       : static_cast<int>(log2_p >= 0 ? ((rlen - 1) * kPackBuckets) >> log2_p
                                                      : ((rlen - 1) * kPackBuckets) / P);

    // Exclusive scan of the five counts across the chunk.
    const Counts inc = wave_inclusive_sum(v);
    if (lane == kWave - 1) s_wave[wave] = inc;
    // Stable rank among this wave's lanes of the same bucket: the lanes
    // sharing a lane's bucket are the AND, over the bucket's 6 bits, of the
    // ballot of that bit (or of its complement where the lane's bit is 0);
    // mbcnt counts the lower ones.  The first lane of each bucket records the
    // wave's count of it.
    const uint64_t with_rem = __ballot(bucket >= 0);
    uint32_t same_lo = static_cast<uint32_t>(with_rem), same_hi = static_cast<uint32_t>(with_rem >> 32);
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const bool bit = bucket >= 0 && ((bucket >> k) & 1);
      const uint64_t ones = __ballot(bit);
      same_lo &= bit ? static_cast<uint32_t>(ones) : ~static_cast<uint32_t>(ones);
      same_hi &= bit ? static_cast<uint32_t>(ones >> 32) : ~static_cast<uint32_t>(ones >> 32);
    }
    const int wave_rank = __builtin_amdgcn_mbcnt_hi(same_hi, __builtin_amdgcn_mbcnt_lo(same_lo, 0));
    s_bucket_wave[wave][lane] = 0;  // LDS stores of one wave land in program order
    if (bucket >= 0 && wave_rank == 0) s_bucket_wave[wave][bucket] = __popc(same_lo) + __popc(same_hi);
    lds_barrier();
    // Every wave scans the 16 wave totals in its first 16 lanes and picks
    // its own prefix and the chunk total.
    const Counts wt = wave_inclusive_sum(lane < kScanWaves ? s_wave[lane] : Counts{0, 0, 0, 0, 0});
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    const Counts total = {__builtin_amdgcn_readlane(wt.tok, kScanWaves - 1),
                          __builtin_amdgcn_readlane(wt.ctx, kScanWaves - 1),
                          __builtin_amdgcn_readlane(wt.full, kScanWaves - 1),
                          __builtin_amdgcn_readlane(wt.merge, kScanWaves - 1),
                          __builtin_amdgcn_readlane(wt.tiles, kScanWaves - 1)};
    Counts before = {0, 0, 0, 0, 0};
    if (wave_s > 0)
      before = {__builtin_amdgcn_readlane(wt.tok, wave_s - 1), __builtin_amdgcn_readlane(wt.ctx, wave_s - 1),
                __builtin_amdgcn_readlane(wt.full, wave_s - 1), __builtin_amdgcn_readlane(wt.merge, wave_s - 1),
                __builtin_amdgcn_readlane(wt.tiles, wave_s - 1)};
    if (tid < kPackBuckets) {
      int32_t c[kScanWaves];
#pragma unroll
      for (int w = 0; w < kScanWaves; ++w) c[w] = s_bucket_wave[w][tid];
      int32_t run = s_bucket_carry[tid];
#pragma unroll
      for (int w = 0; w < kScanWaves; ++w) {
        s_bucket_wave[w][tid] = run;
        run += c[w];
      }
      s_bucket_carry[tid] = run;
    }
    lds_barrier();
    if (valid) {
      const Counts ex = add(before, {inc.tok - v.tok, inc.ctx - v.ctx, inc.full - v.full, inc.merge - v.merge,
                                     inc.tiles - v.tiles});
      const int64_t tok = tok_carry + ex.tok;
      const int64_t ctx = ctx_carry + ex.ctx;
      a.cu_seqlens[seq + 1] = tok + count;
      a.cu_context_offsets[seq + 1] = ctx + clen;
      a.context_lens[seq] = static_cast<int32_t>(clen);
      int4 e;
      e.x = full_carry + ex.full;
      e.y = merge_carry + ex.merge;
      e.z = tiles_carry + ex.tiles;
      e.w = bucket >= 0 ? s_bucket_wave[wave][bucket] + wave_rank : -1;
      int4 in;
      in.x = static_cast<int32_t>(start);
      in.y = static_cast<int32_t>(count);
      in.z = row;
      in.w = 0;
      a.ws_seq[2 * seq] = e;
      a.ws_seq[2 * seq + 1] = in;
      if (a.step_rows != nullptr) a.step_rows[seq] = row;
      if constexpr (kFused) {
        f_e = e;
        f_in = in;
        f_tok = tok;
        f_ctx = ctx;
      }
    }
    tok_carry += total.tok;
    ctx_carry += total.ctx;
    full_carry += total.full;
    merge_carry += total.merge;
    tiles_carry += total.tiles;
    lds_barrier();  // s_wave and s_bucket_wave are rewritten by the next chunk
  }
  if (wave == 0) {
    // Bucket bases, largest bucket first, after every full partition: lane l
    // scans bucket 63 - l.
    const int32_t mine = s_bucket_carry[kPackBuckets - 1 - lane];
    const int32_t incl = wave_inclusive_sum(mine);
    a.ws_header[1 + kPackBuckets - 1 - lane] = full_carry + incl - mine;
    if (lane == 0) a.ws_header[0] = full_carry;
    if constexpr (kFused) s_bases[kPackBuckets - 1 - lane] = full_carry + incl - mine;
  }
  if constexpr (kFused) {
    // The fill, one thread per sequence.  The barrier also makes the table
    // updates above visible to every thread reading a row.
    __syncthreads();
    if (tid < a.num_seqs) fill_sequence(a, tid, f_e, f_in, f_tok, f_ctx, s_bases, 0, 1);
  }
}

__global__ __launch_bounds__(kFillThreads) void pack_fill_kernel(PackArgs a) {
  const int seq = blockIdx.x;
  fill_sequence(a, seq, a.ws_seq[2 * seq], a.ws_seq[2 * seq + 1], a.cu_seqlens[seq], a.cu_context_offsets[seq],
                a.ws_header + 1, threadIdx.x, kFillThreads);
}

size_t pack_workspace_size(int64_t num_seqs) {
  return kPackHeaderBytes + static_cast<size_t>(num_seqs > 0 ? num_seqs : 0) * 2 * sizeof(int4);
}

bool pack_fusable(const PackArgs& a, int32_t max_new_tokens, int32_t max_context) {
  return a.num_seqs > 0 && a.num_seqs <= kScanThreads && a.gather_slots == nullptr &&
         a.step_block_tables == nullptr && max_new_tokens > 0 && max_new_tokens <= kFusedMaxWork &&
         max_context > 0 && max_context / a.partition <= kFusedMaxWork;
}

hipError_t launch_pack(const PackArgs& a, hipStream_t stream) {
  if (a.fused) {
    hipLaunchKernelGGL(pack_scan_kernel<true>, dim3(1), dim3(kScanThreads), 0, stream, a);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(pack_scan_kernel<false>, dim3(1), dim3(kScanThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.num_seqs == 0) return e;
  hipLaunchKernelGGL(pack_fill_kernel, dim3(static_cast<uint32_t>(a.num_seqs)), dim3(kFillThreads), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace pa
