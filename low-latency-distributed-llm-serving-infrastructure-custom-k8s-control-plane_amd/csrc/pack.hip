// Ragged-batch packing on the GPU, in two launches that are linear in the
// batch:
//
//   pack_scan_kernel   one workgroup of 1024 threads.  Applies the queued
//                      block-table updates, then walks the sequences in
//                      chunks of 1024 with block-wide exclusive scans:
//                      cu_seqlens, cu_context_offsets, context_lens, and per
//                      sequence (into the workspace) the offsets of its
//                      full decode partitions, merge entry and prefill tiles
//                      and the rank of its partial partition.
//   pack_fill_kernel   one workgroup per sequence.  Copies the sequence's
//                      block-table row into the step table, writes its
//                      scatter slots, positions, gather slots and work items
//                      at the offsets the scan left.
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
// within a chunk, a wave ranks its lanes of one bucket with a ballot, the 16
// waves' counts are scanned per bucket, and a per-bucket carry crosses the
// chunks; bucket bases (largest bucket first) follow once every chunk is
// counted.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kScanThreads = 1024;
constexpr int kScanWaves = kScanThreads / kWave;
constexpr int kFillThreads = 256;

__device__ __forceinline__ int64_t nonneg(int64_t v) { return v < 0 ? 0 : v; }

// Inclusive scan over a wave (64 lanes) with shuffles.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const T n = __shfl_up(v, o, kWave);
    if (lane >= o) v += n;
  }
  return v;
}

// Exclusive scan of one value per thread across the workgroup; `carry` is
// added to every result and advanced by the workgroup total.  `s_tot` holds
// one entry per wave.  Ends with a barrier, so `s_tot` can be reused.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T& carry, T* s_tot, int lane, int wave) {
  const T inc = wave_inclusive_scan(v, lane);
  if (lane == kWave - 1) s_tot[wave] = inc;
  __syncthreads();
  T before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kScanWaves; ++w) {
    const T t = s_tot[w];
    before += w < wave ? t : T(0);
    total += t;
  }
  const T out = carry + before + inc - v;
  carry += total;
  __syncthreads();
  return out;
}

__global__ __launch_bounds__(kScanThreads) void pack_scan_kernel(PackArgs a) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  // Queued block-table updates land before anything reads the table (the
  // fill kernel runs after this launch on the same stream).
  for (int u = tid; u < a.num_updates; u += kScanThreads) {
    const int32_t row = a.updates[3 * u];
    const int32_t col = a.updates[3 * u + 1];
    if (row >= 0 && row < a.num_table_rows && col >= 0 && col < a.block_table_stride)
      a.block_tables[static_cast<int64_t>(row) * a.block_table_stride + col] = a.updates[3 * u + 2];
  }

  __shared__ int64_t s_tot64[kScanWaves];
  __shared__ int32_t s_tot32[kScanWaves];
  __shared__ int32_t s_bucket_wave[kScanWaves][kPackBuckets];  // per-chunk counts, then offsets
  __shared__ int32_t s_bucket_carry[kPackBuckets];
  if (tid < kPackBuckets) s_bucket_carry[tid] = 0;
  if (tid == 0) {
    a.cu_seqlens[0] = 0;
    a.cu_context_offsets[0] = 0;
  }

  const int64_t P = a.partition;
  int64_t tok_carry = 0, ctx_carry = 0;
  int32_t full_carry = 0, merge_carry = 0, prefill_carry = 0;
  for (int base = 0; base < a.num_seqs; base += kScanThreads) {
    const int seq = base + tid;
    const bool valid = seq < a.num_seqs;
    const int64_t count = valid ? nonneg(a.new_token_counts[seq]) : 0;
    const int64_t clen = valid ? nonneg(a.start_positions[seq]) + count : 0;
    const int32_t nfull = count == 1 ? static_cast<int32_t>(clen / P) : 0;
    const int64_t rlen = count == 1 ? clen % P : 0;
    const int32_t merge = count == 1 && nfull + (rlen > 0 ? 1 : 0) > 1 ? 1 : 0;
    const int32_t tiles = count > 1 ? static_cast<int32_t>((count + a.prefill_tile - 1) / a.prefill_tile) : 0;
    const int bucket = rlen > 0 ? static_cast<int>(((rlen - 1) * kPackBuckets) / P) : -1;

    const int64_t tok = block_exclusive_scan<int64_t>(count, tok_carry, s_tot64, lane, wave);
    const int64_t ctx = block_exclusive_scan<int64_t>(clen, ctx_carry, s_tot64, lane, wave);
    const int32_t fulls = block_exclusive_scan<int32_t>(nfull, full_carry, s_tot32, lane, wave);
    const int32_t mitems = block_exclusive_scan<int32_t>(merge, merge_carry, s_tot32, lane, wave);
    const int32_t pitems = block_exclusive_scan<int32_t>(tiles, prefill_carry, s_tot32, lane, wave);

    // Stable rank of this sequence's partial partition within its bucket.
    for (int i = tid; i < kScanWaves * kPackBuckets; i += kScanThreads)
      (&s_bucket_wave[0][0])[i] = 0;
    __syncthreads();
    int wave_rank = 0;
    uint64_t todo = __ballot(bucket >= 0);
    while (todo != 0) {
      const int leader = __ffsll(static_cast<unsigned long long>(todo)) - 1;
      const int b = __shfl(bucket, leader, kWave);
      const uint64_t same = __ballot(bucket == b);
      if (bucket == b) wave_rank = __popcll(same & ((uint64_t(1) << lane) - 1));
      if (lane == 0) s_bucket_wave[wave][b] = __popcll(same);
      todo &= ~same;
    }
    __syncthreads();
    if (tid < kPackBuckets) {
      int32_t run = s_bucket_carry[tid];
      for (int w = 0; w < kScanWaves; ++w) {
        const int32_t c = s_bucket_wave[w][tid];
        s_bucket_wave[w][tid] = run;
        run += c;
      }
      s_bucket_carry[tid] = run;
    }
    __syncthreads();
    if (valid) {
      a.cu_seqlens[seq + 1] = tok + count;
      a.cu_context_offsets[seq + 1] = ctx + clen;
      a.context_lens[seq] = static_cast<int32_t>(clen);
      int4 e;
      e.x = fulls;
      e.y = mitems;
      e.z = pitems;
      e.w = bucket >= 0 ? s_bucket_wave[wave][bucket] + wave_rank : -1;
      a.ws_seq[seq] = e;
    }
    __syncthreads();  // s_bucket_wave is cleared by the next chunk
  }
  if (tid == 0) {
    // Bucket bases, largest bucket first, after every full partition.
    int32_t run = full_carry;
    for (int b = kPackBuckets - 1; b >= 0; --b) {
      a.ws_header[1 + b] = run;
      run += s_bucket_carry[b];
    }
    a.ws_header[0] = full_carry;
  }
}

__global__ __launch_bounds__(kFillThreads) void pack_fill_kernel(PackArgs a) {
  const int seq = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t start = nonneg(a.start_positions[seq]);
  const int64_t count = nonneg(a.new_token_counts[seq]);
  const int64_t clen = start + count;
  const int64_t tok = a.cu_seqlens[seq];
  const int64_t ctx = a.cu_context_offsets[seq];
  const int4 e = a.ws_seq[seq];
  const int32_t row = a.rows != nullptr ? a.rows[seq] : seq;
  const int32_t* bt = row >= 0 && row < a.num_table_rows
                          ? a.block_tables + static_cast<int64_t>(row) * a.block_table_stride
                          : nullptr;
  const int64_t stride = bt != nullptr ? a.block_table_stride : 0;
  const int64_t bs = a.block_size;

  // The sequence's row of the step's own block table (-1 past its row).
  if (a.step_block_tables != nullptr) {
    int32_t* out = a.step_block_tables + static_cast<int64_t>(seq) * a.step_table_width;
    for (int j = tid; j < a.step_table_width; j += kFillThreads) out[j] = j < stride ? bt[j] : -1;
  }

  // New tokens: scatter slots + positions.
  for (int64_t j = tid; j < count; j += kFillThreads) {
    const int64_t idx = tok + j;
    if (idx >= a.max_query_tokens) break;
    const int64_t p = start + j;
    const int64_t col = p / bs;
    int64_t slot = -1;
    if (col < stride) {
      const int32_t b = bt[col];
      if (b >= 0) slot = static_cast<int64_t>(b) * bs + (p - col * bs);
    }
    a.scatter_slots[idx] = slot;
    a.position_ids[idx] = p;
  }

  // Whole context: gather slots.
  if (a.gather_slots != nullptr) {
    for (int64_t c = tid; c < clen; c += kFillThreads) {
      const int64_t idx = ctx + c;
      if (idx >= a.max_context_tokens) break;
      const int64_t col = c / bs;
      int64_t slot = -1;
      if (col < stride) {
        const int32_t b = bt[col];
        if (b >= 0) slot = static_cast<int64_t>(b) * bs + (c - col * bs);
      }
      a.gather_slots[idx] = slot;
    }
  }

  // Attention work lists.
  const int64_t P = a.partition;
  const int64_t nfull = count == 1 ? clen / P : 0;
  const int64_t rem_idx =
      e.w >= 0 ? static_cast<int64_t>(a.ws_header[1 + ((clen % P - 1) * kPackBuckets) / P]) + e.w : -1;
  if (count == 1 && a.merge_items != nullptr && tid == 0 && e.y < a.max_merge_items &&
      nfull + (rem_idx >= 0 ? 1 : 0) > 1) {
    int4 m;
    m.x = e.x;
    m.y = static_cast<int32_t>(nfull);
    m.z = seq;
    m.w = static_cast<int32_t>(rem_idx);
    reinterpret_cast<int4*>(a.merge_items)[e.y] = m;
  }
  if (count == 1 && a.decode_items != nullptr) {
    for (int64_t p = tid; p < nfull; p += kFillThreads) {
      const int64_t idx = e.x + p;
      if (idx >= a.max_decode_items) break;
      a.decode_items[2 * idx] = seq;
      a.decode_items[2 * idx + 1] = static_cast<int32_t>(p);
    }
    if (tid == 0 && rem_idx >= 0 && rem_idx < a.max_decode_items) {
      a.decode_items[2 * rem_idx] = seq;
      a.decode_items[2 * rem_idx + 1] = static_cast<int32_t>(nfull);
    }
  } else if (count > 1 && a.prefill_items != nullptr) {
    const int64_t ntiles = (count + a.prefill_tile - 1) / a.prefill_tile;
    for (int64_t q = tid; q < ntiles; q += kFillThreads) {
      const int64_t idx = e.z + q;
      if (idx >= a.max_prefill_items) break;
      a.prefill_items[2 * idx] = seq;
      a.prefill_items[2 * idx + 1] = static_cast<int32_t>(q);
    }
  }
}

size_t pack_workspace_size(int64_t num_seqs) {
  return kPackHeaderBytes + static_cast<size_t>(num_seqs > 0 ? num_seqs : 0) * sizeof(int4);
}

hipError_t launch_pack(const PackArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(pack_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.num_seqs == 0) return e;
  hipLaunchKernelGGL(pack_fill_kernel, dim3(static_cast<uint32_t>(a.num_seqs)), dim3(kFillThreads), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace pa
