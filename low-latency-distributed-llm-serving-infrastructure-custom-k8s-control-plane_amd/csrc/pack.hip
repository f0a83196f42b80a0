// Ragged-batch packing on the GPU: one workgroup per sequence.
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
// In addition it emits the work lists of the attention kernels: decode
// items (seq, partition) for sequences with exactly one new token -- every
// full partition first (by sequence), then the partial last partitions from
// longest to shortest -- the merge list ((first full item, number of full
// partitions, sequence, item of the partial one or -1) of every such
// sequence with more than one partition, by sequence) and prefill items
// (seq, query tile) for the multi-token sequences, by sequence.
//
// Each workgroup computes its own prefix sums and ranks by reducing over
// the other sequences (B is at most a few thousand, so this is cheaper than
// a separate scan launch), then writes its sequence's entries.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kPackThreads = 256;

__device__ __forceinline__ int64_t nonneg(int64_t v) { return v < 0 ? 0 : v; }

__global__ __launch_bounds__(kPackThreads) void pack_kernel(PackArgs a) {
  const int seq = blockIdx.x;
  const int tid = threadIdx.x;
  if (a.num_seqs == 0) {  // empty batch: cu arrays are [0]
    if (tid == 0) {
      a.cu_seqlens[0] = 0;
      a.cu_context_offsets[0] = 0;
    }
    return;
  }
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  const int64_t start = nonneg(a.start_positions[seq]);
  const int64_t count = nonneg(a.new_token_counts[seq]);
  const int64_t clen = start + count;
  // Decode partitions of this sequence: `nfull` full ones and, when the
  // context is not a multiple of the partition, one remainder of `rlen`.
  const int64_t P = a.partition;
  const int64_t nfull = count == 1 ? clen / P : 0;
  const int64_t rlen = count == 1 ? clen % P : 0;

  // One pass over all sequences: prefix sums over [0, seq) plus the totals
  // that place the decode items (all full partitions first, by sequence;
  // then the remainders from longest to shortest, ties by sequence, so the
  // short work lands at the end of the launch).
  int64_t tok = 0, ctx = 0, pitems = 0, mitems = 0, fulls = 0, total_full = 0, rank = 0;
  for (int k = tid; k < a.num_seqs; k += kPackThreads) {
    const int64_t cnt = nonneg(a.new_token_counts[k]);
    const int64_t c = nonneg(a.start_positions[k]) + cnt;
    const int64_t kf = cnt == 1 ? c / P : 0;
    const int64_t kr = cnt == 1 ? c % P : 0;
    total_full += kf;
    if (rlen > 0 && kr > 0 && (kr > rlen || (kr == rlen && k < seq))) ++rank;
    if (k < seq) {
      tok += cnt;
      ctx += c;
      fulls += kf;
      if (cnt == 1) {
        mitems += kf + (kr > 0 ? 1 : 0) > 1 ? 1 : 0;
      } else if (cnt > 1) {
        pitems += (cnt + a.prefill_tile - 1) / a.prefill_tile;
      }
    }
  }
  constexpr int kSums = 7;
  __shared__ int64_t s_red[kSums][kPackThreads / kWave];
  int64_t v[kSums] = {tok, ctx, pitems, mitems, fulls, total_full, rank};
#pragma unroll
  for (int i = 0; i < kSums; ++i) {
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) v[i] += __shfl_xor(v[i], o, kWave);
    if (lane == 0) s_red[i][wave] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSums; ++i) {
    v[i] = 0;
#pragma unroll
    for (int w = 0; w < kPackThreads / kWave; ++w) v[i] += s_red[i][w];
  }
  tok = v[0];
  ctx = v[1];
  pitems = v[2];
  mitems = v[3];
  fulls = v[4];
  total_full = v[5];
  rank = v[6];
  const int64_t bs = a.block_size;
  const int32_t* bt = a.block_tables + static_cast<int64_t>(seq) * a.block_table_stride;

  if (tid == 0) {
    if (seq == 0) {
      a.cu_seqlens[0] = 0;
      a.cu_context_offsets[0] = 0;
    }
    a.cu_seqlens[seq + 1] = tok + count;
    a.cu_context_offsets[seq + 1] = ctx + clen;
    a.context_lens[seq] = static_cast<int32_t>(clen);
  }

  // New tokens: scatter slots + positions.
  for (int64_t j = tid; j < count; j += kPackThreads) {
    const int64_t idx = tok + j;
    if (idx >= a.max_query_tokens) break;
    const int64_t p = start + j;
    const int64_t col = p / bs;
    int64_t slot = -1;
    if (col < a.block_table_stride) {
      const int32_t b = bt[col];
      if (b >= 0) slot = static_cast<int64_t>(b) * bs + (p - col * bs);
    }
    a.scatter_slots[idx] = slot;
    a.position_ids[idx] = p;
  }

  // Whole context: gather slots.
  if (a.gather_slots != nullptr) {
    for (int64_t c = tid; c < clen; c += kPackThreads) {
      const int64_t idx = ctx + c;
      if (idx >= a.max_context_tokens) break;
      const int64_t col = c / bs;
      int64_t slot = -1;
      if (col < a.block_table_stride) {
        const int32_t b = bt[col];
        if (b >= 0) slot = static_cast<int64_t>(b) * bs + (c - col * bs);
      }
      a.gather_slots[idx] = slot;
    }
  }

  // Attention work lists.
  const int64_t rem_idx = rlen > 0 ? total_full + rank : -1;
  if (count == 1 && a.merge_items != nullptr && tid == 0 && mitems < a.max_merge_items &&
      nfull + (rlen > 0 ? 1 : 0) > 1) {
    int4 e;
    e.x = static_cast<int32_t>(fulls);
    e.y = static_cast<int32_t>(nfull);
    e.z = seq;
    e.w = static_cast<int32_t>(rem_idx);
    reinterpret_cast<int4*>(a.merge_items)[mitems] = e;
  }
  if (count == 1 && a.decode_items != nullptr) {
    for (int64_t p = tid; p < nfull; p += kPackThreads) {
      const int64_t idx = fulls + p;
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
    for (int64_t q = tid; q < ntiles; q += kPackThreads) {
      const int64_t idx = pitems + q;
      if (idx >= a.max_prefill_items) break;
      a.prefill_items[2 * idx] = seq;
      a.prefill_items[2 * idx + 1] = static_cast<int32_t>(q);
    }
  }
}

hipError_t launch_pack(const PackArgs& a, hipStream_t stream) {
  const uint32_t grid = a.num_seqs > 0 ? static_cast<uint32_t>(a.num_seqs) : 1u;
  hipLaunchKernelGGL(pack_kernel, dim3(grid), dim3(kPackThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace pa
