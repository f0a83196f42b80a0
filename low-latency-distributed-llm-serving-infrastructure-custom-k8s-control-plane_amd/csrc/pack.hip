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
// items (seq, partition) for sequences with exactly one new token, the
// merge list ((first decode item, partition count, sequence, 0) of every
// such sequence with more than one partition) and prefill items (seq, query
// tile) for the multi-token sequences, all ordered by sequence.
//
// Each workgroup computes its own prefix sums by reducing over the
// sequences before it (B is at most a few thousand, so this is cheaper than
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

  // Prefix sums over sequences [0, seq).
  int64_t tok = 0, ctx = 0, ditems = 0, pitems = 0, mitems = 0;
  for (int k = tid; k < seq; k += kPackThreads) {
    const int64_t cnt = nonneg(a.new_token_counts[k]);
    const int64_t c = nonneg(a.start_positions[k]) + cnt;
    tok += cnt;
    ctx += c;
    if (cnt == 1) {
      const int64_t np = (c + a.partition - 1) / a.partition;
      ditems += np;
      mitems += np > 1 ? 1 : 0;
    } else if (cnt > 1) {
      pitems += (cnt + a.prefill_tile - 1) / a.prefill_tile;
    }
  }
  __shared__ int64_t s_red[5][kPackThreads / kWave];
#pragma unroll
  for (int o = kWave / 2; o >= 1; o >>= 1) {
    tok += __shfl_xor(tok, o, kWave);
    ctx += __shfl_xor(ctx, o, kWave);
    ditems += __shfl_xor(ditems, o, kWave);
    pitems += __shfl_xor(pitems, o, kWave);
    mitems += __shfl_xor(mitems, o, kWave);
  }
  if (lane == 0) {
    s_red[0][wave] = tok;
    s_red[1][wave] = ctx;
    s_red[2][wave] = ditems;
    s_red[3][wave] = pitems;
    s_red[4][wave] = mitems;
  }
  __syncthreads();
  tok = ctx = ditems = pitems = mitems = 0;
#pragma unroll
  for (int w = 0; w < kPackThreads / kWave; ++w) {
    tok += s_red[0][w];
    ctx += s_red[1][w];
    ditems += s_red[2][w];
    pitems += s_red[3][w];
    mitems += s_red[4][w];
  }

  const int64_t start = nonneg(a.start_positions[seq]);
  const int64_t count = nonneg(a.new_token_counts[seq]);
  const int64_t clen = start + count;
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
  if (count == 1 && a.merge_items != nullptr && tid == 0 && mitems < a.max_merge_items &&
      clen > a.partition) {
    int4 e;
    e.x = static_cast<int32_t>(ditems);
    e.y = static_cast<int32_t>((clen + a.partition - 1) / a.partition);
    e.z = seq;
    e.w = 0;
    reinterpret_cast<int4*>(a.merge_items)[mitems] = e;
  }
  if (count == 1 && a.decode_items != nullptr) {
    const int64_t nparts = (clen + a.partition - 1) / a.partition;
    for (int64_t p = tid; p < nparts; p += kPackThreads) {
      const int64_t idx = ditems + p;
      if (idx >= a.max_decode_items) break;
      a.decode_items[2 * idx] = seq;
      a.decode_items[2 * idx + 1] = static_cast<int32_t>(p);
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
