// Causal chunked prefill over an fp32 paged cache (VALU, fp32 throughout).
//
// The MFMA prefill takes 16-bit caches; this kernel serves fp32 ones with
// the same work items: one workgroup (4 waves) per (sequence, query tile,
// KV head, sub-group), 128 query rows = tile tokens x G query heads (row
// r = g * MTOK + tok, as in the MFMA kernel).  The context is walked in
// stages of 64 tokens:
//
//   1. the stage's K and V rows go from HBM into LDS (each thread moves
//      16-byte pieces; the block id of a row comes from the block table);
//   2. scores: thread t owns rows t/8 + 32 i (i < 4) and the stage's tokens
//      8 j + t%8 (j < 8), and forms its 4 x 8 dot products from 16-byte LDS
//      reads of q and K (rows padded by 16 bytes: the eight consecutive rows
//      a wave reads at once fall in different banks);
//   3. online softmax in base 2 per row (the 8 threads sharing the rows
//      combine their maxima and sums with DPP), p -> LDS;
//   4. P x V: the same thread owns the same 4 rows and the head-dimension
//      elements 32 e + 4 (t%8) .. +3, so the per-row statistics (max, sum,
//      rescale) never leave the thread and each V read of 8 lanes is one
//      128-byte run.
//
// Masking follows the reference's block-diagonal causal mask
// (app/model/paged_attention.py:92-118 applied by SDPA,
// paged_attention.py:170-178): query token j of a sequence at position
// start + j attends context positions [0, start + j].
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kF32Threads = 256;
constexpr int kF32Rows = 128;  // query rows per workgroup (as the MFMA kernel)
constexpr int kF32Stage = 64;  // context tokens per stage

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 lds4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Sum / max over the 8 consecutive lanes of a row block.
__device__ __forceinline__ float sum8(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  return x + dpp<kDppRowHalfMirror>(x);
}
__device__ __forceinline__ float max8(float x) {
  x = fmaxf(x, dpp<kDppQuadXor1>(x));
  x = fmaxf(x, dpp<kDppQuadXor2>(x));
  return fmaxf(x, dpp<kDppRowHalfMirror>(x));
}

template <int D, int G>
__global__ __launch_bounds__(kF32Threads) void prefill_f32_kernel(PrefillArgs a) {
  constexpr int MTOK = kF32Rows / G;  // query tokens per workgroup
  constexpr int LD = D + 4;           // padded LDS row (floats)
  constexpr int DS = D / 8;           // head-dimension slice of a thread in P x V
  static_assert(DS % 4 == 0, "slices of whole 16-byte pieces");

  // K rows of a stage, then (once the scores are formed) its probabilities
  // p[token][row] in the same space: 132 KB in all for D = 128.
  constexpr int KP = kF32Stage * LD > kF32Stage * kF32Rows ? kF32Stage * LD : kF32Stage * kF32Rows;
  __shared__ __attribute__((aligned(16))) float s_q[kF32Rows * LD];
  __shared__ __attribute__((aligned(16))) float s_kp[KP];
  __shared__ __attribute__((aligned(16))) float s_v[kF32Stage * LD];
  __shared__ int s_ok[kF32Stage];  // the stage's token has a block in the pool
  float* const s_k = s_kp;
  float* const s_p = s_kp;

  const int tid = threadIdx.x;
  const int rb = tid >> 3;  // rows rb + 32 i, i < 4
  const int c = tid & 7;    // tokens 8 j + c (scores), elements 32 e + 4 c .. (P x V)
  const int hkv = a.num_kv_heads;
  // Highest item first: the last query tiles of a sequence see the most context.
  const int64_t blk_id = static_cast<int64_t>(gridDim.x) - 1 - blockIdx.x;
  const int units = hkv * a.sub_groups;
  const int64_t item = blk_id / units;
  const int unit = static_cast<int>(blk_id - item * units);
  const int kvh = unit / a.sub_groups;
  const int h0 = kvh * a.group + (unit - kvh * a.sub_groups) * G;  // first query head
  const int seq = a.items[2 * item];
  const int qt = a.items[2 * item + 1];
  const int64_t first = a.cu_seqlens[seq];
  const int count = static_cast<int>(a.cu_seqlens[seq + 1] - first);
  const int ctx = a.context_lens[seq];
  const int start = ctx - count;
  const int tok0 = qt * MTOK;
  const int ntok = min(MTOK, count - tok0);
  if (ntok <= 0) return;
  const int log2_bs = a.log2_block_size;
  const int bs_mask = (1 << log2_bs) - 1;
  const int64_t row_elems = static_cast<int64_t>(hkv) * D;  // cache row of one token
  const int64_t trow = a.rows != nullptr ? a.rows[seq] : seq;
  const bool row_ok = trow >= 0 && trow < a.num_table_rows;
  // A sequence without a table row reads as one block of id -1.  The pointer
  // stays a global one (a select with a constant array would make every
  // table read a flat load, which the LDS waits then also wait for).
  const int32_t* bt = a.block_tables + (row_ok ? trow * a.block_table_stride : 0);
  const int bt_stride = row_ok ? a.block_table_stride : 1;
  const float* kbase = reinterpret_cast<const float*>(a.key_cache) + kvh * D;
  const float* vbase = reinterpret_cast<const float*>(a.value_cache) + kvh * D;
  const int hq = hkv * a.group;

  // Query rows -> LDS (rows past the tile or past G heads stay zero).
  for (int i = tid; i < kF32Rows * (D / 4); i += kF32Threads) {
    const int r = i / (D / 4), q4 = i - r * (D / 4);
    const int g = r / MTOK, tok = r - g * MTOK;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (tok < ntok && g < G) {
      const float* qrow = reinterpret_cast<const float*>(a.query) +
                          (first + tok0 + tok) * a.q_token_stride + static_cast<int64_t>(h0 + g) * a.q_head_stride;
      v = *reinterpret_cast<const f32x4*>(qrow + 4 * q4);
    }
    *reinterpret_cast<f32x4*>(s_q + r * LD + 4 * q4) = v;
  }

  // This thread's rows: causal limits and liveness.
  int qpos[4];
  bool live[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rb + 32 * i;
    const int g = r / MTOK, tok = r - g * MTOK;
    live[i] = tok < ntok && g < G;
    qpos[i] = start + tok0 + tok;
  }
  const int kv_end = min(ctx, start + tok0 + ntok);  // exclusive
  // Positions that have a block-table column (the rest are never read).
  const int kv_read = static_cast<int>(
      min(static_cast<int64_t>(kv_end), static_cast<int64_t>(bt_stride) << log2_bs));
  const int nstages = (kv_end + kF32Stage - 1) / kF32Stage;
  const float scale = a.scale_log2e;

  float m[4], l[4], acc[4][DS];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = kScoreFloor;
    l[i] = 0.f;
#pragma unroll
    for (int e = 0; e < DS; ++e) acc[i][e] = 0.f;
  }

  // K and V rows of a stage: each thread's NPT 16-byte pieces of both are
  // loaded into registers a stage ahead (during the previous stage's
  // arithmetic) and stored into LDS when the stage starts.  Rows past the
  // readable context re-read its last row and an out-of-pool block id reads
  // block 0 (finite values; their scores are masked: such positions are
  // skipped, as in decode).
  constexpr int NPT = kF32Stage * (D / 4) / kF32Threads;
  static_assert(NPT * kF32Threads == kF32Stage * (D / 4), "whole pieces per thread");
  // The block ids of a stage's rows are loaded one stage earlier still, so
  // that no copy waits on its table read.
  f32x4 pk[NPT], pv[NPT];
  bool pok[NPT];
  int bid[NPT];
  auto load_ids = [&](int st) {
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int r = (tid + j * kF32Threads) / (D / 4);
      bid[j] = row_ok ? bt[min(st * kF32Stage + r, kv_read - 1) >> log2_bs] : -1;
    }
  };
  auto load_stage = [&](int st) {
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int i = tid + j * kF32Threads;
      const int r = i / (D / 4), q4 = i - r * (D / 4);
      const int pos = min(st * kF32Stage + r, kv_read - 1);
      int b = bid[j];
      const bool in_pool = static_cast<uint32_t>(b) < static_cast<uint32_t>(a.total_blocks);
      pok[j] = in_pool && st * kF32Stage + r < kv_read;
      b = in_pool ? b : 0;
      const int64_t off = ((static_cast<int64_t>(b) << log2_bs) + (pos & bs_mask)) * row_elems + 4 * q4;
      pk[j] = *reinterpret_cast<const f32x4*>(kbase + off);
      pv[j] = *reinterpret_cast<const f32x4*>(vbase + off);
    }
  };
  load_ids(0);
  load_stage(0);
  if (nstages > 1) load_ids(1);

  for (int st = 0; st < nstages; ++st) {
    __syncthreads();  // the previous stage's K, V and p are consumed
    // 1. K and V rows of the stage -> LDS; then the next stage's loads.
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int i = tid + j * kF32Threads;
      const int r = i / (D / 4), q4 = i - r * (D / 4);
      if (q4 == 0) s_ok[r] = pok[j];
      *reinterpret_cast<f32x4*>(s_k + r * LD + 4 * q4) = pk[j];
      *reinterpret_cast<f32x4*>(s_v + r * LD + 4 * q4) = pv[j];
    }
    if (st + 1 < nstages) {
      load_stage(st + 1);
      if (st + 2 < nstages) load_ids(st + 2);
    }
    __syncthreads();

    // 2. scores of rows rb + 32 i x tokens 8 j + c of the stage.
    float s[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) s[i][j] = 0.f;
    for (int d = 0; d < D; d += 4) {
      f32x4 q[4], k[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) q[i] = lds4(s_q + (rb + 32 * i) * LD + d);
#pragma unroll
      for (int j = 0; j < 8; ++j) k[j] = lds4(s_k + (8 * j + c) * LD + d);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          s[i][j] = fmaf(q[i].x, k[j].x, s[i][j]);
          s[i][j] = fmaf(q[i].y, k[j].y, s[i][j]);
          s[i][j] = fmaf(q[i].z, k[j].z, s[i][j]);
          s[i][j] = fmaf(q[i].w, k[j].w, s[i][j]);
        }
    }

    __syncthreads();  // every thread's scores are formed: K's space takes p

    // 3. online softmax per row (8 threads per row block), p -> LDS.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float tmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int pos = st * kF32Stage + 8 * j + c;
        if (pos > qpos[i] || pos >= kv_end || !s_ok[8 * j + c]) s[i][j] = -INFINITY;
        tmax = fmaxf(tmax, s[i][j]);
      }
      const float m_new = fmaxf(m[i], max8(tmax));
      const float alpha = fast_exp2((m[i] - m_new) * scale);
      const float msc = m_new * scale;
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        s[i][j] = fast_exp2(fmaf(s[i][j], scale, -msc));
        psum += s[i][j];
      }
      l[i] = l[i] * alpha + sum8(psum);
#pragma unroll
      for (int e = 0; e < DS; ++e) acc[i][e] *= alpha;
      m[i] = m_new;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // p[token][rb][i]: a thread's four rows are one 16-byte piece.
      const f32x4 p = {s[0][j], s[1][j], s[2][j], s[3][j]};
      *reinterpret_cast<f32x4*>(s_p + (8 * j + c) * kF32Rows + 4 * rb) = p;
    }
    __syncthreads();

    // 4. P x V for rows rb + 32 i and elements 32 e + 4 c ..
    for (int j = 0; j < kF32Stage; ++j) {
      const f32x4 p = lds4(s_p + j * kF32Rows + 4 * rb);
#pragma unroll
      for (int e4 = 0; e4 < DS / 4; ++e4) {
        const f32x4 v = lds4(s_v + j * LD + 32 * e4 + 4 * c);
        acc[0][4 * e4 + 0] = fmaf(p.x, v.x, acc[0][4 * e4 + 0]);
        acc[0][4 * e4 + 1] = fmaf(p.x, v.y, acc[0][4 * e4 + 1]);
        acc[0][4 * e4 + 2] = fmaf(p.x, v.z, acc[0][4 * e4 + 2]);
        acc[0][4 * e4 + 3] = fmaf(p.x, v.w, acc[0][4 * e4 + 3]);
        acc[1][4 * e4 + 0] = fmaf(p.y, v.x, acc[1][4 * e4 + 0]);
        acc[1][4 * e4 + 1] = fmaf(p.y, v.y, acc[1][4 * e4 + 1]);
        acc[1][4 * e4 + 2] = fmaf(p.y, v.z, acc[1][4 * e4 + 2]);
        acc[1][4 * e4 + 3] = fmaf(p.y, v.w, acc[1][4 * e4 + 3]);
        acc[2][4 * e4 + 0] = fmaf(p.z, v.x, acc[2][4 * e4 + 0]);
        acc[2][4 * e4 + 1] = fmaf(p.z, v.y, acc[2][4 * e4 + 1]);
        acc[2][4 * e4 + 2] = fmaf(p.z, v.z, acc[2][4 * e4 + 2]);
        acc[2][4 * e4 + 3] = fmaf(p.z, v.w, acc[2][4 * e4 + 3]);
        acc[3][4 * e4 + 0] = fmaf(p.w, v.x, acc[3][4 * e4 + 0]);
        acc[3][4 * e4 + 1] = fmaf(p.w, v.y, acc[3][4 * e4 + 1]);
        acc[3][4 * e4 + 2] = fmaf(p.w, v.z, acc[3][4 * e4 + 2]);
        acc[3][4 * e4 + 3] = fmaf(p.w, v.w, acc[3][4 * e4 + 3]);
      }
    }
  }

  // Normalised rows out ([T, H_q, D]).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (!live[i]) continue;
    const int r = rb + 32 * i;
    const int g = r / MTOK, tok = r - g * MTOK;
    const float inv = l[i] > 0.f ? 1.f / l[i] : 0.f;
    float* orow = reinterpret_cast<float*>(a.output) +
                  ((first + tok0 + tok) * hq + h0 + g) * static_cast<int64_t>(D) + 4 * c;
#pragma unroll
    for (int e4 = 0; e4 < DS / 4; ++e4) {
      const f32x4 o = {acc[i][4 * e4] * inv, acc[i][4 * e4 + 1] * inv, acc[i][4 * e4 + 2] * inv,
                       acc[i][4 * e4 + 3] * inv};
      *reinterpret_cast<f32x4*>(orow + 32 * e4) = o;
    }
  }
}

template <int D>
static hipError_t launch_prefill_f32_d(const PrefillArgs& a, int group, int64_t num_items,
                                       hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(num_items * a.num_kv_heads * a.sub_groups));
  switch (group / a.sub_groups) {
    case 1: hipLaunchKernelGGL((prefill_f32_kernel<D, 1>), grid, dim3(kF32Threads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((prefill_f32_kernel<D, 2>), grid, dim3(kF32Threads), 0, s, a); break;
    case 3: hipLaunchKernelGGL((prefill_f32_kernel<D, 3>), grid, dim3(kF32Threads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((prefill_f32_kernel<D, 4>), grid, dim3(kF32Threads), 0, s, a); break;
    case 5: hipLaunchKernelGGL((prefill_f32_kernel<D, 5>), grid, dim3(kF32Threads), 0, s, a); break;
    case 6: hipLaunchKernelGGL((prefill_f32_kernel<D, 6>), grid, dim3(kF32Threads), 0, s, a); break;
    case 7: hipLaunchKernelGGL((prefill_f32_kernel<D, 7>), grid, dim3(kF32Threads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((prefill_f32_kernel<D, 8>), grid, dim3(kF32Threads), 0, s, a); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

hipError_t launch_prefill_f32(const PrefillArgs& a, int head_dim, int group, int64_t num_items,
                              hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  if (head_dim == 128) return launch_prefill_f32_d<128>(a, group, num_items, stream);
  if (head_dim == 64) return launch_prefill_f32_d<64>(a, group, num_items, stream);
  return hipErrorNotSupported;
}

}  // namespace pa
