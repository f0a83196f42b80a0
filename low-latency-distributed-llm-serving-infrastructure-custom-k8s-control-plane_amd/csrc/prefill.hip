// Causal chunked prefill over the paged cache with gfx950 MFMA tiles.
//
// One workgroup (4 waves) per (sequence, query tile, KV head).  The tile
// holds 128 query rows = (128 / G) query tokens x the G query heads that
// share the KV head; wave w owns rows [32w, 32w + 32).  The context is
// walked in tiles of 32 tokens staged through LDS (K row-major, V
// transposed), with flash-style online softmax in fp32.
//
// Both products are computed transposed so that a lane owns one query row:
//   S^T[kv][row] = sum_d K[kv][d] Q[row][d]     (A = K from LDS, B = Q regs)
//   O^T[d][row] += sum_kv V^T[d][kv] P^T[kv][row] (A = V^T from LDS, B = P)
// with v_mfma_f32_32x32x16_bf16.  In the 32x32 accumulator lane l holds
// column l % 32 and rows 8*(i/4) + 4*(l/32) + (i%4), i = 0..15, so the
// softmax max/sum of a query row needs only its own 16 values plus the
// partner lane l ^ 32.  The P^T values a lane already holds are exactly the
// B operand of the PV product once the context index inside each 16-token
// step is permuted (bits 2 and 3 swapped); V^T is stored in LDS in that
// permuted order so each A operand is one 16-byte LDS read.
//
// Reference: the block-diagonal causal mask of app/model/paged_attention.py:
// 92-118 applied by SDPA (paged_attention.py:170-178); query token j of a
// sequence at position start + j attends context positions [0, start + j].
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPrefillThreads = 256;
constexpr int kPrefillRows = 128;  // query rows per workgroup
constexpr int kKvTile = 32;        // context tokens per LDS tile

__device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                 __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
}

// Position of context index kv (0..31) inside a V^T LDS row: bits 2 and 3
// swapped, so the 8 values one lane feeds to an MFMA step are contiguous.
__device__ __forceinline__ int vt_pos(int kv) {
  return (kv & ~12) | ((kv & 4) << 1) | ((kv & 8) >> 1);
}

template <int D, int G>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(PrefillArgs a) {
  constexpr int MTOK = kPrefillRows / G;   // query tokens per workgroup
  constexpr int KS = D / 16;               // MFMA k-steps for QK^T
  constexpr int DB = D / 32;               // 32-wide d blocks of the output
  constexpr int KPAD = 8;                  // bf16 padding per K row
  constexpr int VPAD = 8;                  // bf16 padding per V^T row
  constexpr int CHUNKS = D / 8;            // 16-byte pieces per row

  __shared__ uint16_t s_k[kKvTile][D + KPAD];
  __shared__ uint16_t s_vt[D][kKvTile + VPAD];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int hkv = a.num_kv_heads;
  const int64_t item = blockIdx.x / hkv;
  const int kvh = blockIdx.x - static_cast<int>(item) * hkv;
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
  const int64_t row_stride = static_cast<int64_t>(hkv) * D;
  const int32_t* bt = a.block_tables + static_cast<int64_t>(seq) * a.block_table_stride;

  // This lane's query row.
  const int row = wave * 32 + (lane & 31);
  const int half = lane >> 5;
  const int g = row / MTOK;
  const int tok = row - g * MTOK;
  const bool row_live = tok < ntok;
  const int qpos = start + tok0 + tok;  // causal limit (inclusive)
  const int h = kvh * G + g;

  uint4 qreg[KS];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.query) +
                           (first + tok0 + tok) * a.q_token_stride + h * a.q_head_stride;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qreg[ks] = row_live ? ld16(qrow + ks * 16 + half * 8) : make_uint4(0, 0, 0, 0);
  }

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m = kScoreFloor, l = 0.f;

  const int kv_end = min(ctx, start + tok0 + ntok);  // exclusive
  const float scale = a.scale_log2e;

  for (int kv0 = 0; kv0 < kv_end; kv0 += kKvTile) {
    // ---- stage K (row-major) and V (transposed, permuted) into LDS ----
#pragma unroll
    for (int it = 0; it < (kKvTile * CHUNKS) / kPrefillThreads; ++it) {
      const int idx = it * kPrefillThreads + tid;
      const int kv = idx / CHUNKS;
      const int ch = idx - kv * CHUNKS;
      const int pos = kv0 + kv;
      uint4 kq = make_uint4(0, 0, 0, 0), vq = make_uint4(0, 0, 0, 0);
      if (pos < kv_end) {
        const int col = pos >> log2_bs;
        const int b = col < a.block_table_stride ? bt[col] : -1;
        if (b >= 0 && b < a.total_blocks) {
          const int64_t slot = (static_cast<int64_t>(b) << log2_bs) | (pos & bs_mask);
          const uint16_t* kr = reinterpret_cast<const uint16_t*>(a.key_cache) +
                               slot * row_stride + kvh * D + ch * 8;
          const uint16_t* vr = reinterpret_cast<const uint16_t*>(a.value_cache) +
                               slot * row_stride + kvh * D + ch * 8;
          kq = ld16(kr);
          vq = ld16(vr);
        }
      }
      *reinterpret_cast<uint4*>(&s_k[kv][ch * 8]) = kq;
      const int vp = vt_pos(kv);
      const uint32_t w[4] = {vq.x, vq.y, vq.z, vq.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s_vt[ch * 8 + 2 * e][vp] = static_cast<uint16_t>(w[e] & 0xffffu);
        s_vt[ch * 8 + 2 * e + 1][vp] = static_cast<uint16_t>(w[e] >> 16);
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T --------------------------------------------------
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 ka = *reinterpret_cast<const uint4*>(&s_k[lane & 31][ks * 16 + half * 8]);
      s = mfma32(ka, qreg[ks], s);
    }

    // ---- online softmax for this lane's row ---------------------------
    float tmax = kScoreFloor;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kv = kv0 + 8 * (i >> 2) + 4 * half + (i & 3);
      float v = s[i] * scale;
      if (kv > qpos || kv >= kv_end) v = -INFINITY;
      s[i] = v;
      tmax = fmaxf(tmax, v);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float m_new = fmaxf(m, tmax);
    const float alpha = fast_exp2(m - m_new);
    float rsum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = fast_exp2(s[i] - m_new);
      rsum += s[i];
    }
    rsum += __shfl_xor(rsum, 32, kWave);
    l = l * alpha + rsum;
    m = m_new;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[db][i] *= alpha;

    // ---- O^T += V^T P^T -------------------------------------------------
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 pb;
      pb.x = pack_bf16x2(s[8 * ks + 0], s[8 * ks + 1]);
      pb.y = pack_bf16x2(s[8 * ks + 2], s[8 * ks + 3]);
      pb.z = pack_bf16x2(s[8 * ks + 4], s[8 * ks + 5]);
      pb.w = pack_bf16x2(s[8 * ks + 6], s[8 * ks + 7]);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint4 va =
            *reinterpret_cast<const uint4*>(&s_vt[db * 32 + (lane & 31)][ks * 16 + half * 8]);
        acc[db] = mfma32(va, pb, acc[db]);
      }
    }
    __syncthreads();
  }

  if (!row_live) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = reinterpret_cast<uint16_t*>(a.output) +
                   ((first + tok0 + tok) * (hkv * G) + h) * static_cast<int64_t>(D);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = db * 32 + 8 * q4 + 4 * half;
      uint2 w;
      w.x = pack_bf16x2(acc[db][4 * q4 + 0] * inv, acc[db][4 * q4 + 1] * inv);
      w.y = pack_bf16x2(acc[db][4 * q4 + 2] * inv, acc[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = w;
    }
}

bool prefill_fast_path_supported(int dtype, int head_dim, int group, int block_size) {
  if (dtype != PA_DTYPE_BF16) return false;
  if (head_dim != 64 && head_dim != 128) return false;
  if (group != 1 && group != 2 && group != 4 && group != 8) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  return true;
}

int prefill_tile_for(int group) { return group > 0 ? kPrefillRows / group : kPrefillRows; }

template <int D>
static hipError_t launch_prefill_d(const PrefillArgs& a, int group, int64_t num_items,
                                   hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(num_items * a.num_kv_heads));
  switch (group) {
    case 1: hipLaunchKernelGGL((prefill_kernel<D, 1>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<D, 2>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<D, 4>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((prefill_kernel<D, 8>), grid, dim3(kPrefillThreads), 0, s, a); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int dtype, int head_dim, int group,
                          int64_t num_items, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  if (dtype != PA_DTYPE_BF16) return hipErrorNotSupported;
  if (head_dim == 128) return launch_prefill_d<128>(a, group, num_items, stream);
  if (head_dim == 64) return launch_prefill_d<64>(a, group, num_items, stream);
  return hipErrorNotSupported;
}

}  // namespace pa
