// Generic paged attention: one wavefront per (query token, query head).
//
// Covers every shape the tuned kernels do not (head dims other than 64 and
// 128 up to 256, groups above 64, block sizes that are not powers of two)
// and implements the reference C ABI
// (csrc/include/paged_kernels.h:22-34) over a flat gather list plus a dense
// uint8 mask.  Semantics follow csrc/src/paged_kernels.cpp:30-104: masked
// context tokens are skipped, a row with no attended token and an empty
// context produce zeros.  Softmax is computed online (running max and sum)
// in base 2, accumulation is fp32.
//
// Context tokens are visited in chunks of 64: each lane resolves one token's
// slot (from the mask + gather list, or from the block table), a ballot
// keeps the attended ones, and the wave then walks them in ascending order,
// the lanes splitting the head dimension.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

template <typename T, int EPL, bool kMasked>
__global__ __launch_bounds__(kWave) void generic_attention_kernel(GenericArgs a) {
  const int lane = threadIdx.x;
  const int hq = a.num_query_heads;
  const int64_t rowid = blockIdx.x;
  const int t = static_cast<int>(rowid / hq);
  const int h = static_cast<int>(rowid - static_cast<int64_t>(t) * hq);
  const int group = hq / a.num_kv_heads;
  const int kvh = h / group;
  const int D = a.head_dim;
  const int64_t row_stride = static_cast<int64_t>(a.num_kv_heads) * D;

  int seq = 0;
  int64_t trow = 0;
  int n_ctx;
  if constexpr (kMasked) {
    n_ctx = a.num_context_tokens;
  } else {
    // Largest s with cu_seqlens[s] <= t.
    int lo = 0, hi = a.num_seqs;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.cu_seqlens[mid] <= t) lo = mid; else hi = mid;
    }
    seq = lo;
    trow = a.rows != nullptr ? a.rows[seq] : seq;
    const int64_t first = a.cu_seqlens[seq];
    const int64_t count = a.cu_seqlens[seq + 1] - first;
    if ((a.filter == 1 && count != 1) || (a.filter == 2 && count == 1)) return;
    const int64_t pos = a.context_lens[seq] - count + (t - first);
    n_ctx = static_cast<int>(pos + 1);
    if (n_ctx < 0) n_ctx = 0;
  }

  const T* qrow = reinterpret_cast<const T*>(a.query) + t * a.q_token_stride + h * a.q_head_stride;
  float q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int d = lane + e * kWave;
    q[e] = d < D ? load_scalar<T>(qrow + d) : 0.f;
  }
  const T* kbase = reinterpret_cast<const T*>(a.key_cache) + kvh * D;
  const T* vbase = reinterpret_cast<const T*>(a.value_cache) + kvh * D;

  float m = kScoreFloor, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;

  for (int c0 = 0; c0 < n_ctx; c0 += kWave) {
    const int c = c0 + lane;
    int64_t slot = -1;
    if (c < n_ctx) {
      if constexpr (kMasked) {
        if (a.mask[static_cast<int64_t>(t) * n_ctx + c] != 0) {
          slot = a.gather_slots[c];
          if (slot >= static_cast<int64_t>(a.total_blocks) * a.block_size) slot = -1;
        }
      } else {
        const int col = c / a.block_size;
        if (trow >= 0 && trow < a.num_table_rows && col < a.block_table_stride) {
          const int b = a.block_tables[trow * a.block_table_stride + col];
          if (b >= 0 && b < a.total_blocks)
            slot = static_cast<int64_t>(b) * a.block_size + (c - col * a.block_size);
        }
      }
    }
    uint64_t live = __ballot(slot >= 0);
    while (live) {
      const int src = __builtin_ctzll(live);
      live &= live - 1;
      const int64_t s = __shfl(slot, src, kWave);
      const T* krow = kbase + s * row_stride;
      const T* vrow = vbase + s * row_stride;
      float part = 0.f;
      float v[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int d = lane + e * kWave;
        const bool in = d < D;
        part = fmaf(q[e], in ? load_scalar<T>(krow + d) : 0.f, part);
        v[e] = in ? load_scalar<T>(vrow + d) : 0.f;
      }
      const float score = wave_sum(part) * a.scale_log2e;
      const float m_new = fmaxf(m, score);
      const float alpha = fast_exp2(m - m_new);
      const float p = fast_exp2(score - m_new);
      l = l * alpha + p;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = fmaf(p, v[e], acc[e] * alpha);
      m = m_new;
    }
  }

  T* orow = reinterpret_cast<T*>(a.output) + (static_cast<int64_t>(t) * hq + h) * D;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int d = lane + e * kWave;
    if (d < D) store_scalar<T>(orow + d, acc[e] * inv);
  }
}

bool generic_supported(int dtype, int head_dim) {
  if (dtype != PA_DTYPE_F32 && dtype != PA_DTYPE_BF16 && dtype != PA_DTYPE_F16) return false;
  return head_dim >= 1 && head_dim <= 256;
}

template <typename T, bool kMasked>
static hipError_t launch_generic_t(const GenericArgs& a, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.num_query_tokens) * a.num_query_heads;
  if (rows <= 0) return hipSuccess;
  const dim3 grid(static_cast<uint32_t>(rows));
  if (a.head_dim <= 64)
    hipLaunchKernelGGL((generic_attention_kernel<T, 1, kMasked>), grid, dim3(kWave), 0, s, a);
  else if (a.head_dim <= 128)
    hipLaunchKernelGGL((generic_attention_kernel<T, 2, kMasked>), grid, dim3(kWave), 0, s, a);
  else
    hipLaunchKernelGGL((generic_attention_kernel<T, 4, kMasked>), grid, dim3(kWave), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_generic(const GenericArgs& a, int dtype, bool masked, hipStream_t s) {
  switch (dtype) {
    case PA_DTYPE_F32:
      return masked ? launch_generic_t<float, true>(a, s) : launch_generic_t<float, false>(a, s);
    case PA_DTYPE_BF16:
      return masked ? launch_generic_t<bf16_t, true>(a, s) : launch_generic_t<bf16_t, false>(a, s);
    case PA_DTYPE_F16:
      return masked ? launch_generic_t<f16_t, true>(a, s) : launch_generic_t<f16_t, false>(a, s);
    default:
      return hipErrorNotSupported;
  }
}

}  // namespace pa
