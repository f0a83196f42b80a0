// reshape_and_cache: write the step's new K/V rows into the paged cache.
//
// Reference: PagedKVCacheManager.scatter_layer_kv (app/memory/manager.py:
// 150-168), key_cache[layer].view(N*bs, H_kv, D)[slot_mapping] = keys.
// A pure copy (bit-exact).  Each thread moves 16-byte pieces of a (token,
// head) row; consecutive threads cover a row contiguously, so both the reads
// (from the model's possibly transposed [T, H_kv, D] view) and the writes (a
// 16-byte-aligned row of the cache) are coalesced.  Rows whose slot lies
// outside [0, N*bs) are skipped.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kCacheThreads = 256;

// Vector path: head_dim * elem_bytes is a multiple of 16 and all row
// starts are 16-byte aligned.  One workgroup per token (grid-stride over
// tokens): its slot is one scalar load, and its threads move the token's
// H_kv * D * elem_bytes / 16 pieces of K and of V with 32-bit index math (a
// shift when the pieces per head are a power of two).
template <bool kPow2>
__global__ __launch_bounds__(kCacheThreads) void cache_write_vec_kernel(CacheWriteArgs a, int elem_bytes,
                                                                        int chunks_log2) {
  const int chunks = a.head_dim * elem_bytes / 16;  // pieces per (token, head) row
  const int pieces = a.num_kv_heads * chunks;       // pieces per token
  const int64_t row_bytes = static_cast<int64_t>(a.num_kv_heads) * a.head_dim * elem_bytes;
  const int64_t k_tok = a.key_token_stride * elem_bytes, k_head = a.key_head_stride * elem_bytes;
  const int64_t v_tok = a.value_token_stride * elem_bytes, v_head = a.value_head_stride * elem_bytes;
  for (int64_t t = blockIdx.x; t < a.num_tokens; t += gridDim.x) {
    const int64_t slot = a.slot_mapping[t];
    if (slot < 0 || slot >= a.num_slots) continue;
    char* kd = reinterpret_cast<char*>(a.key_cache) + slot * row_bytes;
    char* vd = reinterpret_cast<char*>(a.value_cache) + slot * row_bytes;
    const char* ks = reinterpret_cast<const char*>(a.key) + t * k_tok;
    const char* vs = reinterpret_cast<const char*>(a.value) + t * v_tok;
    for (int p = threadIdx.x; p < pieces; p += blockDim.x) {
      const int h = kPow2 ? p >> chunks_log2 : p / chunks;
      const int c = (p - h * chunks) * 16;
      const uint4 kv = ld16(ks + h * k_head + c);
      const uint4 vv = ld16(vs + h * v_head + c);
      st16(kd + p * 16, kv);
      st16(vd + p * 16, vv);
    }
  }
}

// Element path for any shape / alignment.
template <typename W>
__global__ __launch_bounds__(kCacheThreads) void cache_write_elem_kernel(CacheWriteArgs a) {
  const int64_t total = static_cast<int64_t>(a.num_tokens) * a.num_kv_heads * a.head_dim;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kCacheThreads) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kCacheThreads) {
    const int d = static_cast<int>(i % a.head_dim);
    const int64_t r = i / a.head_dim;
    const int h = static_cast<int>(r % a.num_kv_heads);
    const int64_t t = r / a.num_kv_heads;
    const int64_t slot = a.slot_mapping[t];
    if (slot < 0 || slot >= a.num_slots) continue;
    const int64_t dst = (slot * a.num_kv_heads + h) * a.head_dim + d;
    reinterpret_cast<W*>(a.key_cache)[dst] =
        reinterpret_cast<const W*>(a.key)[t * a.key_token_stride + h * a.key_head_stride + d];
    reinterpret_cast<W*>(a.value_cache)[dst] =
        reinterpret_cast<const W*>(a.value)[t * a.value_token_stride + h * a.value_head_stride + d];
  }
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

hipError_t launch_cache_write(const CacheWriteArgs& a, int dtype, hipStream_t stream) {
  if (a.num_tokens <= 0) return hipSuccess;
  const int eb = dtype == PA_DTYPE_F32 ? 4 : 2;
  const bool vec = (a.head_dim * eb) % 16 == 0 && aligned16(a.key) && aligned16(a.value) &&
                   aligned16(a.key_cache) && aligned16(a.value_cache) &&
                   (a.key_token_stride * eb) % 16 == 0 && (a.key_head_stride * eb) % 16 == 0 &&
                   (a.value_token_stride * eb) % 16 == 0 && (a.value_head_stride * eb) % 16 == 0;
  if (vec) {
    const int chunks = a.head_dim * eb / 16;
    const int pieces = a.num_kv_heads * chunks;
    // Threads per workgroup: the token's pieces, in whole waves, at most 256.
    const int threads = pieces >= kCacheThreads ? kCacheThreads : ((pieces + kWave - 1) / kWave) * kWave;
    const dim3 grid(static_cast<uint32_t>(a.num_tokens < 65536 ? a.num_tokens : 65536));
    int log2c = 0;
    while ((1 << log2c) < chunks) ++log2c;
    if ((1 << log2c) == chunks)
      hipLaunchKernelGGL(cache_write_vec_kernel<true>, grid, dim3(threads), 0, stream, a, eb, log2c);
    else
      hipLaunchKernelGGL(cache_write_vec_kernel<false>, grid, dim3(threads), 0, stream, a, eb, 0);
    return hipGetLastError();
  }
  const int64_t work = static_cast<int64_t>(a.num_tokens) * a.num_kv_heads * a.head_dim;
  int64_t blocks = (work + kCacheThreads - 1) / kCacheThreads;
  if (blocks > 65536) blocks = 65536;
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (eb == 4) {
    hipLaunchKernelGGL((cache_write_elem_kernel<uint32_t>), grid, dim3(kCacheThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((cache_write_elem_kernel<uint16_t>), grid, dim3(kCacheThreads), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace pa
