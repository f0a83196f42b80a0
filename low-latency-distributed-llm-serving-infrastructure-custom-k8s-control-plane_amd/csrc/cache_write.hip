// reshape_and_cache: write the step's new K/V rows into the paged cache.
//
// Reference: PagedKVCacheManager.scatter_layer_kv (app/memory/manager.py:
// 150-168), key_cache[layer].view(N*bs, H_kv, D)[slot_mapping] = keys.
// A pure copy (bit-exact).  Each thread moves one 16-byte piece of a
// (token, head) row; consecutive threads cover a row contiguously, so both
// the reads (from the model's possibly transposed [T, H_kv, D] view) and the
// writes (a 16-byte-aligned row of the cache) are coalesced.  Rows whose
// slot lies outside [0, N*bs) are skipped.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kCacheThreads = 256;

// Vector path: head_dim * elem_bytes is a multiple of 16 and all row
// starts are 16-byte aligned.
__global__ __launch_bounds__(kCacheThreads) void cache_write_vec_kernel(CacheWriteArgs a,
                                                                        int elem_bytes) {
  const int chunks = a.head_dim * elem_bytes / 16;  // per (token, head) row
  const int64_t total = static_cast<int64_t>(a.num_tokens) * a.num_kv_heads * chunks;
  const int64_t row_bytes = static_cast<int64_t>(a.num_kv_heads) * a.head_dim * elem_bytes;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kCacheThreads) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kCacheThreads) {
    const int c = static_cast<int>(i % chunks);
    const int64_t r = i / chunks;
    const int h = static_cast<int>(r % a.num_kv_heads);
    const int64_t t = r / a.num_kv_heads;
    const int64_t slot = a.slot_mapping[t];
    if (slot < 0 || slot >= a.num_slots) continue;
    const int64_t dst = slot * row_bytes + (static_cast<int64_t>(h) * a.head_dim) * elem_bytes + c * 16;
    const char* ks = reinterpret_cast<const char*>(a.key) +
                     (t * a.key_token_stride + h * a.key_head_stride) * elem_bytes + c * 16;
    const char* vs = reinterpret_cast<const char*>(a.value) +
                     (t * a.value_token_stride + h * a.value_head_stride) * elem_bytes + c * 16;
    const uint4 kv = ld16(ks);
    const uint4 vv = ld16(vs);
    st16(reinterpret_cast<char*>(a.key_cache) + dst, kv);
    st16(reinterpret_cast<char*>(a.value_cache) + dst, vv);
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
  const int64_t work = static_cast<int64_t>(a.num_tokens) * a.num_kv_heads *
                       (vec ? a.head_dim * eb / 16 : a.head_dim);
  int64_t blocks = (work + kCacheThreads - 1) / kCacheThreads;
  if (blocks > 65536) blocks = 65536;
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (vec) {
    hipLaunchKernelGGL(cache_write_vec_kernel, grid, dim3(kCacheThreads), 0, stream, a, eb);
  } else if (eb == 4) {
    hipLaunchKernelGGL((cache_write_elem_kernel<uint32_t>), grid, dim3(kCacheThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((cache_write_elem_kernel<uint16_t>), grid, dim3(kCacheThreads), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace pa
