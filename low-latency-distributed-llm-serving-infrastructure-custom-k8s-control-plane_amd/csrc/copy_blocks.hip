// KV block copy: for every (src block, dst block) pair and every layer, copy
// the block's bs x H_kv x D elements of one cache into another (or the same)
// cache.  This is the device side of KVCacheMemoryStrategy.copy_blocks
// (app/memory/strategies.py:50-56, 117-122), which the reference runs as one
// torch copy per block.
//
// One workgroup per (pair, layer); 256 threads move the block in 16-byte
// pieces (4-byte pieces when the block size in bytes is not a multiple of 16
// or a cache is not 16-byte aligned), four pieces in flight per thread, so
// reads and writes are contiguous and coalesced.  Pairs with an index
// outside its cache are skipped.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 4;

template <typename V>
__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(CopyBlocksArgs a) {
  const int64_t pair = blockIdx.x / a.num_layers;
  const int layer = static_cast<int>(blockIdx.x - pair * a.num_layers);
  const int64_t src = a.block_mapping[2 * pair];
  const int64_t dst = a.block_mapping[2 * pair + 1];
  if (src < 0 || src >= a.src_total_blocks || dst < 0 || dst >= a.dst_total_blocks) return;
  const int64_t n = a.block_bytes / static_cast<int64_t>(sizeof(V));
  const V* s = reinterpret_cast<const V*>(static_cast<const char*>(a.src) +
                                          (layer * a.src_total_blocks + src) * a.block_bytes);
  V* d = reinterpret_cast<V*>(static_cast<char*>(a.dst) + (layer * a.dst_total_blocks + dst) * a.block_bytes);
  constexpr int64_t kStep = static_cast<int64_t>(kCopyThreads) * kCopyUnroll;
  int64_t i = threadIdx.x;
  for (; i + (kCopyUnroll - 1) * kCopyThreads < n; i += kStep) {
    V v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) v[u] = s[i + u * kCopyThreads];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) d[i + u * kCopyThreads] = v[u];
  }
  for (; i < n; i += kCopyThreads) d[i] = s[i];
}

hipError_t launch_copy_blocks(const CopyBlocksArgs& a, bool vec16, hipStream_t stream) {
  if (a.num_pairs <= 0 || a.num_layers <= 0 || a.block_bytes <= 0) return hipSuccess;
  const dim3 grid(static_cast<uint32_t>(a.num_pairs * a.num_layers));
  if (vec16)
    hipLaunchKernelGGL(copy_blocks_kernel<uint4>, grid, dim3(kCopyThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(copy_blocks_kernel<uint32_t>, grid, dim3(kCopyThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace pa
