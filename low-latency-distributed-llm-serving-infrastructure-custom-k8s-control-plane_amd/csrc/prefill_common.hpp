// Device helpers shared by the MFMA prefill kernels (prefill.hip, heads of
// 64-128; prefill256.hip, heads of 256): MFMA tiles, the LDS transpose read,
// direct global -> LDS copies issued from inline assembly, and the swizzle of
// the 16-byte chunks of an unpadded LDS row.
#pragma once

#include "pa_common.hpp"

namespace pa {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(4))) int32_t const_i32;
// A global-address view of a block-table row: the row pointer may also point
// at a __device__ constant (no table row), which makes plain reads through it
// flat loads, and an LDS wait (lgkmcnt) would then wait for them as well.
typedef const __attribute__((address_space(1))) int32_t global_i32;

// sched_group_barrier classes
constexpr int kSchedValu = 0x002;
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

template <typename T>
__device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
  if constexpr (Elem<T>::kDtype == PA_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                   __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8v, a),
                                                  __builtin_bit_cast(f16x8v, b), c, 0, 0, 0);
  }
}

// ds_read_b64_tr_b16 at an LDS address: inside each group of 16 lanes, lane
// i receives element j from the 8-byte word addressed by lane (i/4 + 4j),
// element i%4 (a 4x4 transpose of 16-bit elements).
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) i16x4v lds_i16x4;
  const i16x4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Direct global -> LDS loads.  Each lane's 16 bytes land at lds_base + 16 *
// lane; lds_base must be wave-uniform.  dma16 takes a per-lane address,
// dma16_s a wave-uniform base plus a per-lane 32-bit offset.  They are
// issued from inline assembly so that the compiler, which cannot tell the
// stage buffers apart, does not drain them before every LDS read; the
// kernel waits for them itself (s_waitcnt vmcnt) before the barrier that
// publishes a stage, and every LDS access is ordered against them by that
// barrier (an asm statement with a memory clobber).
__device__ __forceinline__ void dma16(uint32_t lds_base, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_base), "v"(src)
               : "memory", "m0");
}
// A wave-uniform pointer in scalar registers (the scalar-base copies take
// their base from an SGPR pair).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ void dma4_s(uint32_t lds_base, uint32_t voff, const void* sbase) {
  sbase = uniform_ptr(sbase);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_base), "v"(voff), "s"(sbase)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16_s(uint32_t lds_base, uint32_t voff, const void* sbase) {
  sbase = uniform_ptr(sbase);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_base), "v"(voff),
               "s"(sbase)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until at most n (wave-uniform, 0 <= n <= MAX) vector memory
// operations are outstanding: one s_waitcnt with the count as its immediate.
template <int MAX>
__device__ __forceinline__ void wait_vmcnt_at_most(int n) {
  if constexpr (MAX <= 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= MAX) wait_vmcnt<MAX>();
    else wait_vmcnt_at_most<MAX - 1>(n);
  }
}
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Swizzle of the 16-byte chunks of an unpadded LDS row: chunk c of row r sits
// at position c ^ chunk_swizzle(r).  It keeps the 16-byte K reads (16 rows,
// one chunk) and the transpose reads of V (4 rows x 4 chunks per 32 lanes)
// free of bank conflicts.
template <int CHUNKS>
__device__ __forceinline__ int chunk_swizzle(int r) {
  // (rows of 32 chunks: banks repeat every 16 chunks, so the swizzle of 16)
  if constexpr (CHUNKS >= 16) return 4 * (r & 3) + ((r >> 2) & 3);
  else return 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
}

constexpr float kLazyRescale = 8.f;  // log2 headroom before a row maximum moves

}  // namespace pa
