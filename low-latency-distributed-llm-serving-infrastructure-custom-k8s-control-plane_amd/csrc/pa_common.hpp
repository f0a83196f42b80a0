// Shared device helpers for the gfx950 paged-attention kernels.
//
// Conventions used by every kernel in this directory:
//  * wavefront = 64 lanes; workgroups are 256 threads (4 waves) unless a
//    kernel says otherwise;
//  * bf16 values travel as raw uint16 pairs packed in uint32 and are widened
//    to fp32 with shifts (exact); fp32 -> bf16 rounds to nearest even;
//  * all accumulation is fp32;
//  * softmax runs in base 2: scores are pre-multiplied by scale*log2(e) and
//    exponentiated with the hardware exp2 (v_exp_f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "paged_attention_amd.h"

namespace pa {

constexpr int kWave = 64;

// The block-table row a sequence with an invalid table row reads: one -1
// (no block), so no kernel reads outside a caller's table.
static __device__ const int32_t kNoBlockRow[1] = {-1};
// XCDs of an MI355X: workgroup ids of one launch are dealt to them round-robin,
// and each XCD has its own L2.
constexpr int kXcds = 8;
constexpr float kLog2e = 1.4426950408889634f;
// Finite floor used as the initial running maximum: exp2 of a masked score
// (-inf) minus the floor is exactly 0 and no (-inf) - (-inf) NaN can appear.
// -1e30 is also the reference's own "masked" threshold
// (csrc/src/paged_kernels.cpp:79), and floor * scale stays finite.
constexpr float kScoreFloor = -1e30f;

struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  _Float16 v;
};

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static constexpr int kBytes = 4;
  static constexpr int kDtype = PA_DTYPE_F32;
};
template <>
struct Elem<bf16_t> {
  static constexpr int kBytes = 2;
  static constexpr int kDtype = PA_DTYPE_BF16;
};
template <>
struct Elem<f16_t> {
  static constexpr int kBytes = 2;
  static constexpr int kDtype = PA_DTYPE_F16;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2cv __attribute__((ext_vector_type(2)));

// fp32 pair -> packed bf16 pair, round to nearest even: one gfx950
// v_cvt_pk_bf16_f32 (NaN stays NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2cv));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(pack_bf16x2(f, 0.f) & 0xffffu);
}

typedef _Float16 f16x2cv __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2dv __attribute__((ext_vector_type(2)));

// fp32 pair -> packed pair of a 16-bit element type (round to nearest even).
template <typename T>
__device__ __forceinline__ uint32_t pack_half2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack_half2<bf16_t>(float lo, float hi) {
  return pack_bf16x2(lo, hi);
}
template <>
__device__ __forceinline__ uint32_t pack_half2<f16_t>(float lo, float hi) {
  const f32x2v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2cv));
}

// Dot product of two packed pairs of a 16-bit element type, accumulated in
// fp32 (v_dot2_f32_bf16 / v_dot2_f32_f16).
template <typename T>
__device__ __forceinline__ float dot2_half(uint32_t a, uint32_t b, float c);
template <>
__device__ __forceinline__ float dot2_half<bf16_t>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2dv, a),
                                         __builtin_bit_cast(bf16x2dv, b), c, false);
}
template <>
__device__ __forceinline__ float dot2_half<f16_t>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2cv, a), __builtin_bit_cast(f16x2cv, b), c,
                                false);
}

template <typename T>
__device__ __forceinline__ float load_scalar(const T* p);
template <>
__device__ __forceinline__ float load_scalar<float>(const float* p) {
  return *p;
}
template <>
__device__ __forceinline__ float load_scalar<bf16_t>(const bf16_t* p) {
  return bf16_to_f32(p->bits);
}
template <>
__device__ __forceinline__ float load_scalar<f16_t>(const f16_t* p) {
  return static_cast<float>(p->v);
}

template <typename T>
__device__ __forceinline__ void store_scalar(T* p, float v);
template <>
__device__ __forceinline__ void store_scalar<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void store_scalar<bf16_t>(bf16_t* p, float v) {
  p->bits = f32_to_bf16(v);
}
template <>
__device__ __forceinline__ void store_scalar<f16_t>(f16_t* p, float v) {
  p->v = static_cast<_Float16>(v);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// ---- cross-lane helpers -----------------------------------------------
// DPP controls (gfx9 encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i within 8
constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15-i within 16
constexpr int kDppRowRor1 = 0x121;        // lane i <- lane (i+1)%16 within 16
constexpr int kDppRowRor2 = 0x122;        // lane i <- lane (i+2)%16 within 16
constexpr int kDppRowRor4 = 0x124;        // lane i <- lane (i+4)%16 within 16
constexpr int kDppRowRor8 = 0x128;        // lane i <- lane (i+8)%16 within 16

template <int Ctrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), Ctrl, 0xF, 0xF, false));
}

// Sum over aligned groups of L consecutive lanes (L in {1,2,4,8,16}); every
// lane of the group ends with the group total.
template <int L>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (L >= 2) x += dpp<kDppQuadXor1>(x);
  if constexpr (L >= 4) x += dpp<kDppQuadXor2>(x);
  if constexpr (L >= 8) x += dpp<kDppRowHalfMirror>(x);
  if constexpr (L >= 16) x += dpp<kDppRowMirror>(x);
  static_assert(L <= 16, "group_sum supports groups of at most 16 lanes");
  return x;
}

// Combine every lane with its partner lane ^ 32 in the other half of the
// wave.  gfx950 v_permlane32_swap with both operands = x leaves, at every
// lane position, element 0 = the value of half 0 and element 1 = the value
// of half 1, so one VALU op replaces an LDS permute round trip.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, kWave);
  return x;
}

// 16-byte global load / store.
__device__ __forceinline__ uint4 ld16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ void st16(void* p, uint4 v) {
  *reinterpret_cast<uint4*>(p) = v;
}

}  // namespace pa
