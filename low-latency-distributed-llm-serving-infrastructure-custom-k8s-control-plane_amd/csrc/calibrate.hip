// Measurement aid (no reference counterpart): the matrix-core rate this
// device sustains, so that an MFMA kernel's utilisation can be read against
// what the part delivers under load as well as against its nominal peak.
//
// Every wave runs two independent chains of v_mfma_f32_32x32x16_bf16 on
// register operands (no memory traffic) with NV independent fp32 FMAs issued
// after each MFMA, and writes one float per lane at the end so the chains
// are kept.  NV = 0 gives the matrix-core rate; NV = 4, 8, 16 show how much
// vector-ALU work the part overlaps with its MFMAs.
//
// The same for HBM: read_rate_kernel streams a buffer once with 16-byte
// non-temporal loads, each workgroup one contiguous range with eight loads
// in flight per thread, and keeps an XOR of what it read (stored only when
// it equals a constant no fill of the buffer produces, so the loads are
// kept and nothing is written).  A read of about the bytes a decode launch
// reads gives the rate the device sustains for that traffic.  Of the
// layouts tried (grid-stride or one range per workgroup, four or eight
// loads in flight, 4-64 workgroups per CU) this one read fastest: 6.99
// TB/s over 1.7 GB and 7.07 TB/s over 8.9 GB at 32-64 workgroups per CU,
// against 5.6-6.9 TB/s for grid-stride.
#include "pa_common.hpp"
#include "pa_error.hpp"
#include "pa_launch.hpp"

namespace pa {

typedef __bf16 bf16x8c __attribute__((ext_vector_type(8)));
typedef float f32x16c __attribute__((ext_vector_type(16)));

constexpr int kCalibrateThreads = 512;

template <int NV>
__global__ __launch_bounds__(kCalibrateThreads) void mfma_rate_kernel(float* out, int iters) {
  f32x16c acc0, acc1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    acc0[i] = 0.f;
    acc1[i] = 0.f;
  }
  bf16x8c a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(1e-3f * static_cast<float>(threadIdx.x + i));
    b[i] = static_cast<__bf16>(2e-3f * static_cast<float>(i) - 1e-3f * static_cast<float>(threadIdx.x));
  }
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = 1e-2f * static_cast<float>(threadIdx.x + i);
  for (int it = 0; it < iters; ++it) {
    acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc0, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < NV; ++v) x[v % 16] = fmaf(x[v % 16], 0.999f, 1e-3f);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc1, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < NV; ++v) x[(v + 8) % 16] = fmaf(x[(v + 8) % 16], 0.999f, 1e-3f);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += acc0[i] + acc1[i] + x[i];
  out[static_cast<int64_t>(blockIdx.x) * kCalibrateThreads + threadIdx.x] = s;
}

constexpr int kReadThreads = 256;

__global__ __launch_bounds__(kReadThreads) void read_rate_kernel(const uint4* __restrict__ p, int64_t n16,
                                                                 uint4* out) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int kInFlight = 8;
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t beg = static_cast<int64_t>(blockIdx.x) * per;
  const int64_t end = beg + per < n16 ? beg + per : n16;
  uint32_t acc = 0;
  int64_t i = beg + threadIdx.x;
  for (; i + (kInFlight - 1) * kReadThreads < end; i += kInFlight * kReadThreads) {
    u32x4 v[kInFlight];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u)
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + i + u * kReadThreads));
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < end; i += kReadThreads) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) out[0] = make_uint4(acc, 0u, 0u, 0u);
}

}  // namespace pa

extern "C" {

int pa_calibrate_read(const void* data, int64_t bytes, void* out, int32_t workgroups, void* stream) {
  if (data == nullptr || out == nullptr || workgroups <= 0 || bytes <= 0 || bytes % 16 != 0 ||
      reinterpret_cast<uintptr_t>(data) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0)
    return pa::set_error(PA_ERR_INVALID_ARGUMENT,
                         "pa_calibrate_read: 16-byte aligned data and out, bytes a positive multiple of 16 and "
                         "workgroups > 0 are required");
  hipLaunchKernelGGL(pa::read_rate_kernel, dim3(static_cast<uint32_t>(workgroups)), dim3(pa::kReadThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(data), bytes / 16,
                     static_cast<uint4*>(out));
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pa::set_error(PA_ERR_LAUNCH, "pa_calibrate_read: %s", hipGetErrorString(e));
  return PA_OK;
}

int64_t pa_calibrate_mfma_flops(int32_t workgroups, int32_t iters) {
  if (workgroups <= 0 || iters <= 0) return 0;
  return static_cast<int64_t>(workgroups) * (pa::kCalibrateThreads / pa::kWave) * iters * 2 * 32768;
}

int pa_calibrate_mfma(float* out, int32_t workgroups, int32_t iters, int32_t valu_per_mfma, void* stream) {
  if (out == nullptr || workgroups <= 0 || iters <= 0)
    return pa::set_error(PA_ERR_INVALID_ARGUMENT, "pa_calibrate_mfma: out, workgroups > 0 and iters > 0 are required");
  const dim3 grid(static_cast<uint32_t>(workgroups)), block(pa::kCalibrateThreads);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (valu_per_mfma) {
    case 0: hipLaunchKernelGGL(pa::mfma_rate_kernel<0>, grid, block, 0, s, out, iters); break;
    case 4: hipLaunchKernelGGL(pa::mfma_rate_kernel<4>, grid, block, 0, s, out, iters); break;
    case 8: hipLaunchKernelGGL(pa::mfma_rate_kernel<8>, grid, block, 0, s, out, iters); break;
    case 16: hipLaunchKernelGGL(pa::mfma_rate_kernel<16>, grid, block, 0, s, out, iters); break;
    default:
      return pa::set_error(PA_ERR_INVALID_ARGUMENT, "pa_calibrate_mfma: valu_per_mfma must be 0, 4, 8 or 16, got %d",
                           valu_per_mfma);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return pa::set_error(PA_ERR_LAUNCH, "pa_calibrate_mfma: %s", hipGetErrorString(e));
  return PA_OK;
}

}  // extern "C"
