// Paged-attention decode for gfx950: one workgroup per
// (sequence, 512-token context partition, KV head), split-K merge after.
//
// Work per workgroup (256 threads = 4 waves), for the H_q/H_kv = G query
// heads that share one KV head, so every K/V row is read from HBM once:
//
//  phase 1 (QK)  tokens are spread over "row groups" of kQkLanes lanes; each
//                lane reads two 16-byte pieces of the token's K row (the two
//                loads of a group cover the row contiguously), dots them with
//                its slice of the G query rows (v_dot2_f32_bf16 for bf16),
//                and a DPP butterfly sums the group.  Scores (log2 domain)
//                go to LDS.
//  phase 2       workgroup max per head, p = exp2(s - max) in place, sums.
//  phase 3 (PV)  each wave streams whole V rows (one row per wave load for
//                256-byte rows), every lane owning a fixed slice of the head
//                dimension for all G heads; waves then add their partial
//                outputs through LDS.
//
// A sequence whose context fits one partition gets its normalised output
// written directly; otherwise (max, sum, unnormalised acc) partials go to
// the workspace and decode_merge_kernel combines them.
//
// The reference computes the same quantity with its CPU loop nest
// (csrc/src/paged_kernels.cpp:49-104) over a flat gather list and dense mask.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kDecodeThreads = 256;
constexpr int kDecodeWaves = kDecodeThreads / kWave;
constexpr int kMaxPartition = PA_DECODE_PARTITION;

template <typename T, int D>
struct DecodeShape {
  static constexpr int kE = Elem<T>::kBytes;
  static constexpr int kRowBytes = D * kE;
  static constexpr int kChunkElems = 16 / kE;           // elements per 16 B
  static constexpr int kQkLanes = kRowBytes / 32;        // lanes per K row
  static constexpr int kQkChunks = 2;                    // 16 B loads per lane
  static constexpr int kQkElems = kQkChunks * kChunkElems;
  static constexpr int kQkGroups = kDecodeThreads / kQkLanes;
  static constexpr int kPvBytes = (kRowBytes / kWave) >= 4 ? (kRowBytes / kWave) : 4;
  static constexpr int kPvLanes = kRowBytes / kPvBytes;  // lanes per V row
  static constexpr int kPvElems = kPvBytes / kE;
  static constexpr int kPvRows = kWave / kPvLanes;       // V rows per wave load
  static_assert(kQkLanes >= 1 && kQkLanes <= 16, "row must be 32..512 bytes");
  static_assert(kPvLanes <= kWave, "V row wider than a wave");
};

// Dot product of one lane's slice of a query row with the matching K slice.
template <typename T, int N>
__device__ __forceinline__ float slice_dot(const uint4 (&q)[N], const uint4 (&k)[N]);

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

template <>
__device__ __forceinline__ float slice_dot<bf16_t, 2>(const uint4 (&q)[2], const uint4 (&k)[2]) {
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q[c].x),
                                          __builtin_bit_cast(bf16x2v, k[c].x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q[c].y),
                                          __builtin_bit_cast(bf16x2v, k[c].y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q[c].z),
                                          __builtin_bit_cast(bf16x2v, k[c].z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q[c].w),
                                          __builtin_bit_cast(bf16x2v, k[c].w), acc, false);
  }
  return acc;
}

template <>
__device__ __forceinline__ float slice_dot<float, 2>(const uint4 (&q)[2], const uint4 (&k)[2]) {
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    acc = fmaf(__uint_as_float(q[c].x), __uint_as_float(k[c].x), acc);
    acc = fmaf(__uint_as_float(q[c].y), __uint_as_float(k[c].y), acc);
    acc = fmaf(__uint_as_float(q[c].z), __uint_as_float(k[c].z), acc);
    acc = fmaf(__uint_as_float(q[c].w), __uint_as_float(k[c].w), acc);
  }
  return acc;
}

// Widen one lane's V slice (kPvBytes bytes) to fp32.
template <typename T, int NB>
struct PvSlice;
template <>
struct PvSlice<bf16_t, 4> {
  using raw = uint32_t;
  static constexpr int kElems = 2;
  __device__ static raw load(const bf16_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
  __device__ static void widen(raw r, float (&v)[2]) {
    v[0] = bf16_lo(r);
    v[1] = bf16_hi(r);
  }
};
template <>
struct PvSlice<bf16_t, 8> {
  using raw = uint2;
  static constexpr int kElems = 4;
  __device__ static raw load(const bf16_t* p) { return *reinterpret_cast<const uint2*>(p); }
  __device__ static void widen(raw r, float (&v)[4]) {
    v[0] = bf16_lo(r.x);
    v[1] = bf16_hi(r.x);
    v[2] = bf16_lo(r.y);
    v[3] = bf16_hi(r.y);
  }
};
template <>
struct PvSlice<float, 4> {
  using raw = uint32_t;
  static constexpr int kElems = 1;
  __device__ static raw load(const float* p) { return *reinterpret_cast<const uint32_t*>(p); }
  __device__ static void widen(raw r, float (&v)[1]) { v[0] = __uint_as_float(r); }
};
template <>
struct PvSlice<float, 8> {
  using raw = uint2;
  static constexpr int kElems = 2;
  __device__ static raw load(const float* p) { return *reinterpret_cast<const uint2*>(p); }
  __device__ static void widen(raw r, float (&v)[2]) {
    v[0] = __uint_as_float(r.x);
    v[1] = __uint_as_float(r.y);
  }
};

template <typename T, int D, int G>
__global__ __launch_bounds__(kDecodeThreads) void decode_partition_kernel(DecodeArgs a) {
  using S = DecodeShape<T, D>;
  using PV = PvSlice<T, S::kPvBytes>;
  constexpr int L = S::kQkLanes;
  constexpr int NG = S::kQkGroups;
  constexpr int CE = S::kChunkElems;
  constexpr int U = 4;   // K rows in flight per group
  constexpr int U3 = 8;  // V loads in flight per wave

  __shared__ float s_logit[kMaxPartition * G];
  __shared__ int s_blk[kMaxPartition + 2];
  __shared__ float s_part[kDecodeWaves][G];
  __shared__ float s_acc[kDecodeWaves][G * D];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int hkv = a.num_kv_heads;
  const int64_t item = blockIdx.x / hkv;
  const int kvh = blockIdx.x - static_cast<int>(item) * hkv;
  const int seq = a.items[2 * item];
  const int part = a.items[2 * item + 1];
  const int ctx = a.context_lens[seq];
  const int p0 = part * a.partition;
  const int n = max(0, min(a.partition, ctx - p0));
  const int64_t qtok = a.cu_seqlens[seq];
  const int log2_bs = a.log2_block_size;
  const int bs_mask = (1 << log2_bs) - 1;
  const int64_t row_stride = static_cast<int64_t>(hkv) * D;
  const T* kbase = reinterpret_cast<const T*>(a.key_cache) + kvh * D;
  const T* vbase = reinterpret_cast<const T*>(a.value_cache) + kvh * D;

  // Block ids covering this partition -> LDS (invalid ids become -1).
  const int first_blk = p0 >> log2_bs;
  const int nblk = n > 0 ? ((p0 + n - 1) >> log2_bs) - first_blk + 1 : 0;
  for (int i = tid; i < nblk; i += kDecodeThreads) {
    const int col = first_blk + i;
    int b = -1;
    if (col < a.block_table_stride) {
      b = a.block_tables[static_cast<int64_t>(seq) * a.block_table_stride + col];
      if (b < 0 || b >= a.total_blocks) b = -1;
    }
    s_blk[i] = b;
  }

  // Query slices for the G heads of this KV head.
  const int lig = tid % L;
  const int grp = tid / L;
  uint4 qv[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const T* qrow = reinterpret_cast<const T*>(a.query) + qtok * a.q_token_stride +
                    static_cast<int64_t>(kvh * G + g) * a.q_head_stride;
    qv[g][0] = ld16(qrow + lig * CE);
    qv[g][1] = ld16(qrow + (L + lig) * CE);
  }
  __syncthreads();

  // ---- phase 1: scores ------------------------------------------------
  float run_max[G];
#pragma unroll
  for (int g = 0; g < G; ++g) run_max[g] = kScoreFloor;
  const float scale = a.scale_log2e;

  for (int t0 = 0; t0 < n; t0 += NG * U) {
    uint4 kb[U][2];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * NG + grp;
      int b = -1;
      if (t < n) b = s_blk[((p0 + t) >> log2_bs) - first_blk];
      ok[u] = b >= 0;
      if (ok[u]) {
        const int64_t slot = (static_cast<int64_t>(b) << log2_bs) | ((p0 + t) & bs_mask);
        const T* row = kbase + slot * row_stride;
        kb[u][0] = ld16(row + lig * CE);
        kb[u][1] = ld16(row + (L + lig) * CE);
      } else {
        kb[u][0] = make_uint4(0, 0, 0, 0);
        kb[u][1] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * NG + grp;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = group_sum<L>(slice_dot<T, 2>(qv[g], kb[u])) * scale;
        if (!ok[u]) s = -INFINITY;
        run_max[g] = fmaxf(run_max[g], s);
        if (lig == 0 && t < n) s_logit[t * G + g] = s;
      }
    }
  }

  // ---- phase 2: softmax over the partition --------------------------
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(run_max[g]);
    if (lane == 0) s_part[wave][g] = m;
  }
  __syncthreads();
  float pmax[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = s_part[0][g];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) m = fmaxf(m, s_part[w][g]);
    pmax[g] = m;
  }
  __syncthreads();  // s_part is reused for the sums below

  // Thread tid always sees head tid % G (G divides the block size).
  float psum = 0.f;
  {
    const int g = tid % G;
    float m = pmax[0];
#pragma unroll
    for (int gg = 1; gg < G; ++gg)
      if (g == gg) m = pmax[gg];
    for (int i = tid; i < n * G; i += kDecodeThreads) {
      const float p = fast_exp2(s_logit[i] - m);
      s_logit[i] = p;
      psum += p;
    }
  }
#pragma unroll
  for (int o = kWave / 2; o >= G; o >>= 1) psum += __shfl_xor(psum, o, kWave);
  if (lane < G) s_part[wave][lane] = psum;
  __syncthreads();
  float lsum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) l += s_part[w][g];
    lsum[g] = l;
  }

  // ---- phase 3: P x V -------------------------------------------------
  constexpr int PE = S::kPvElems;
  constexpr int R = S::kPvRows;
  const int sub = lane / S::kPvLanes;   // V row within a wave load
  const int lp = lane % S::kPvLanes;    // slice of the head dimension
  float acc[G][PE];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < PE; ++e) acc[g][e] = 0.f;

  for (int t0 = 0; t0 < n; t0 += kDecodeWaves * R * U3) {
    typename PV::raw vb[U3];
    bool ok[U3];
#pragma unroll
    for (int u = 0; u < U3; ++u) {
      const int t = t0 + (u * kDecodeWaves + wave) * R + sub;
      int b = -1;
      if (t < n) b = s_blk[((p0 + t) >> log2_bs) - first_blk];
      ok[u] = b >= 0;
      if (ok[u]) {
        const int64_t slot = (static_cast<int64_t>(b) << log2_bs) | ((p0 + t) & bs_mask);
        vb[u] = PV::load(vbase + slot * row_stride + lp * PE);
      } else {
        vb[u] = typename PV::raw{};
      }
    }
#pragma unroll
    for (int u = 0; u < U3; ++u) {
      const int t = t0 + (u * kDecodeWaves + wave) * R + sub;
      if (ok[u]) {
        float v[PE];
        PV::widen(vb[u], v);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float p = s_logit[t * G + g];
#pragma unroll
          for (int e = 0; e < PE; ++e) acc[g][e] = fmaf(p, v[e], acc[g][e]);
        }
      }
    }
  }
  // Rows of one wave load that hold different tokens -> add them up.
#pragma unroll
  for (int o = kWave / 2; o >= S::kPvLanes; o >>= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < PE; ++e) acc[g][e] += __shfl_xor(acc[g][e], o, kWave);
  if (sub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < PE; ++e) s_acc[wave][g * D + lp * PE + e] = acc[g][e];
  }
  __syncthreads();

  const int hq = hkv * G;
  const int nparts = (ctx + a.partition - 1) / a.partition;
  if (nparts <= 1) {
    T* out = reinterpret_cast<T*>(a.output) + (qtok * hq + kvh * G) * D;
    for (int i = tid; i < G * D; i += kDecodeThreads) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < kDecodeWaves; ++w) o += s_acc[w][i];
      const int g = i / D;
      float l = lsum[0];
#pragma unroll
      for (int gg = 1; gg < G; ++gg)
        if (g == gg) l = lsum[gg];
      store_scalar<T>(out + i, l > 0.f ? o / l : 0.f);
    }
  } else {
    float* pacc = a.part_acc + (item * hq + kvh * G) * D;
    for (int i = tid; i < G * D; i += kDecodeThreads) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < kDecodeWaves; ++w) o += s_acc[w][i];
      pacc[i] = o;
    }
    if (tid < G) {
      float m = pmax[0], l = lsum[0];
#pragma unroll
      for (int gg = 1; gg < G; ++gg)
        if (tid == gg) {
          m = pmax[gg];
          l = lsum[gg];
        }
      float* pml = a.part_ml + (item * hq + kvh * G + tid) * 2;
      pml[0] = m;
      pml[1] = l;
    }
  }
}

// Combines the split-K partials of every multi-partition sequence.  One
// workgroup per (first work item of a sequence, KV head); the items of a
// sequence are contiguous in `items` (pa_pack orders them that way).
template <typename T>
__global__ __launch_bounds__(kDecodeThreads) void decode_merge_kernel(DecodeArgs a, int G, int D) {
  const int hkv = a.num_kv_heads;
  const int64_t item = blockIdx.x / hkv;
  const int kvh = blockIdx.x - static_cast<int>(item) * hkv;
  if (a.items[2 * item + 1] != 0) return;
  const int seq = a.items[2 * item];
  const int ctx = a.context_lens[seq];
  int nparts = (ctx + a.partition - 1) / a.partition;
  if (nparts <= 1) return;
  if (item + nparts > a.num_items) nparts = static_cast<int>(a.num_items - item);
  const int hq = hkv * G;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  __shared__ float s_max[64];
  __shared__ float s_inv[64];
  // Per-head global max and normaliser; wave w handles heads w, w+4, ...
  for (int g = wave; g < G; g += kDecodeWaves) {
    const int h = kvh * G + g;
    float m = kScoreFloor;
    for (int p = lane; p < nparts; p += kWave)
      m = fmaxf(m, a.part_ml[((item + p) * hq + h) * 2]);
    m = wave_max(m);
    float l = 0.f;
    for (int p = lane; p < nparts; p += kWave) {
      const float* ml = a.part_ml + ((item + p) * hq + h) * 2;
      l += ml[1] * fast_exp2(ml[0] - m);
    }
    l = wave_sum(l);
    if (lane == 0) {
      s_max[g] = m;
      s_inv[g] = l > 0.f ? 1.f / l : 0.f;
    }
  }
  __syncthreads();
  const int64_t qtok = a.cu_seqlens[seq];
  T* out = reinterpret_cast<T*>(a.output) + (qtok * hq + kvh * G) * D;
  for (int i = tid; i < G * D; i += kDecodeThreads) {
    const int g = i / D;
    const int h = kvh * G + g;
    const float m = s_max[g];
    float o = 0.f;
    for (int p = 0; p < nparts; ++p) {
      const float w = fast_exp2(a.part_ml[((item + p) * hq + h) * 2] - m);
      o = fmaf(a.part_acc[((item + p) * hq + kvh * G) * D + i], w, o);
    }
    store_scalar<T>(out + i, o * s_inv[g]);
  }
}

// ---- host-side dispatch ------------------------------------------------

template <typename T, int D, int G>
static hipError_t launch_decode_t(const DecodeArgs& a, int64_t num_items, hipStream_t stream) {
  const int64_t grid = num_items * a.num_kv_heads;
  hipLaunchKernelGGL((decode_partition_kernel<T, D, G>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kDecodeThreads), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((decode_merge_kernel<T>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kDecodeThreads), 0, stream, a, G, D);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_decode_g(const DecodeArgs& a, int G, int64_t num_items, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode_t<T, D, 1>(a, num_items, s);
    case 2: return launch_decode_t<T, D, 2>(a, num_items, s);
    case 4: return launch_decode_t<T, D, 4>(a, num_items, s);
    case 8: return launch_decode_t<T, D, 8>(a, num_items, s);
    default: return hipErrorNotSupported;
  }
}

bool decode_fast_path_supported(int dtype, int head_dim, int group, int block_size,
                                int partition) {
  if (dtype != PA_DTYPE_F32 && dtype != PA_DTYPE_BF16) return false;
  if (head_dim != 64 && head_dim != 128) return false;
  if (group != 1 && group != 2 && group != 4 && group != 8) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  if (partition <= 0 || partition > kMaxPartition) return false;
  return true;
}

hipError_t launch_decode(const DecodeArgs& a, int dtype, int head_dim, int group,
                         int64_t num_items, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  if (dtype == PA_DTYPE_BF16) {
    if (head_dim == 128) return launch_decode_g<bf16_t, 128>(a, group, num_items, stream);
    if (head_dim == 64) return launch_decode_g<bf16_t, 64>(a, group, num_items, stream);
  } else if (dtype == PA_DTYPE_F32) {
    if (head_dim == 128) return launch_decode_g<float, 128>(a, group, num_items, stream);
    if (head_dim == 64) return launch_decode_g<float, 64>(a, group, num_items, stream);
  }
  return hipErrorNotSupported;
}

}  // namespace pa
