// Paged-attention decode for gfx950: one workgroup per
// (sequence, context partition of up to 4096 tokens, KV head), split-K merge
// after.  For bf16/fp16 with an even KV head count and up to 4 query heads per KV
// head, two adjacent KV heads run as one workgroup that reads each token's
// rows of both heads as one row of twice the length (see PAIR below).
//
// The workgroup (4 waves) serves the G = H_q / H_kv query heads that share
// one KV head, so every K/V row of the partition is read from HBM once
// (groups above 8 run as sub-groups of at most 8 on SHARED instances, whose
// re-reads are ordered to meet in one XCD's L2).  Heads of 64, 128 and 256
// have their own instances; heads of 80 and 96 run those of 128 with the
// pieces past the head masked (DM below).
// The partition is cut into 32-token tiles (16 for groups above 4 and for
// 512-byte rows) dealt round-robin to the waves;
// each wave runs flash-style online softmax over its tiles with no
// workgroup barrier inside the loop:
//
//  K (QK layout)  a "row group" of kL lanes holds one token's K row, each
//                 lane two 16-byte pieces (the group's loads cover the row
//                 contiguously); a wave covers 64 / kL tokens per load.
//                 Dots with the G query slices use v_dot2_f32_bf16 /
//                 v_dot2_f32_f16 (16-bit types) and a DPP butterfly sums
//                 each group; groups of more than half a row group use a
//                 reduce-scatter instead, after which each lane holds one
//                 head's scores (qk_softmax_rs).
//  V (PV layout)  one wave load covers whole V rows (one 256-byte row for
//                 bf16 D=128, 4 bytes per lane), so the row address of a
//                 load is wave-uniform and is formed in scalar registers
//                 from the block id fetched with v_readlane.  Every lane
//                 owns a fixed slice of the head dimension for all G heads.
//  softmax        per tile: wave-wide max per head (DPP + shuffles), rescale
//                 of the running sum / accumulator only when the max moved,
//                 p = exp2(s - max) staged in LDS.  For bf16/fp16 the p of
//                 two tokens are packed as a pair of the cache type and the
//                 PV product uses v_dot2 on the matching V pair (one v_perm_b32 per
//                 two elements); fp32 keeps fp32 FMAs throughout.
//
// At the end the four waves combine (max, sum, acc) through LDS.  A sequence
// whose context fits one partition gets its normalised output directly;
// otherwise the partials go to the workspace and decode_merge_kernel
// combines them.
//
// The reference computes the same quantity with its CPU loop nest
// (csrc/src/paged_kernels.cpp:49-104) over a flat gather list and dense mask.
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

constexpr int kDecodeThreads = 256;
constexpr int kMaxDecodeGroup = 8;  // query heads one unpaired workgroup serves
constexpr int kDecodeWaves = kDecodeThreads / kWave;
// Largest split-K partition (context tokens per workgroup) the kernel takes.
constexpr int kMaxPartition = PA_DECODE_MAX_PARTITION;
#ifndef PA_DECODE_TILE
#define PA_DECODE_TILE 32  // context tokens per wave iteration (at least 2 rows per group)
#endif
#ifndef PA_DECODE_TILE_WIDE
#define PA_DECODE_TILE_WIDE 16  // the same for groups of more than 4 query heads
#endif

// Tuning switches (compile-time; the defaults are the shipped choice).
#ifndef PA_DECODE_NT
#define PA_DECODE_NT 1  // non-temporal K/V loads
#endif
#ifndef PA_DECODE_MIN_WAVES
#define PA_DECODE_MIN_WAVES 4  // occupancy floor per SIMD for groups of up to 4 heads
#endif
// Occupancy floor for a group of G query heads: the register budget of the
// wider groups does not fit four waves per SIMD without spilling.
#ifndef PA_DECODE_MIN_WAVES_WIDE
#define PA_DECODE_MIN_WAVES_WIDE 2  // the same for wider groups or rows
#endif
#ifndef PA_DECODE_MIN_WAVES_PAIR512
#define PA_DECODE_MIN_WAVES_PAIR512 3  // the same for 16-bit rows of 512 bytes (pairs, D 256)
#endif
// GA: query heads whose accumulators one lane holds (G, or G/2 when paired,
// whose rows of up to 512 bytes come in half-length tiles).
#define PA_DECODE_OCCUPANCY(T, D, GA, PAIR)                                                  \
  __attribute__((amdgpu_waves_per_eu(                                                        \
      ((GA) <= 4 && ((PAIR) || sizeof(T) == 2) && (D) * sizeof(T) > 256)                     \
          ? PA_DECODE_MIN_WAVES_PAIR512                                                      \
      : ((GA) <= 4 && ((D) * sizeof(T) <= 256 || (PAIR))) ? PA_DECODE_MIN_WAVES              \
                                                          : PA_DECODE_MIN_WAVES_WIDE)))

typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

// K/V loads.  NT: streaming (non-temporal) loads, for rows no other
// workgroup reads; plain cached loads where sibling workgroups re-read them.
template <typename V, bool NT>
__device__ __forceinline__ V kv_load(const void* p);
template <>
__device__ __forceinline__ uint4 kv_load<uint4, true>(const void* p) {
  const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <>
__device__ __forceinline__ uint2 kv_load<uint2, true>(const void* p) {
  const u32x2v v = __builtin_nontemporal_load(reinterpret_cast<const u32x2v*>(p));
  return make_uint2(v.x, v.y);
}
template <>
__device__ __forceinline__ uint32_t kv_load<uint32_t, true>(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
template <>
__device__ __forceinline__ uint4 kv_load<uint4, false>(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
template <>
__device__ __forceinline__ uint2 kv_load<uint2, false>(const void* p) {
  return *reinterpret_cast<const uint2*>(p);
}
template <>
__device__ __forceinline__ uint32_t kv_load<uint32_t, false>(const void* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

template <typename T, int D, int TILE>
struct DecodeShape {
  static constexpr bool kHalf = Elem<T>::kBytes == 2;  // bf16 or fp16
  static constexpr int kE = Elem<T>::kBytes;
  static constexpr int kRowBytes = D * kE;
  // QK layout
  static constexpr int kChunkElems = 16 / kE;  // elements per 16-byte piece
  static constexpr int kL = kRowBytes / 32;    // lanes per K row
  static constexpr int kGpw = kWave / kL;      // K rows per wave load
  static constexpr int kTile = TILE >= 2 * kGpw ? TILE : 2 * kGpw;
  static constexpr int kLog2Gpw = kGpw == 4 ? 2 : kGpw == 8 ? 3 : kGpw == 16 ? 4 : kGpw == 32 ? 5 : 6;
  static constexpr int kTpg = kTile / kGpw;    // tile tokens per row group
  // PV layout
  static constexpr int kPvBytes = (kRowBytes / kWave) >= 4 ? (kRowBytes / kWave) : 4;
  static constexpr int kLp = kRowBytes / kPvBytes;  // lanes per V row
  static constexpr int kR = kWave / kLp;            // V rows per wave load
  static constexpr int kPe = kPvBytes / kE;         // elements per lane
  static constexpr int kRows = kTile / kR;          // V loads per lane per tile
  static_assert(kL >= 1 && kL <= 16, "row must be 32..512 bytes");
  static_assert(kTpg >= 2 && kTpg % 2 == 0, "token pairs need an even count per group");
  static_assert(kGpw % kR == 0, "pair partner must sit in the same lane");
};

template <int NB>
struct VRaw;
template <>
struct VRaw<4> {
  using type = uint32_t;
};
template <>
struct VRaw<8> {
  using type = uint2;
};

// Dot product of one 16-byte piece of K with the matching piece of q
// (16-bit elements).
template <typename T>
__device__ __forceinline__ float piece_dot(uint4 q, uint4 k) {
  static_assert(Elem<T>::kBytes == 2, "paired heads have 16-bit elements");
  float acc = dot2_half<T>(q.x, k.x, 0.f);
  acc = dot2_half<T>(q.y, k.y, acc);
  acc = dot2_half<T>(q.z, k.z, acc);
  return dot2_half<T>(q.w, k.w, acc);
}

// 32-bit word w of a lane's V piece (a pair of 16-bit elements).
__device__ __forceinline__ uint32_t v_word(uint32_t v, int) { return v; }
__device__ __forceinline__ uint32_t v_word(uint2 v, int w) { return w == 0 ? v.x : v.y; }

// Dot product of one lane's K slice (two 16-byte pieces) with its q slice.
template <typename T>
__device__ __forceinline__ float slice_dot(const uint4 (&q)[2], const uint4 (&k)[2]) {
  float acc = 0.f;
  if constexpr (Elem<T>::kBytes == 2) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      acc = dot2_half<T>(q[c].x, k[c].x, acc);
      acc = dot2_half<T>(q[c].y, k[c].y, acc);
      acc = dot2_half<T>(q[c].z, k[c].z, acc);
      acc = dot2_half<T>(q[c].w, k[c].w, acc);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      acc = fmaf(__uint_as_float(q[c].x), __uint_as_float(k[c].x), acc);
      acc = fmaf(__uint_as_float(q[c].y), __uint_as_float(k[c].y), acc);
      acc = fmaf(__uint_as_float(q[c].z), __uint_as_float(k[c].z), acc);
      acc = fmaf(__uint_as_float(q[c].w), __uint_as_float(k[c].w), acc);
    }
  }
  return acc;
}

// Max over the lanes of a wave that share (lane % L): every row group.
// gfx950 v_permlane16_swap / v_permlane32_swap with both operands = x:
// element 0 holds rows {0,0,2,2} (halves {0,0}) and element 1 rows {1,1,3,3}
// (halves {1,1}) of the 16-lane rows, so their max pairs rows (0,1),(2,3)
// (resp. the two 32-lane halves).
__device__ __forceinline__ float max_row_pairs(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Every step pairs lanes of equal (lane % L) only (rotations by multiples of
// L within a row of 16, then the row and half swaps), so the lanes of one
// row group may hold different values (the reduce-scatter score layout).
template <int L>
__device__ __forceinline__ float across_groups_max(float x) {
  if constexpr (L <= 1) x = fmaxf(x, dpp<kDppRowRor1>(x));
  if constexpr (L <= 2) x = fmaxf(x, dpp<kDppRowRor2>(x));
  if constexpr (L <= 4) x = fmaxf(x, dpp<kDppRowRor4>(x));
  if constexpr (L <= 8) x = fmaxf(x, dpp<kDppRowRor8>(x));
  if constexpr (L <= 16) x = max_row_pairs(x);
  return max_halves(x);
}

// K output elements of one head of a multi-partition sequence from its
// split-K partials: ml addresses the head's (max, sum) pair in item 0, acc
// the first element's accumulator and out its output; element k sits
// k * estride elements further.  Partitions 0 .. nfull-1 are items first ..
// first + nfull - 1, partition nfull (when nparts > nfull) is item rem;
// ml_stride / stride step one item.  kMergeBatch partitions per round trip,
// with a running maximum (the stored maxima are already in the exp2
// domain); slots past the last partition read the first one again and get
// no weight.  The elements share each partial's (max, sum), loaded once for
// all of them, and their loads go out together: one round trip per batch
// for the K elements (one after the other, eight heads of 128 took four).
// Each element's arithmetic is the same whatever K, and both merge paths
// (the merge kernel, K = 1, and the in-launch merge of the partition
// kernel) run this, so they give the same bits.
constexpr int kMergeBatch = 8;
constexpr int kMergeOutputs = 4;  // elements a thread of the in-launch merge merges at once

// Partials read by the in-launch merge are written by workgroups on other
// XCDs in the same launch: they are stored and loaded as device-scope
// relaxed atomics, which write through and read past the XCD's L2, so no
// L2 write-back or invalidate is needed (see the partition kernel's tail).
__device__ __forceinline__ void store_device(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_device(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T, int K, bool DEVICE_LOADS = false>
__device__ __forceinline__ void merge_partials(const float* ml, const float* acc, int estride, int64_t ml_stride,
                                               int64_t stride, int64_t first, int nfull, int64_t rem, int nparts,
                                               T* out) {
  auto item_of = [&](int p) -> int64_t { return p < nfull ? first + p : rem; };
  auto ld = [&](const float* q) { return DEVICE_LOADS ? load_device(q) : *q; };
  float mx = kScoreFloor, sum = 0.f, o[K];
#pragma unroll
  for (int k = 0; k < K; ++k) o[k] = 0.f;
  for (int p = 0; p < nparts; p += kMergeBatch) {
    float mp[kMergeBatch], lp[kMergeBatch], xp[kMergeBatch][K];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const int64_t it = item_of(p + u < nparts ? p + u : 0);
      mp[u] = ld(ml + it * ml_stride);
      lp[u] = ld(ml + it * ml_stride + 1);
#pragma unroll
      for (int k = 0; k < K; ++k) xp[u][k] = ld(acc + it * stride + k * estride);
    }
    float mn = mx;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      if (u > 0 && p + u >= nparts) {
        mp[u] = kScoreFloor;
        lp[u] = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) xp[u][k] = 0.f;
      }
      mn = fmaxf(mn, mp[u]);
    }
    const float r = fast_exp2(mx - mn);
    sum *= r;
#pragma unroll
    for (int k = 0; k < K; ++k) o[k] *= r;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const float w = fast_exp2(mp[u] - mn);
      sum = fmaf(lp[u], w, sum);
#pragma unroll
      for (int k = 0; k < K; ++k) o[k] = fmaf(xp[u][k], w, o[k]);
    }
    mx = mn;
  }
#pragma unroll
  for (int k = 0; k < K; ++k) store_scalar<T>(out + k * estride, sum > 0.f ? o[k] / sum : 0.f);
}

// PAIR: two adjacent real KV heads of D/2 run as one head of D with the G
// query heads of both (the first G/2 belong to the first real head); every
// query head reads only its own real head's half of the rows.  QK layout:
//  - rows of 512 bytes ("split"): the first half of a row group's lanes holds
//    the first real head's half of the row (two pieces per lane, as for an
//    unpaired row), the second half the other's; a lane scores the G/2 heads
//    of its own real head, summed over L/2 lanes.
//  - rows of 256 bytes: every lane's first piece lies in the first real
//    head's half and its second piece in the other's (so each wave load still
//    reads 128-byte runs); each head dots its own piece, summed over L lanes.
// PV layout: lanes [0, 32) hold the first half of the row, and each lane
// accumulates only the G/2 heads of its half.
// SHARED: the workgroup is one of several sub-groups of a KV head's query
// heads, whose siblings read the same K/V rows (cached loads).
// DM: the head dim in memory, when smaller than the lane layout's D (heads
// of 80 and 96 on the layout of 128, in every dtype).  Lanes whose K pieces or V slice lie
// past DM read the row's first piece or slice instead (always in bounds);
// their q pieces are zero, so those K pieces add nothing to the scores, and
// their accumulators are never stored.
template <typename T, int D, int G, bool PAIR, bool SHARED, int DM>
__global__ __launch_bounds__(kDecodeThreads) PA_DECODE_OCCUPANCY(T, D, (PAIR ? G / 2 : G), PAIR) void decode_partition_kernel(DecodeArgs a) {
  // Tiles of 16 tokens for wide groups and for 16-bit rows of 512 bytes
  // (pairs of heads of 128, heads of 256: the same bytes per tile as 32
  // tokens of 256-byte rows).
  using S = DecodeShape<T, D,
                        ((G > 4 || (Elem<T>::kBytes == 2 && D * sizeof(T) > 256)) ? PA_DECODE_TILE_WIDE
                                                                                   : PA_DECODE_TILE)>;
  using VR = typename VRaw<S::kPvBytes>::type;
  // Nontemporal K/V loads, except where other workgroups re-read the same
  // lines: sibling sub-groups (SHARED), and the rows of heads of 80 and 96,
  // whose 128-byte lines straddle two KV heads.
  constexpr bool kNt = PA_DECODE_NT && !SHARED && DM == D;
  constexpr int L = S::kL;
  constexpr int GPW = S::kGpw;
  constexpr int TPG = S::kTpg;
  constexpr int CE = S::kChunkElems;
  constexpr int PE = S::kPe;
  constexpr int R = S::kR;
  constexpr int ROWS = S::kRows;
  constexpr bool HALF = S::kHalf;  // 16-bit elements (bf16 or fp16)
  // p staging per wave: 16-bit pairs [16 pairs][G] or fp32 [32 tokens][G]
  constexpr int kTile = S::kTile;
  constexpr int PWORDS = HALF ? (kTile / 2) * G : kTile * G;
  constexpr int GA = PAIR ? G / 2 : G;    // heads a lane accumulates
  constexpr int OUT_D = PAIR ? D / 2 : D;  // s_acc elements per query head
  constexpr bool MASKD = DM < D;
  constexpr int ODM = PAIR ? D / 2 : DM;  // output elements per query head in memory
  constexpr int KPM = DM / S::kChunkElems;  // 16-byte pieces of a row in memory
  static_assert(!MASKD || (!PAIR && DM % S::kChunkElems == 0 && KPM >= S::kL && DM % S::kPe == 0),
                "masked head dims: unpaired, whole 16-byte pieces, at least one piece per lane");
  static_assert(!PAIR || (HALF && G % 2 == 0 && S::kR == 1 && S::kTpg >= 1),
                "pairs: 16-bit elements, an even head count, one V row per wave load");
  // RS: reduce-scatter scores, for unpaired groups of more than half a row
  // group of lanes (L of 4 or 8): NP score positions (G rounded up to a power
  // of two, at least L), and lane lig of every row group ends with the
  // scores of its HPL query heads lig*HPL .. lig*HPL + HPL-1 alone (see
  // qk_softmax_rs).
  constexpr bool RS = !PAIR && (L == 4 || L == 8) && G > L / 2;
  constexpr int NP = !RS ? 1 : (G <= L ? L : 8);
  constexpr int HPL = RS ? NP / L : 1;

  // Block ids of the partition; its tail from kParkStart holds the new
  // token's pieces and their destinations from the staging to the last tile
  // (pa_decode_append): a 16-byte piece and an 8-byte address per lane.
  constexpr int kBlkInts = kMaxPartition + 2;
  constexpr int kParkStart = (kBlkInts - kWave * 6) & ~3;  // 16-byte aligned
  __shared__ __align__(16) int s_blk[kBlkInts];
  __shared__ uint4 s_q[(RS ? NP : G) * D * S::kE / 16];
  __shared__ uint32_t s_p[kDecodeWaves][PWORDS];
  __shared__ float s_m[kDecodeWaves][G];
  __shared__ float s_l[kDecodeWaves][G];
  __shared__ float s_acc[kDecodeWaves][G * OUT_D];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int hkv = a.num_kv_heads;
  // Workgroup -> (item, KV head, sub-group of G of the head's a.group query
  // heads; one sub-group unless a.group exceeds the largest kernel group).
  int64_t item;
  int kvh, sg = 0;
  if (a.sub_groups == 1) {
    item = blockIdx.x / hkv;
    kvh = static_cast<int>(blockIdx.x - item * hkv);
  } else {
    // Sibling sub-groups read the same K/V rows.  Workgroup ids are dealt to
    // the XCDs round-robin, so siblings get ids that are equal modulo the XCD
    // count and close together: the later reads hit that XCD's L2.  Runs of
    // kXcds (item, KV head) units, each run repeated once per sub-group; the
    // last run may be shorter.
    const int64_t span = static_cast<int64_t>(kXcds) * a.sub_groups;
    const int64_t run = blockIdx.x / span;
    const int64_t base = run * kXcds;
    const int width = static_cast<int>(min<int64_t>(kXcds, gridDim.x / a.sub_groups - base));
    const int r = static_cast<int>(blockIdx.x - run * span);
    sg = r / width;
    const int64_t u = base + (r - sg * width);
    item = u / hkv;
    kvh = static_cast<int>(u - item * hkv);
  }
  const int h0 = kvh * a.group + sg * G;  // first query head
  const int seq = a.items[2 * item];
  const int part = a.items[2 * item + 1];
  const int64_t trow = a.rows != nullptr ? a.rows[seq] : seq;
  const bool row_ok = trow >= 0 && trow < a.num_table_rows;
  int ctx = a.context_lens[seq];
  int64_t qtok = a.cu_seqlens[seq];
  const int p0 = part * a.partition;
  const int log2_bs = a.log2_block_size;
  const int bs_mask = (1 << log2_bs) - 1;

  // Block ids covering this partition -> LDS (invalid ids become -1).  The
  // whole partition's span is read, whatever the context length, so that
  // the reads do not wait for it (entries past the context are never used);
  // each thread's first entry is loaded here, beside the context length and
  // the query token, and stored with the first query piece below.
  const int first_blk = p0 >> log2_bs;
  const int nblk = ((p0 + a.partition - 1) >> log2_bs) - first_blk + 1;
  auto table_entry = [&](int i) {
    const int col = first_blk + i;
    return row_ok && col < a.block_table_stride ? a.block_tables[trow * a.block_table_stride + col] : -1;
  };
  auto valid_block = [&](int b) { return b < 0 || b >= a.total_blocks ? -1 : b; };
  const int b0 = tid < nblk ? table_entry(tid) : -1;
  // (both scalar loads issued before either is waited for: one round trip)
  asm volatile("" : "+s"(ctx), "+s"(qtok));
  const int n = max(0, min(a.partition, ctx - p0));
  const int64_t row_stride = static_cast<int64_t>(hkv) * DM;
  const T* kbase = reinterpret_cast<const T*>(a.key_cache) + kvh * DM;
  const T* vbase = reinterpret_cast<const T*>(a.value_cache) + kvh * DM;

  // pa_decode_append: the workgroups of the partition holding the new token
  // (position ctx - 1) write its K and V rows of this unit (one KV head, or
  // the pair's two) into the cache, as pa_reshape_and_cache would; sibling
  // sub-groups write the same bytes.  The wave that attends the partition's
  // last tile (the one holding that position) does it, a lane per 16-byte
  // piece: it loads the piece here, so the load overlaps the staging below,
  // parks it in the tail of s_blk (past the partition's block ids) and
  // stores it in the tile loop just before that tile's loads, with a
  // barrier of the wave between them, which orders the stores before its
  // own reads of that position; no other wave or workgroup of the launch
  // reads it.  (Stored at the top of the launch, the rows were counted by
  // every later wait of the wave's loads.)  When the block ids leave no
  // room (more than kParkStart of them: one-token blocks and a partition
  // above 3712 tokens), the pieces are stored before the staging barrier
  // instead, which orders them before the whole workgroup's reads.
  constexpr int kPieceElems = 16 / static_cast<int>(sizeof(T));
  constexpr int kAppendPieces = DM / kPieceElems;  // 16-byte pieces of the unit's row
  static_assert(2 * kAppendPieces <= kWave, "one piece of K or V per lane of a wave");
  const bool append = a.new_key != nullptr && n > 0 && p0 + n == ctx;
  const int last_tile = (n + S::kTile - 1) / S::kTile - 1;
  const int append_wave = append ? last_tile % kDecodeWaves : -1;
  // Lane l's piece: l < kAppendPieces of K, the rest of V; its element in
  // the token's row, and where it goes given the block b holding ctx - 1.
  auto append_elem = [&](int l) { return kvh * DM + (l >= kAppendPieces ? l - kAppendPieces : l) * kPieceElems; };
  auto append_target = [&](int b, int l) {
    const int64_t slot = (static_cast<int64_t>(b) << log2_bs) + ((ctx - 1) & bs_mask);
    return const_cast<T*>(reinterpret_cast<const T*>(l >= kAppendPieces ? a.value_cache : a.key_cache)) +
           slot * row_stride + append_elem(l);
  };
  T* append_dst = nullptr;
  uint4 append_piece = make_uint4(0, 0, 0, 0);
  if (wave == append_wave && lane < 2 * kAppendPieces) {
    const int col = (ctx - 1) >> log2_bs;
    const int b = row_ok && col < a.block_table_stride ? a.block_tables[trow * a.block_table_stride + col] : -1;
    if (b >= 0 && b < a.total_blocks) {
      const bool is_v = lane >= kAppendPieces;
      const int g = append_elem(lane);  // element in the token's row
      const int h = g / a.head_dim;
      const T* src = reinterpret_cast<const T*>(is_v ? a.new_value : a.new_key) +
                     qtok * (is_v ? a.new_value_token_stride : a.new_key_token_stride) +
                     static_cast<int64_t>(h) * (is_v ? a.new_value_head_stride : a.new_key_head_stride) +
                     (g - h * a.head_dim);
      append_dst = append_target(b, lane);
      append_piece = ld16(src);
    }
  }

  // The G query rows of this KV head -> LDS (read back per tile, one head
  // at a time, so they do not occupy registers across the loop).
  const int lig = lane % L;  // lane within its row group
  const int gi = lane / L;   // row group within the wave
  constexpr int QCHUNKS = G * D / CE;  // 16-byte pieces of the G query rows
  constexpr int HC = D / CE / 2;  // 16-byte pieces of a real head when paired
  constexpr int QN = RS ? 2 * L * NP : QCHUNKS;  // 16-byte pieces staged
  auto query_piece = [&](int i) -> uint4 {
    if constexpr (RS) {
      // Per (position p, lane l) of a row group, the two pieces (l and l + L)
      // lane l dots at position p: those of query head p ^ (l * HPL), zero
      // past G.  A lane's reads for p = 0 .. NP-1 are then one base address
      // plus constants.
      const int piece = i & 1;
      const int ln = (i >> 1) % L;
      const int g = ((i >> 1) / L) ^ (ln * HPL);
      const T* qrow = reinterpret_cast<const T*>(a.query) + qtok * a.q_token_stride +
                      static_cast<int64_t>(h0 + min(g, G - 1)) * a.q_head_stride;
      return (g < G && (!MASKD || ln + piece * L < KPM)) ? ld16(qrow + (ln + piece * L) * CE)
                                                        : make_uint4(0, 0, 0, 0);
    } else {
      const int g = i / (D / CE);
      const int c = i - g * (D / CE);
      const T* qrow = reinterpret_cast<const T*>(a.query) + qtok * a.q_token_stride +
                      static_cast<int64_t>(h0 + g) * a.q_head_stride;
      if constexpr (PAIR) {
        // Query head g belongs to real KV head g / GA of the pair: its D/2
        // elements go into that half of the row (the other half is never read).
        return (c / HC) == (g / GA) ? ld16(qrow + (c % HC) * CE) : make_uint4(0, 0, 0, 0);
      } else {
        return (!MASKD || c < KPM) ? ld16(qrow + c * CE) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  // Each thread's first table entry and first query piece are both loaded
  // before either is stored, so that the two round trips overlap; the rest
  // (partitions of more than kDecodeThreads blocks, more query pieces than
  // threads) follow.
  {
    const uint4 q0 = tid < QN ? query_piece(tid) : make_uint4(0, 0, 0, 0);
    if (tid < nblk) s_blk[tid] = valid_block(b0);
    if (tid < QN) s_q[tid] = q0;
  }
  for (int i = tid + kDecodeThreads; i < nblk; i += kDecodeThreads) s_blk[i] = valid_block(table_entry(i));
  for (int i = tid + kDecodeThreads; i < QN; i += kDecodeThreads) s_q[i] = query_piece(i);
  // The new token's pieces: parked past the block ids with their
  // destinations (null: none), or (no room there) stored now, before the
  // barrier.
  uint4* const park_piece = reinterpret_cast<uint4*>(s_blk + kParkStart);
  T** const park_dst = reinterpret_cast<T**>(s_blk + kParkStart + kWave * 4);
  const bool park = nblk <= kParkStart;
  // Whether the last tile's wave stores parked pieces (the array's last
  // word, past every block id).
  if (tid == 0) s_blk[kBlkInts - 1] = append && park ? 1 : 0;
  if (wave == append_wave && lane < 2 * kAppendPieces) {
    if (park) {
      park_piece[lane] = append_piece;
      park_dst[lane] = append_dst;
    } else if (append_dst != nullptr) {
      st16(append_dst, append_piece);
    }
  }
  __syncthreads();

  const float scale = a.scale_log2e;
  const int sub = lane / S::kLp;  // V row of this lane within a wave load
  const int lp = lane % S::kLp;   // head-dimension slice of this lane
  // Paired: which real head's half of the row the lane's V slice lies in.
  const int hh = PAIR ? lp / (S::kLp / 2) : 0;
  float m[G], acc[GA][PE];
#pragma unroll
  for (int g = 0; g < G; ++g) m[g] = kScoreFloor;
#pragma unroll
  for (int j = 0; j < GA; ++j)
#pragma unroll
    for (int e = 0; e < PE; ++e) acc[j][e] = 0.f;

  // ---- per-tile work ------------------------------------------------------
  // A lane computes the scores of NS query heads, summed over LS lanes: all
  // G over the row group, or, in the split pair layout, the G/2 of its own
  // real head over its half of the group.  Its K pieces are kp0 and
  // kp0 + KP1 (16-byte pieces of the row).
  constexpr bool SPLIT = PAIR && D * sizeof(T) > 256;
  constexpr int NS = SPLIT ? GA : G;
  constexpr int LS = SPLIT ? L / 2 : L;
  constexpr int KP1 = SPLIT ? L / 2 : L;
  const int khalf = SPLIT ? lig / LS : 0;              // real head of the lane's pieces
  const int kp0 = SPLIT ? khalf * L + lig % LS : lig;  // first 16-byte piece of the lane
  const int gq0 = SPLIT ? khalf * GA : 0;              // first query head it scores
  // Softmax exponentials are spread over the LS lanes that share those
  // scores: lane lig owns "combos" k = lig % LS + LS*r, each one (token pair,
  // head) for bf16 or (token, head) for fp32, and computes, sums and stages
  // only those.
  constexpr int NC = (HALF ? TPG / 2 : TPG) * NS;  // combos per lane group
  constexpr int CPL = (NC + LS - 1) / LS;          // combos per lane
  float lsum[NS];  // this lane's share of the softmax denominators of its NS heads
#pragma unroll
  for (int j = 0; j < NS; ++j) lsum[j] = 0.f;
  float ml[HPL];  // RS: running maxima of the lane's own heads (sums in lsum[0 .. HPL-1])
#pragma unroll
  for (int h = 0; h < HPL; ++h) ml[h] = kScoreFloor;

  uint4 kb[TPG][2];
  bool kok[TPG];
  VR vb[ROWS];

  auto tile_blocks = [&](int tile) {
    const int t = tile * kTile + (lane & (kTile - 1));
    return t < n ? s_blk[((p0 + t) >> log2_bs) - first_blk] : -1;
  };
  // Per-lane element offset of its K slice within a wave load: row group gi
  // reads row gi of the load (GPW consecutive tokens).
  const int64_t koff = static_cast<int64_t>(gi) * row_stride + kp0 * CE;
  // Second K piece of the lane (its first piece again past DM).
  const int kp1 = (!MASKD || kp0 + KP1 < KPM) ? kp0 + KP1 : kp0;
  const bool k_uniform = log2_bs >= S::kLog2Gpw;  // a load's GPW tokens share a block
  auto issue_k = [&](int tile, int blk_lane) {
    const int t0 = tile * kTile;
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
      const int t = t0 + gi + GPW * i;
      if (k_uniform) {
        // Block id and row base of the load are wave-uniform (scalar regs).
        // Lanes past the end of the partition still read a row of the same
        // (valid) block; their scores are masked.
        const int b = __builtin_amdgcn_readlane(blk_lane, GPW * i);
        kok[i] = t < n && b >= 0;
        if (b >= 0) {
          const int64_t slot0 =
              (static_cast<int64_t>(b) << log2_bs) | ((p0 + t0 + GPW * i) & bs_mask);
          const T* row = kbase + slot0 * row_stride + koff;
          kb[i][0] = kv_load<uint4, kNt>(row);
          kb[i][1] = kv_load<uint4, kNt>(row + (MASKD ? (kp1 - kp0) * CE : KP1 * CE));
        } else {
          kb[i][0] = make_uint4(0, 0, 0, 0);
          kb[i][1] = make_uint4(0, 0, 0, 0);
        }
      } else {
        int b = -1;
        if (t < n) b = s_blk[((p0 + t) >> log2_bs) - first_blk];
        kok[i] = b >= 0;
        if (kok[i]) {
          const int64_t slot = (static_cast<int64_t>(b) << log2_bs) | ((p0 + t) & bs_mask);
          const T* row = kbase + slot * row_stride;
          kb[i][0] = kv_load<uint4, kNt>(row + kp0 * CE);
          kb[i][1] = kv_load<uint4, kNt>(row + (MASKD ? kp1 : kp0 + KP1) * CE);
        } else {
          kb[i][0] = make_uint4(0, 0, 0, 0);
          kb[i][1] = make_uint4(0, 0, 0, 0);
        }
      }
    }
  };
  // V rows.  Fast path (one V row per wave load, blocks of >= 16 tokens):
  // rows come in runs of 16 consecutive tokens inside one block, so the
  // block lookup and the 64-bit row address are formed once per run in
  // scalar registers and each further row is one scalar pointer increment.
  // Rows past the end of the partition are zeroed (p = 0 must not meet
  // uninitialised cache contents).
  constexpr int kRun = 16;
  const bool v_runs = R == 1 && log2_bs >= 4;
  // Element offset of the lane's V slice (formed at each use: a value kept
  // across the loop costs registers).
  auto v_slice = [&]() -> int {
    if constexpr (MASKD) {
      return lp * PE < DM ? lp * PE : 0;
    } else {
      return lp * PE;
    }
  };
  auto issue_v = [&](int tile, int blk_lane, bool full) {
    const int t0 = tile * kTile;
    if (v_runs) {
#pragma unroll
      for (int run = 0; run < ROWS / kRun; ++run) {
        const int b = __builtin_amdgcn_readlane(blk_lane, run * kRun);
        if (b >= 0) {
          const int64_t slot0 =
              (static_cast<int64_t>(b) << log2_bs) | ((p0 + t0 + run * kRun) & bs_mask);
          const T* rowp = vbase + slot0 * row_stride + v_slice();
          if (full) {
#pragma unroll
            for (int r = 0; r < kRun; ++r) {
              vb[run * kRun + r] = kv_load<VR, kNt>(rowp);
              rowp += row_stride;
            }
          } else {
#pragma unroll
            for (int r = 0; r < kRun; ++r) {
              const int u = run * kRun + r;
              vb[u] = t0 + u < n ? kv_load<VR, kNt>(rowp) : VR{};
              rowp += row_stride;
            }
          }
        } else {
#pragma unroll
          for (int r = 0; r < kRun; ++r) vb[run * kRun + r] = VR{};
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < ROWS; ++u) {
        int b;
        int t;
        if constexpr (R == 1) {
          t = t0 + u;
          b = __builtin_amdgcn_readlane(blk_lane, u);
        } else {
          t = t0 + R * u + sub;
          b = __shfl(blk_lane, R * u + sub, kWave);
        }
        if (b >= 0) {
          const int64_t slot = (static_cast<int64_t>(b) << log2_bs) | ((p0 + t) & bs_mask);
          vb[u] = kv_load<VR, kNt>(vbase + slot * row_stride + v_slice());
        } else {
          vb[u] = VR{};
        }
      }
    }
  };

  // Scores of the loaded K tile, online-softmax update, p -> LDS.
  // Scores stay unscaled (the max commutes with the positive scale); the
  // scale is applied inside the exponent: p = exp2(s * scale - max * scale).
  //
  // RS layout: position p of lane lig dots the query head p ^ (lig * HPL),
  // so after the NP partial dots every lane holds one partial of each head.
  // Halving steps over the row group each add the partner lane's partial of
  // the heads the lane keeps: partners lig ^ 7 (row half-mirror), ^ 2, ^ 1
  // for rows of 8 lanes; lig ^ 2, ^ 1 for rows of 4.  The partner holds head
  // h at position h ^ ((lig ^ c) * HPL), so for a kept position p it is
  // p ^ (c * HPL), in the discarded half.  After the steps (NP - HPL adds
  // instead of log2(L) per head) positions 0 .. HPL-1 of lane lig hold the
  // scores of heads lig*HPL + h.  The tile maxima are then HPL reductions
  // over the row groups, and the lane computes, sums and stages its own
  // heads' exponentials with no selection among heads.
  auto qk_softmax_rs = [&](bool full) {
    float s[TPG][HPL];
    {
      float x[TPG][NP];
      const uint4* sq = s_q + 2 * lig;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const uint4 qg[2] = {sq[2 * L * p], sq[2 * L * p + 1]};
#pragma unroll
        for (int i = 0; i < TPG; ++i) x[i][p] = slice_dot<T>(qg, kb[i]);
      }
#pragma unroll
      for (int i = 0; i < TPG; ++i) {
        if constexpr (L == 8) {
#pragma unroll
          for (int q = 0; q < 4; ++q) x[i][q] += dpp<kDppRowHalfMirror>(x[i][q ^ 7]);
#pragma unroll
          for (int q = 0; q < 2; ++q) x[i][q] += dpp<kDppQuadXor2>(x[i][q ^ 2]);
          x[i][0] += dpp<kDppQuadXor1>(x[i][1]);
        } else if constexpr (NP == 4) {
#pragma unroll
          for (int q = 0; q < 2; ++q) x[i][q] += dpp<kDppQuadXor2>(x[i][q ^ 2]);
          x[i][0] += dpp<kDppQuadXor1>(x[i][1]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) x[i][q] += dpp<kDppQuadXor2>(x[i][q ^ 4]);
#pragma unroll
          for (int q = 0; q < 2; ++q) x[i][q] += dpp<kDppQuadXor1>(x[i][q ^ 2]);
        }
#pragma unroll
        for (int h = 0; h < HPL; ++h) s[i][h] = (full || kok[i]) ? x[i][h] : -INFINITY;
      }
    }
    // Head lig*HPL + h's tile maximum, in every row group; head g's is read
    // from lane g / HPL (row group 0).
    float tm[HPL];
#pragma unroll
    for (int h = 0; h < HPL; ++h) {
      tm[h] = s[0][h];
#pragma unroll
      for (int i = 1; i < TPG; ++i) tm[h] = fmaxf(tm[h], s[i][h]);
      tm[h] = across_groups_max<L>(tm[h]);
    }
    bool moved = false;
    float m_new[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m_new[g] = fmaxf(m[g], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tm[g % HPL]), g / HPL)));
      moved |= m_new[g] != m[g];
    }
    float ml_new[HPL];  // m_new of the lane's heads (those below G)
#pragma unroll
    for (int h = 0; h < HPL; ++h) ml_new[h] = fmaxf(ml[h], tm[h]);
    if (moved) {  // wave-uniform
      float alpha[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        alpha[g] = fast_exp2((m[g] - m_new[g]) * scale);
        m[g] = m_new[g];
      }
#pragma unroll
      for (int h = 0; h < HPL; ++h) lsum[h] *= fast_exp2((ml[h] - ml_new[h]) * scale);
#pragma unroll
      for (int j = 0; j < GA; ++j)
#pragma unroll
        for (int e = 0; e < PE; ++e) acc[j][e] *= alpha[j];
    }
    uint32_t* sp = s_p[wave];
#pragma unroll
    for (int h = 0; h < HPL; ++h) {
      ml[h] = ml_new[h];
      const float mc = -ml[h] * scale;
      const int head = lig * HPL + h;
      if (head < G) {
        if constexpr (HALF) {
#pragma unroll
          for (int k = 0; k < TPG / 2; ++k) {
            const float pa = fast_exp2(fmaf(s[2 * k][h], scale, mc));
            const float pb = fast_exp2(fmaf(s[2 * k + 1][h], scale, mc));
            lsum[h] += pa + pb;
            sp[(k * GPW + gi) * G + head] = pack_half2<T>(pa, pb);
          }
        } else {
#pragma unroll
          for (int i = 0; i < TPG; ++i) {
            const float pa = fast_exp2(fmaf(s[i][h], scale, mc));
            lsum[h] += pa;
            sp[(gi + GPW * i) * G + head] = __float_as_uint(pa);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  auto qk_softmax = [&](bool full) {
    float s[TPG][NS];
    float tmax[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) tmax[j] = -INFINITY;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      uint4 qg[2];
      if constexpr (PAIR && !SPLIT) {
        // Head j's own piece: piece 0 for the first G/2 heads, piece 1 after.
        qg[0] = s_q[j * (D / CE) + (j / GA) * L + lig];
      } else {
        qg[0] = s_q[(gq0 + j) * (D / CE) + kp0];
        qg[1] = s_q[(gq0 + j) * (D / CE) + kp0 + KP1];
      }
#pragma unroll
      for (int i = 0; i < TPG; ++i) {
        float v;
        if constexpr (PAIR && !SPLIT) v = group_sum<L>(piece_dot<T>(qg[0], kb[i][j / GA]));
        else v = group_sum<LS>(slice_dot<T>(qg, kb[i]));
        if (!full) v = kok[i] ? v : -INFINITY;
        s[i][j] = v;
        tmax[j] = fmaxf(tmax[j], v);
      }
    }
    // Tile maxima over the row groups.  In the split pair layout head g's is
    // held by lane 0, or, for the second real head, by lane LS (the first
    // lane of the second half of row group 0).
    bool moved = false;
    float m_new[G];
    float red[NS];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (SPLIT) {
        if (g < GA) red[g] = across_groups_max<L>(tmax[g]);
        m_new[g] = fmaxf(m[g], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(red[g % GA]),
                                                                          g < GA ? 0 : LS)));
      } else {
        m_new[g] = __int_as_float(__builtin_amdgcn_readfirstlane(
            __float_as_int(fmaxf(m[g], across_groups_max<L>(tmax[g])))));
      }
      moved |= m_new[g] != m[g];
    }
    if (moved) {  // wave-uniform
      float alpha[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        alpha[g] = fast_exp2((m[g] - m_new[g]) * scale);
        if constexpr (!SPLIT) lsum[g] *= alpha[g];
        m[g] = m_new[g];
      }
      if constexpr (SPLIT) {
#pragma unroll
        for (int j = 0; j < GA; ++j) lsum[j] *= khalf ? alpha[GA + j] : alpha[j];
      }
#pragma unroll
      for (int j = 0; j < GA; ++j) {
        const float al = PAIR ? (hh ? alpha[GA + j] : alpha[j]) : alpha[j];
#pragma unroll
        for (int e = 0; e < PE; ++e) acc[j][e] *= al;
      }
    }
    float mneg[G];
#pragma unroll
    for (int g = 0; g < G; ++g) mneg[g] = -m[g] * scale;
    uint32_t* sp = s_p[wave];
#pragma unroll
    for (int r = 0; r < CPL; ++r) {
      const int c = (SPLIT ? lig % LS : lig) + LS * r;
      if (NC % LS != 0 && c >= NC) break;
      float sa = -INFINITY, sb = -INFINITY, mc = 0.f;  // mc: -max * scale of the head
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const bool mine = c == cc;
        if constexpr (HALF) {
          sa = mine ? s[2 * (cc / NS)][cc % NS] : sa;
          sb = mine ? s[2 * (cc / NS) + 1][cc % NS] : sb;
        } else {
          sa = mine ? s[cc / NS][cc % NS] : sa;
        }
      }
      const int g = SPLIT ? gq0 + c % NS : c % G;
      const int jl = SPLIT ? c % NS : g;  // its slot in lsum
#pragma unroll
      for (int gg = 0; gg < G; ++gg) mc = g == gg ? mneg[gg] : mc;
      if constexpr (HALF) {
        const float pa = fast_exp2(fmaf(sa, scale, mc));
        const float pb = fast_exp2(fmaf(sb, scale, mc));
#pragma unroll
        for (int gg = 0; gg < NS; ++gg) lsum[gg] += jl == gg ? pa + pb : 0.f;
        sp[((c / NS) * GPW + gi) * G + g] = pack_half2<T>(pa, pb);
      } else {
        const float pa = fast_exp2(fmaf(sa, scale, mc));
#pragma unroll
        for (int gg = 0; gg < NS; ++gg) lsum[gg] += jl == gg ? pa : 0.f;
        sp[(gi + GPW * (c / NS)) * G + g] = __float_as_uint(pa);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // Accumulate P x V of the loaded V tile.
  auto pv = [&]() {
    const uint32_t* sp = s_p[wave];
    if constexpr (HALF) {
      constexpr int PARTNER = GPW / R;  // V load holding token t + GPW
#pragma unroll
      for (int u = 0; u < ROWS; ++u) {
        if (((R * u) % (2 * GPW)) >= GPW) continue;
        const int t = R * u + sub;
        const int pidx = (t / (2 * GPW)) * GPW + (t % GPW);
        uint32_t pw[GA];
#pragma unroll
        for (int j = 0; j < GA; ++j) pw[j] = sp[pidx * G + (PAIR ? hh * GA + j : j)];
#pragma unroll
        for (int w = 0; w < PE / 2; ++w) {
          // Element 2w (lo) and 2w+1 (hi) of tokens t and t + GPW, paired.
          const uint32_t va = v_word(vb[u], w), vbb = v_word(vb[u + PARTNER], w);
          const uint32_t lo = __builtin_amdgcn_perm(vbb, va, 0x05040100u);
          const uint32_t hi = __builtin_amdgcn_perm(vbb, va, 0x07060302u);
#pragma unroll
          for (int j = 0; j < GA; ++j) {
            acc[j][2 * w] = dot2_half<T>(pw[j], lo, acc[j][2 * w]);
            acc[j][2 * w + 1] = dot2_half<T>(pw[j], hi, acc[j][2 * w + 1]);
          }
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < ROWS; ++u) {
        const int t = R * u + sub;
        float v[PE];
        if constexpr (PE == 1) {
          v[0] = __uint_as_float(vb[u]);
        } else {
          v[0] = __uint_as_float(vb[u].x);
          v[1] = __uint_as_float(vb[u].y);
        }
#pragma unroll
        for (int g = 0; g < GA; ++g) {
          const float p = __uint_as_float(sp[t * G + g]);
#pragma unroll
          for (int e = 0; e < PE; ++e) acc[g][e] = fmaf(p, v[e], acc[g][e]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // Each wave walks its tiles: all K and V loads of a tile are issued at
  // the top of the iteration (several waves per SIMD hide the latency; a
  // pipeline carrying the next tile's loads across the loop did not fit the
  // register budget).
  const int ntiles = (n + kTile - 1) / kTile;
  for (int tile = wave; tile < ntiles; tile += kDecodeWaves) {
    if (tile == ntiles - 1) {
      // The new token's parked pieces, stored by the wave that attends the
      // last tile just before its loads.  (The flag and the pieces are read
      // here, with the index made opaque, so that nothing of them is held
      // in registers across the loop.)
      int l = lane, flag = kBlkInts - 1;
      asm volatile("" : "+v"(l), "+v"(flag));
      if (s_blk[flag] != 0) {
        if (l < 2 * kAppendPieces) {
          T* const dst = park_dst[l];
          if (dst != nullptr) st16(dst, park_piece[l]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      }
    }
    const int blk_lane = tile_blocks(tile);
    // Tile fully inside the partition with every block valid: no masking.
    const bool full = (tile + 1) * kTile <= n && __ballot(lane < kTile && blk_lane < 0) == 0;
    issue_k(tile, blk_lane);
    issue_v(tile, blk_lane, full);
    if constexpr (RS) {
      qk_softmax_rs(full);
    } else {
      qk_softmax(full);
    }
    pv();
  }

  // ---- combine the waves -------------------------------------------------
  // Each (token, head) exponential was summed by exactly one lane.
  float ltot[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float l = SPLIT ? (khalf == g / GA ? lsum[g % NS] : 0.f)
              : RS  ? (lig == g / HPL ? lsum[g % HPL] : 0.f)
                    : lsum[g % NS];
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) l += __shfl_xor(l, o, kWave);
    ltot[g] = l;
  }
  // V rows of one wave load that hold different tokens -> add them up.
#pragma unroll
  for (int o = kWave / 2; o >= S::kLp; o >>= 1)
#pragma unroll
    for (int j = 0; j < GA; ++j)
#pragma unroll
      for (int e = 0; e < PE; ++e) acc[j][e] += __shfl_xor(acc[j][e], o, kWave);
  if (sub == 0) {
    // s_acc rows hold OUT_D elements: when paired, the half of the row that
    // belongs to the head's own real KV head (the lane's slice lies in the
    // half of real head hh, whose query heads are hh*GA .. hh*GA + GA-1).
#pragma unroll
    for (int j = 0; j < GA; ++j)
#pragma unroll
      for (int e = 0; e < PE; ++e)
        s_acc[wave][(PAIR ? hh * GA + j : j) * OUT_D + lp * PE - hh * OUT_D + e] = acc[j][e];
  }
  if (lane < G) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (lane == g) {
        s_m[wave][g] = m[g] * scale;
        s_l[wave][g] = ltot[g];
      }
  }
  __syncthreads();

  // Outputs and partials use the real layout [.., H_q, OUT_D]: this
  // workgroup's G query heads are the real heads h0 .. h0 + G-1 (for a pair,
  // those of both of its KV heads).
  const int hq = hkv * a.group;
  const int nparts = (ctx + a.partition - 1) / a.partition;
  float* pacc = a.part_acc + (item * hq + h0) * ODM;
  T* out = reinterpret_cast<T*>(a.output) + (qtok * hq + h0) * ODM;
  for (int i = tid; i < G * ODM; i += kDecodeThreads) {
    const int g = i / ODM;
    const int si = MASKD ? g * OUT_D + (i - g * ODM) : i;  // its s_acc element
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; ++w) mx = fmaxf(mx, s_m[w][g]);
    float o = 0.f, l = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float f = fast_exp2(s_m[w][g] - mx);
      o = fmaf(s_acc[w][si], f, o);
      l = fmaf(s_l[w][g], f, l);
    }
    if (nparts <= 1) {
      store_scalar<T>(out + i, l > 0.f ? o / l : 0.f);
    } else {
      store_device(pacc + i, o);
      if (i % ODM == 0) {
        float* pml = a.part_ml + (item * hq + h0 + g) * 2;
        store_device(pml, mx);
        store_device(pml + 1, l);
      }
    }
  }

  // ---- in-launch split-K merge ---------------------------------------------
  // The last of a sequence's partition workgroups (for this unit and
  // sub-group) to finish merges the sequence's partials; no workgroup waits
  // for another.  The workgroups run on different XCDs, whose L2s are
  // separate: the partials above are device-scope stores (written through
  // past the L2), and every wave waits for its stores to complete before
  // the barrier.  Then one thread adds the workgroup's arrival to the
  // sequence's 64-bit record with one device-scope atomic: bits 0-15 count
  // arrivals, bits 16-39 hold 1 + the item of the partial last partition
  // (added by that workgroup) and bits 40-63 1 + the item of partition 0,
  // the first of the sequence's full partitions, which pa_pack lists as
  // consecutive items (added by that workgroup; the host passes records
  // only for fewer than 65535 items, so every field fits).  The workgroup
  // whose addition brings the count to nparts has every field in the value
  // the atomic returns; it resets the record for the next launch (the
  // records start at zero and every launch leaves them at zero) and merges
  // as the merge kernel does, with device-scope loads that read past its
  // L2.  An agent-scope release or acquire fence here instead writes back or
  // invalidates a whole L2 per workgroup, and made the decode slower than a
  // second launch.
  if (nparts > 1 && n > 0 && a.merge_state != nullptr && seq >= 0 && seq < a.num_seqs) {
    __shared__ int64_t s_merge[3];
    const int nfull = ctx / a.partition;
    const bool has_rem = nfull * a.partition < ctx;
    uint64_t* rec = reinterpret_cast<uint64_t*>(a.merge_state) +
                    ((static_cast<int64_t>(seq) * hkv + kvh) * a.sub_groups + sg);
    uint64_t add = 1;
    if (part == 0) add += static_cast<uint64_t>(item + 1) << 40;
    if (part == nfull) add += static_cast<uint64_t>(item + 1) << 16;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint64_t now = __hip_atomic_fetch_add(rec, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
      const bool last = static_cast<int>(now & 0xffff) == nparts;
      if (last) {
        __hip_atomic_store(rec, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_merge[1] = static_cast<int64_t>(now >> 40) - 1;
        s_merge[2] = static_cast<int64_t>((now >> 16) & 0xffffff) - 1;
      }
      s_merge[0] = last;
    }
    __syncthreads();
    if (s_merge[0]) {
      const int64_t first = s_merge[1];
      const int64_t rem = has_rem ? s_merge[2] : -1;
      const bool ok = first >= 0 && first + nfull <= a.num_items && (!has_rem || (rem >= 0 && rem < a.num_items));
      if (ok) {
        // KC elements of one head per thread, ODM / KC apart, so that the
        // lanes of a wave read consecutive floats of each partial; the
        // thread's group r = tid, tid + 256, ... covers elements j + k *
        // ODM / KC (k < KC) of head r / (ODM / KC), j = r % (ODM / KC).
        // (fp32 heads of 80 and 96 take one at a time, which keeps their
        // occupancy.)
        constexpr int KO = (G * ODM + kDecodeThreads - 1) / kDecodeThreads;
        constexpr int KM = MASKD && sizeof(T) == 4 ? 1 : kMergeOutputs;
        constexpr int KC = KO >= 4 && KM >= 4 ? 4 : KO >= 2 && KM >= 2 ? 2 : 1;
        constexpr int RUN = ODM / KC;  // groups per head
        static_assert(ODM % KC == 0, "a group's elements stay inside one head");
        for (int r = tid; r < G * RUN; r += kDecodeThreads) {
          const int g = r / RUN;
          const int e = g * ODM + (r - g * RUN);
          merge_partials<T, KC, true>(a.part_ml + 2 * (h0 + g), a.part_acc + static_cast<int64_t>(h0) * ODM + e,
                                      RUN, 2 * static_cast<int64_t>(hq), static_cast<int64_t>(hq) * ODM, first,
                                      nfull, rem, nparts, out + e);
        }
      }
    }
  }
}

// Combines the split-K partials (max, sum, unnormalised acc) of one
// multi-partition sequence for the G heads of one KV head.  One workgroup
// per (entry of the merge list, KV head, 256 of the G*D outputs); an entry,
// written by pa_pack, is (first full-partition item, number of full
// partitions, sequence, item of the partial last partition or -1): the full
// partitions of a sequence are contiguous items, its partial one sits among
// the short work at the end.  Every thread owns one output (merge_partials):
// no LDS and no barrier, so the only dependent global round trips are the
// entry and then the partials.  (With several outputs per thread their
// round trips queued one behind the other: eight heads of 128 at partition
// 2048 took 19 us.)
template <typename T>
__global__ __launch_bounds__(kDecodeThreads) void decode_merge_kernel(DecodeArgs a, int G, int D) {
  const int hkv = a.num_kv_heads;
  const int64_t m = blockIdx.x / hkv;
  const int kvh = static_cast<int>(blockIdx.x - m * hkv);
  const int4 e = reinterpret_cast<const int4*>(a.merge_items)[m];
  const int64_t first = e.x;
  const int nfull = static_cast<int>(min(static_cast<int64_t>(e.y), a.num_items - first));
  const bool has_rem = e.w >= 0 && e.w < a.num_items;
  const int nparts = nfull + (has_rem ? 1 : 0);
  if (nfull < 0 || nparts <= 1) return;
  const int hq = hkv * G;
  T* out = reinterpret_cast<T*>(a.output) + (a.cu_seqlens[e.z] * hq + kvh * G) * D;
  const int i = static_cast<int>(blockIdx.y) * kDecodeThreads + static_cast<int>(threadIdx.x);
  if (i >= G * D) return;
  const int h = kvh * G + i / D;
  merge_partials<T, 1>(a.part_ml + 2 * h, a.part_acc + static_cast<int64_t>(kvh) * G * D + i, 0,
                       2 * static_cast<int64_t>(hq), static_cast<int64_t>(hq) * D, first, nfull, has_rem ? e.w : -1,
                       nparts, out + i);
}

// ---- host-side dispatch ------------------------------------------------

// Launches both phases of one kernel instance.  D, G: the kernel's head dim
// and group (twice the real ones when paired).
struct LaunchOp {
  const DecodeArgs& a;
  int64_t num_items;
  int phases;
  hipStream_t stream;
  template <typename T, int D, int G, bool PAIR, bool SHARED, int DM>
  hipError_t run() const {
    const int64_t grid = num_items * a.num_kv_heads * a.sub_groups;
    const int64_t merge_grid = a.num_merge * a.num_kv_heads;
    if (phases & PA_DECODE_PHASE_PARTITIONS) {
      hipLaunchKernelGGL((decode_partition_kernel<T, D, G, PAIR, SHARED, DM>), dim3(static_cast<uint32_t>(grid)),
                         dim3(kDecodeThreads), 0, stream, a);
      const hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (!(phases & PA_DECODE_PHASE_MERGE) || merge_grid <= 0) return hipSuccess;
    // The partition launch merged in place (merge records given).
    if ((phases & PA_DECODE_PHASE_PARTITIONS) && a.merge_state != nullptr) return hipSuccess;
    // Partials are in the real layout: rows of D/2 when paired; all a.group
    // query heads of a KV head (or pair) merge in one workgroup row.
    constexpr int kOutD = PAIR ? D / 2 : DM;
    const int chunks = (a.group * kOutD + kDecodeThreads - 1) / kDecodeThreads;
    hipLaunchKernelGGL((decode_merge_kernel<T>),
                       dim3(static_cast<uint32_t>(merge_grid), static_cast<uint32_t>(chunks)),
                       dim3(kDecodeThreads), 0, stream, a, a.group, kOutD);
    return hipGetLastError();
  }
};

// Resident partition workgroups per CU of one kernel instance.
struct OccupancyOp {
  int* per_cu;
  template <typename T, int D, int G, bool PAIR, bool SHARED, int DM>
  hipError_t run() const {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, decode_partition_kernel<T, D, G, PAIR, SHARED, DM>,
                                                        kDecodeThreads, 0);
  }
};

template <typename T, int D, int G, bool PAIR, bool SHARED, int DM, typename Op>
static hipError_t visit_one(const Op& op) {
  if constexpr (PAIR && G % 2 != 0) {
    return hipErrorNotSupported;  // a pair's group is even
  } else {
    return op.template run<T, D, G, PAIR, SHARED, DM>();
  }
}

template <typename T, int D, bool PAIR, bool SHARED = false, int DM = D, typename Op>
static hipError_t visit_group(int G, const Op& op) {
  switch (G) {
    case 1: return visit_one<T, D, 1, PAIR, SHARED, DM>(op);
    case 2: return visit_one<T, D, 2, PAIR, SHARED, DM>(op);
    case 3: return visit_one<T, D, 3, PAIR, SHARED, DM>(op);
    case 4: return visit_one<T, D, 4, PAIR, SHARED, DM>(op);
    case 5: return visit_one<T, D, 5, PAIR, SHARED, DM>(op);
    case 6: return visit_one<T, D, 6, PAIR, SHARED, DM>(op);
    case 7: return visit_one<T, D, 7, PAIR, SHARED, DM>(op);
    case 8: return visit_one<T, D, 8, PAIR, SHARED, DM>(op);
    default: return hipErrorNotSupported;
  }
}

template <bool SHARED, typename Op>
static hipError_t visit_unpaired(int dtype, int head_dim, int g, const Op& op) {
  if (dtype == PA_DTYPE_BF16) {
    if (head_dim == 128) return visit_group<bf16_t, 128, false, SHARED>(g, op);
    if (head_dim == 64) return visit_group<bf16_t, 64, false, SHARED>(g, op);
    if (head_dim == 256) return visit_group<bf16_t, 256, false, SHARED>(g, op);
    if (head_dim == 96) return visit_group<bf16_t, 128, false, SHARED, 96>(g, op);
    if (head_dim == 80) return visit_group<bf16_t, 128, false, SHARED, 80>(g, op);
  } else if (dtype == PA_DTYPE_F16) {
    if (head_dim == 128) return visit_group<f16_t, 128, false, SHARED>(g, op);
    if (head_dim == 64) return visit_group<f16_t, 64, false, SHARED>(g, op);
    if (head_dim == 256) return visit_group<f16_t, 256, false, SHARED>(g, op);
    if (head_dim == 96) return visit_group<f16_t, 128, false, SHARED, 96>(g, op);
    if (head_dim == 80) return visit_group<f16_t, 128, false, SHARED, 80>(g, op);
  } else if (dtype == PA_DTYPE_F32) {
    if (head_dim == 128) return visit_group<float, 128, false, SHARED>(g, op);
    if (head_dim == 64) return visit_group<float, 64, false, SHARED>(g, op);
    if (head_dim == 96) return visit_group<float, 128, false, SHARED, 96>(g, op);
    if (head_dim == 80) return visit_group<float, 128, false, SHARED, 80>(g, op);
  }
  return hipErrorNotSupported;
}

// The kernel instance of a real shape: paired heads of D run as the
// instance of head dim 2D and group 2G; a group above the largest kernel
// group runs as decode_sub_groups(group) workgroups per KV head, on the
// SHARED instances (cached K/V loads: the siblings' re-reads hit L2).
template <typename Op>
static hipError_t visit_decode(int dtype, int head_dim, int group, bool pair, const Op& op) {
  if (pair) {
    if (group < 1 || group > 4) return hipErrorNotSupported;
    if (dtype == PA_DTYPE_BF16) {
      if (head_dim == 64) return visit_group<bf16_t, 128, true>(2 * group, op);
      if (head_dim == 128) return visit_group<bf16_t, 256, true>(2 * group, op);
    } else if (dtype == PA_DTYPE_F16) {
      if (head_dim == 64) return visit_group<f16_t, 128, true>(2 * group, op);
      if (head_dim == 128) return visit_group<f16_t, 256, true>(2 * group, op);
    }
    return hipErrorNotSupported;
  }
  if (group < 1) return hipErrorNotSupported;
  const int nsub = decode_sub_groups(group);
  return nsub > 1 ? visit_unpaired<true>(dtype, head_dim, group / nsub, op)
                  : visit_unpaired<false>(dtype, head_dim, group, op);
}

// Largest real group run as pairs, per real head dim (bf16 and fp16; 0 = never).
// Kernel time on 256 lognormal contexts (median 1024) with 8 KV heads,
// unpaired -> paired, each at its best partition:
//   D 64:  G 1 0.180 -> 0.141 ms, G 2 0.181 -> 0.140, G 3 0.183 -> 0.147,
//          G 4 0.183 -> 0.149;
//   D 128: G 1 0.267 -> 0.253, G 2 0.267 -> 0.259, G 3 0.269 -> 0.261,
//          G 4 0.271 -> 0.267 (three waves per SIMD: the eight heads' state
//          does not fit the register budget of four without spilling).
#ifndef PA_DECODE_PAIR_MAX_GROUP_D64
#define PA_DECODE_PAIR_MAX_GROUP_D64 4
#endif
#ifndef PA_DECODE_PAIR_MAX_GROUP_D128
#define PA_DECODE_PAIR_MAX_GROUP_D128 4
#endif

bool decode_pairs_heads(int dtype, int head_dim, int num_kv_heads, int group) {
  if ((dtype != PA_DTYPE_BF16 && dtype != PA_DTYPE_F16) || num_kv_heads % 2 != 0 || group < 1)
    return false;
  if (head_dim == 64) return group <= PA_DECODE_PAIR_MAX_GROUP_D64;
  if (head_dim == 128) return group <= PA_DECODE_PAIR_MAX_GROUP_D128;
  return false;
}

int decode_sub_groups(int group) {
  // The fewest equal sub-groups of at most kMaxDecodeGroup query heads.
  int n = (group + kMaxDecodeGroup - 1) / kMaxDecodeGroup;
  while (n < group && group % n != 0) ++n;
  return n > 0 ? n : 1;
}

bool decode_fast_path_supported(int dtype, int head_dim, int group, int block_size,
                                int partition) {
  if (dtype != PA_DTYPE_F32 && dtype != PA_DTYPE_BF16 && dtype != PA_DTYPE_F16) return false;
  // Rows of up to 512 bytes: heads of 64 and 128, and of 256 in 16-bit types;
  // heads of 80 and 96 on the lane layout of 128.
  const bool wide16 = dtype != PA_DTYPE_F32 && head_dim == 256;
  if (head_dim != 64 && head_dim != 128 && head_dim != 80 && head_dim != 96 && !wide16) return false;
  if (group < 1 || group > kMaxDecodeQueryGroup) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  if (partition <= 0 || partition > kMaxPartition || partition % 32 != 0) return false;
  return true;
}

hipError_t launch_decode(const DecodeArgs& a, int dtype, int head_dim, int group,
                         int64_t num_items, int phases, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  return visit_decode(dtype, head_dim, group, a.pair != 0, LaunchOp{a, num_items, phases, stream});
}

hipError_t decode_workgroups_per_cu(int dtype, int head_dim, int group, bool pair, int* per_cu) {
  *per_cu = 0;
  return visit_decode(dtype, head_dim, group, pair, OccupancyOp{per_cu});
}

}  // namespace pa
