// Causal chunked prefill for heads of 256 (bf16 / fp16) with gfx950 MFMA tiles.
//
// The kernel for heads of 64-128 (prefill.hip) keeps a 32-row tile's query
// and its accumulator in the VGPRs of two waves per SIMD; at 256 dims that is
// 64 + 128 registers before any operand, and its 64-token K and V stages of
// 512-byte rows would need 256 KB of LDS.  Here one workgroup of 4 waves (one
// per SIMD) takes the same 128 query rows: wave w owns rows
// [32 w, 32 w + 32) over the whole context and the whole head, with its
// accumulator (8 tiles of 32x32 fp32) in AGPRs, so the wave has the 512
// registers of its SIMD.  The context is walked in stages of 32 tokens (one
// MFMA tile), K and V in separate 4-slot LDS rings of 16 KB per stage.
//
// The products, the score layout, the swizzled LDS rows, the transpose read
// of V, the copies (each wave copies 8 rows of a stage: one scalar base when
// they share a block; block ids from an LDS ring that wave 0 fills 8 stages
// ahead), the lazy rescale and the masking follow prefill.hip:
//   S^T[kv][row] = sum_d K[kv][d] Q[row][d]       (16 k-steps of 16)
//   O^T[d][row] += sum_kv V^T[d][kv] P^T[kv][row]  (8 d blocks x 2 k-steps)
// A step: the QK MFMAs of stage st+1 (K read into registers during step
// st-1) beside the exponentials of stage st; then the PV MFMAs of stage st,
// each after its own V^T reads, beside the row maxima of stage st+1 and the
// K reads of stage st+2.  No merge: a wave owns its rows.
//
// Reference: the block-diagonal causal mask of app/model/paged_attention.py:
// 92-118 applied by SDPA (paged_attention.py:170-178); query token j of a
// sequence at position start + j attends context positions [0, start + j].
#include <type_traits>

#include "pa_common.hpp"
#include "pa_launch.hpp"
#include "prefill_common.hpp"

namespace pa {

namespace {

constexpr int kThreads = 256;   // 4 waves, one per SIMD
constexpr int kRows = 128;      // query rows per workgroup
constexpr int kD = 256;
constexpr int kTile = 32;       // context tokens per stage
constexpr int kKS = kD / 16;    // QK k-steps
constexpr int kDB = kD / 32;    // output d blocks
constexpr int kChunks = kD / 8;  // 16-byte pieces per row
constexpr int kRowBytes = kD * 2;
constexpr int kRowsPerDma = kWave / kChunks;        // 2
constexpr int kCopyRows = kTile / 4;                // rows of a stage each wave copies
constexpr int kDmaPerWave = kCopyRows / kRowsPerDma;  // 4 per tensor
constexpr int kRegion = kTile * kRowBytes;          // 16 KB
constexpr int kBufs = 4;
constexpr int kVBase = kBufs * kRegion;
constexpr int kIdBase = 2 * kBufs * kRegion;
constexpr int kIdSlots = 8;
constexpr int kIdSlotBytes = 256;
constexpr int kIdAhead = 8;
constexpr int kLdsBytes = kIdBase + kIdSlots * kIdSlotBytes;

template <typename T, bool LANE_IDS>
__global__ __launch_bounds__(kThreads) void prefill256_kernel(PrefillArgs a) {
  static_assert(Elem<T>::kBytes == 2, "16-bit caches (bf16 or fp16)");
  __shared__ __attribute__((aligned(16))) char s_lds[kLdsBytes];

  const int G = a.group / a.sub_groups;
  const int MTOK = kRows / G;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int hkv = a.num_kv_heads;
  const int64_t blk_id = static_cast<int64_t>(gridDim.x) - 1 - blockIdx.x;
  const int units = hkv * a.sub_groups;
  const int64_t item = blk_id / units;
  const int unit = static_cast<int>(blk_id - item * units);
  const int kvh = unit / a.sub_groups;
  const int h0 = kvh * a.group + (unit - kvh * a.sub_groups) * G;
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
  const uint32_t row_bytes = static_cast<uint32_t>(hkv) * kRowBytes;
  const uint32_t block_bytes = row_bytes << log2_bs;
  const int64_t trow = a.rows != nullptr ? a.rows[seq] : seq;
  const bool row_ok = trow >= 0 && trow < a.num_table_rows;
  const int32_t* bt = row_ok ? a.block_tables + trow * a.block_table_stride : kNoBlockRow;
  global_i32* btg = (global_i32*)(bt);
  const int bt_stride = row_ok ? a.block_table_stride : 1;
  const char* kbase = reinterpret_cast<const char*>(a.key_cache) + kvh * kRowBytes;
  const char* vbase = reinterpret_cast<const char*>(a.value_cache) + kvh * kRowBytes;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_lds));

  const int row = wave * 32 + (lane & 31);
  const int half = lane >> 5;
  const int g = row / MTOK;
  const int tok = row - g * MTOK;
  const bool row_live = tok < ntok && g < G;
  const int qpos = start + tok0 + tok;
  const int h = h0 + g;

  uint4 qreg[kKS];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.query) +
                           (first + tok0 + tok) * a.q_token_stride + h * a.q_head_stride;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks)
      qreg[ks] = row_live ? ld16(qrow + ks * 16 + half * 8) : make_uint4(0, 0, 0, 0);
  }

  const int kv_end = min(ctx, start + tok0 + ntok);
  const int kv_read = static_cast<int>(
      min(static_cast<int64_t>(kv_end), static_cast<int64_t>(bt_stride) << log2_bs));
  const int kv_last = kv_read - 1;
  const int nstages = (kv_end + kTile - 1) / kTile;
  const float scale = a.scale_log2e;
  const int last_col = bt_stride - 1;
  const int ncols = (kv_read + bs_mask) >> log2_bs;
  int scan0 = tid < ncols ? btg[tid] : 0;
  bool bad_ids = false;

  // ---- copies (wave cw copies rows [8 cw, 8 cw + 8) of a stage) ----------------
  const int cw = wave;
  const int delta = lane / kChunks;
  uint32_t chunk_off[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int r = cw * kCopyRows + j * kRowsPerDma + delta;
    chunk_off[j] = static_cast<uint32_t>(((lane % kChunks) ^ chunk_swizzle<kChunks>(r)) * 16);
  }
  uint32_t row_off[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j)
    row_off[j] = __umul24(static_cast<uint32_t>(j * kRowsPerDma + delta), row_bytes) + chunk_off[j];
  const bool one_block = (1 << log2_bs) >= kCopyRows;
  auto valid_block = [&](int b) {
    return static_cast<uint32_t>(b) < static_cast<uint32_t>(a.total_blocks) ? static_cast<uint32_t>(b) : 0u;
  };
  const_i32* btc = (const_i32*)(bt);
  auto col0 = [&](int x) { return min((x * kTile) >> log2_bs, last_col); };
  auto dma_ids = [&](int x) {
    const int c0 = col0(x);
    dma4_s(lds0 + kIdBase + (x & (kIdSlots - 1)) * kIdSlotBytes,
           static_cast<uint32_t>(min(lane, last_col - c0)) * 4u, bt + c0);
  };
  auto ring_id = [&](int x, int p) {
    const int idx = min(max((p >> log2_bs) - col0(x), 0), kWave - 1);
    return *reinterpret_cast<const int*>(s_lds + kIdBase + (x & (kIdSlots - 1)) * kIdSlotBytes + idx * 4);
  };
  const int fast_idx4 = kIdBase + ((cw * kCopyRows) >> log2_bs) * 4;
  auto ring_fast = [&](int x) {
    return *reinterpret_cast<const int*>(s_lds + fast_idx4 + (x & (kIdSlots - 1)) * kIdSlotBytes);
  };
  const int id_last = btc[min(kv_last >> log2_bs, last_col)];
  auto copy_each = [&](int x, uint32_t region, const char* base, auto get_id) {
    const int p0 = x * kTile + cw * kCopyRows;
    const uint32_t dst0 = lds0 + region + cw * kCopyRows * kRowBytes;
    if constexpr (!LANE_IDS) {
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) {
        const int p = p0 + j * kRowsPerDma;
        const int pc = min(p, kv_last);
        const uint32_t bb = valid_block(p <= kv_last ? get_id(j, p) : id_last);
        const char* src = base + (static_cast<uint64_t>(bb) * block_bytes +
                                  static_cast<uint32_t>(pc & bs_mask) * row_bytes);
        const uint32_t voff =
            __umul24(min(static_cast<uint32_t>(delta), static_cast<uint32_t>(kv_last - pc)), row_bytes) +
            chunk_off[j];
        dma16_s(dst0 + j * kRowsPerDma * kRowBytes, voff, src);
      }
    } else {
      // Blocks smaller than a copying wave's rows: each lane's row has its own
      // block, read from the ring for every copy of the tensor first (one
      // wait for all of them, not one per copy).
      int pos[kDmaPerWave], b[kDmaPerWave];
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) {
        pos[j] = min(p0 + j * kRowsPerDma + delta, kv_last);
        b[j] = pos[j] >= x * kTile ? ring_id(x, pos[j]) : id_last;
      }
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j)
        dma16(dst0 + j * kRowsPerDma * kRowBytes,
              base + (static_cast<uint64_t>(valid_block(b[j])) * block_bytes +
                      (static_cast<uint32_t>(pos[j] & bs_mask) * row_bytes + chunk_off[j])));
    }
  };

  auto copy_step = [&](int x, uint32_t region, const char* base, int id_fast) {
    const int p0 = x * kTile + cw * kCopyRows;
    if (!LANE_IDS && one_block && p0 + kCopyRows - 1 <= kv_last) {
      const uint32_t bb = valid_block(__builtin_amdgcn_readfirstlane(id_fast));
      const char* src = base + (static_cast<uint64_t>(bb) * block_bytes +
                                static_cast<uint32_t>(p0 & bs_mask) * row_bytes);
      const uint32_t dst0 = lds0 + region + cw * kCopyRows * kRowBytes;
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) dma16_s(dst0 + j * kRowsPerDma * kRowBytes, row_off[j], src);
    } else {
      copy_each(x, region, base, [&](int, int p) { return __builtin_amdgcn_readfirstlane(ring_id(x, p)); });
    }
  };
  // Block ids of this wave's copies in stages 0-3, all loaded before the
  // first copy: one memory round trip, where loads issued copy by copy were
  // waited for one at a time.
  int first_ids[4][kDmaPerWave];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j)
      first_ids[x][j] = btc[min(x * kTile + cw * kCopyRows + j * kRowsPerDma, kv_last) >> log2_bs];
  auto copy_prologue = [&](int x, uint32_t region, const char* base) {
    copy_each(x, region, base, [&](int j, int) { return first_ids[x][j]; });
  };

  // ---- LDS operands ------------------------------------------------------------
  // K: chunk half + 2 ks of token (lane & 31); the chunks of k-steps 8-15 sit
  // 16 positions after those of 0-7 (the swizzle permutes within 16).
  const int k_row = lane & 31;
  int k_off[kKS / 2];
#pragma unroll
  for (int ks = 0; ks < kKS / 2; ++ks)
    k_off[ks] = k_row * kRowBytes + (((half + 2 * ks) ^ chunk_swizzle<kChunks>(k_row)) * 16);
  // V^T: lane (i of a 16-lane group) addresses token 4 half + i/4 (+ 8 for
  // the second read, + 16 per k-step) and column 16 ((lane >> 4) & 1) +
  // 4 (i & 3) of each 32-wide d block; per (d block, 8-row half) offsets
  // inside slot 0 of the V ring.
  const int li = lane & 15;
  int v_off[kDB][2];
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int r = 4 * half + (li >> 2) + 8 * hi;
      const int col = 16 * ((lane >> 4) & 1) + 4 * (li & 3) + 32 * db;
      v_off[db][hi] = kVBase + r * kRowBytes + (((col >> 3) ^ chunk_swizzle<kChunks>(r)) * 16) + (col & 7) * 2;
    }
  auto read_k = [&](int slot, uint4* ka) {
    const char* buf = s_lds + slot * kRegion;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks)
      ka[ks] = *reinterpret_cast<const uint4*>(buf + k_off[ks & 7] + (ks >> 3) * 256);
  };
  // (rows 16 apart share the swizzle, so a k-step is an immediate offset)
  auto read_vt = [&](int slot, int kk, int db) {
    const char* base = s_lds + slot * kRegion + kk * 16 * kRowBytes;
    const uint2 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(base + v_off[db][0]));
    const uint2 hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(base + v_off[db][1]));
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
  };

  const int kv_lim = min(qpos, kv_last);
  auto mask_tile = [&](int t, f32x16& s) {
    const int lim = kv_lim - (t * kTile + 4 * half);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (8 * (i >> 2) + (i & 3) > lim) s[i] = -INFINITY;
  };
  auto mask_bad = [&](int t, f32x16& s) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kv = t * kTile + 8 * (i >> 2) + 4 * half + (i & 3);
      if (kv <= kv_lim && static_cast<uint32_t>(btg[kv >> log2_bs]) >= static_cast<uint32_t>(a.total_blocks))
        s[i] = -INFINITY;
    }
  };
  auto max3 = [](float x, float y, float z) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(y), "v"(z));
    return r;
  };
  auto tile_max = [&](const f32x16& s) {
    const float a0 = max3(s[0], s[1], s[2]), a1 = max3(s[3], s[4], s[5]), a2 = max3(s[6], s[7], s[8]);
    const float a3 = max3(s[9], s[10], s[11]), a4 = max3(s[12], s[13], s[14]);
    const float b0 = max3(a0, a1, a2), b1 = max3(a3, a4, s[15]);
    return max_halves(max3(b0, b1, b1));
  };

  f32x16 acc[kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m = kScoreFloor, l = 0.f;
  auto rescale = [&](float tmax) {
    const bool grow = (tmax - m) * scale > kLazyRescale;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = grow ? tmax : m;
      const float alpha = fast_exp2((m - m_new) * scale);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[db][i] *= alpha;
      m = m_new;
    }
  };

  // ---- prologue: K of stages 0-2, V of stage 0 and the id ring of stages 0-7
  // landed, then K 3 / V 1 in flight.
  {
    if (wave == 0) {
#pragma unroll
      for (int x = 0; x < kIdAhead; ++x) dma_ids(x);
    }
    if constexpr (LANE_IDS) {
      wait_vmcnt<0>();
      __syncthreads();
    }
#pragma unroll
    for (int x = 0; x < 3; ++x) copy_prologue(x, x * kRegion, kbase);
    copy_prologue(0, kVBase, vbase);
    wait_vmcnt<0>();
  }
  asm volatile("" : "+v"(scan0));
  int bad_local = static_cast<uint32_t>(scan0) >= static_cast<uint32_t>(a.total_blocks) ? 1 : 0;
  for (int c = tid + kThreads; c < ncols; c += kThreads)
    bad_local |= static_cast<uint32_t>(btg[c]) >= static_cast<uint32_t>(a.total_blocks) ? 1 : 0;
  bad_ids = __syncthreads_or(bad_local) != 0;
  const int first_masked = bad_ids ? 0 : min(start + tok0 + 1, kv_read) / kTile;
  copy_prologue(3, 3 * kRegion, kbase);
  copy_prologue(1, kVBase + kRegion, vbase);
  int idk = ring_fast(4), idv = ring_fast(2);
  f32x16 s0, s1;
  uint4 ka[kKS];
  {
#pragma unroll
    for (int i = 0; i < 16; ++i) s0[i] = 0.f;
    read_k(0, ka);
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) s0 = mfma32<T>(ka[ks], qreg[ks], s0);
    read_k(1, ka);
    mask_tile(0, s0);
    rescale(tile_max(s0));
  }
  stage_barrier();

  constexpr uint32_t kOnes = Elem<T>::kDtype == PA_DTYPE_BF16 ? 0x3F803F80u : 0x3C003C00u;

  auto step = [&](int st, f32x16& s_cur, f32x16& s_nxt, auto masked, auto slot_c) {
    constexpr bool MASKED = decltype(masked)::value;
    constexpr int SLOT = decltype(slot_c)::value;
    copy_step(st + 4, SLOT * kRegion, kbase, idk);
    if (bad_ids) mask_bad(st, s_cur);

    // ---- A: S_next = K_next Q^T | P = exp2(S - m)
    const float msc = m * scale;
    f32x16 sn;
#pragma unroll
    for (int i = 0; i < 16; ++i) sn[i] = 0.f;
    uint4 pb[2];
    float rsum0 = 0.f, rsum1 = 0.f;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      sn = mfma32<T>(ka[ks], qreg[ks], sn);
      s_cur[ks] = fast_exp2(fmaf(s_cur[ks], scale, -msc));
      if (ks % 8 == 7) {
        const int c = ks / 8;
        pb[c].x = pack_half2<T>(s_cur[8 * c + 0], s_cur[8 * c + 1]);
        pb[c].y = pack_half2<T>(s_cur[8 * c + 2], s_cur[8 * c + 3]);
        pb[c].z = pack_half2<T>(s_cur[8 * c + 4], s_cur[8 * c + 5]);
        pb[c].w = pack_half2<T>(s_cur[8 * c + 6], s_cur[8 * c + 7]);
        rsum0 = dot2_half<T>(pb[c].x, kOnes, rsum0);
        rsum1 = dot2_half<T>(pb[c].y, kOnes, rsum1);
        rsum0 = dot2_half<T>(pb[c].z, kOnes, rsum0);
        rsum1 = dot2_half<T>(pb[c].w, kOnes, rsum1);
      }
    }
    // ---- B: O^T += V^T P^T (V^T read per d block) | row maxima | K reads of st+2
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) acc[db] = mfma32<T>(read_vt(SLOT, kk, db), pb[kk], acc[db]);
    read_k((SLOT + 2) & (kBufs - 1), ka);
    if constexpr (MASKED) mask_tile(st + 1, sn);
    const float tmax = tile_max(sn);
    l += rsum0 + rsum1;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 3, 0);
    }
#pragma unroll
    for (int i = 0; i < 2 * kDB; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 1, 0);
    }
    rescale(tmax);
    s_nxt = sn;
    copy_step(st + 2, kVBase + ((SLOT + 2) & (kBufs - 1)) * kRegion, vbase, idv);
    if (wave == 0) dma_ids(st + kIdAhead);
    idk = ring_fast(st + 5);
    idv = ring_fast(st + 3);
    if (wave == 0) wait_vmcnt<2 * kDmaPerWave + 1>();
    else wait_vmcnt<2 * kDmaPerWave>();
    stage_barrier();
  };

  using U = std::false_type;
  using M = std::true_type;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  const int n_main = min(max(first_masked - 1, 0), nstages);
  int st = 0;
  for (; st + 3 < n_main; st += 4) {
    step(st, s0, s1, U{}, S0{});
    step(st + 1, s1, s0, U{}, S1{});
    step(st + 2, s0, s1, U{}, S2{});
    step(st + 3, s1, s0, U{}, S3{});
  }
  while (st < nstages) {
    step(st, s0, s1, M{}, S0{});
    if (++st == nstages) break;
    step(st, s1, s0, M{}, S1{});
    if (++st == nstages) break;
    step(st, s0, s1, M{}, S2{});
    if (++st == nstages) break;
    step(st, s1, s0, M{}, S3{});
    ++st;
  }
  wait_vmcnt<0>();
  l += __shfl_xor(l, 32, kWave);

  if (!row_live) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = reinterpret_cast<uint16_t*>(a.output) +
                   ((first + tok0 + tok) * (hkv * a.group) + h) * static_cast<int64_t>(kD);
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = db * 32 + 8 * q4 + 4 * half;
      uint2 w;
      w.x = pack_half2<T>(acc[db][4 * q4 + 0] * inv, acc[db][4 * q4 + 1] * inv);
      w.y = pack_half2<T>(acc[db][4 * q4 + 2] * inv, acc[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = w;
    }
}

template <typename T>
hipError_t launch_t(const PrefillArgs& a, int64_t num_items, hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(num_items * a.num_kv_heads * a.sub_groups));
  if ((1 << a.log2_block_size) >= kRowsPerDma)
    hipLaunchKernelGGL((prefill256_kernel<T, false>), grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((prefill256_kernel<T, true>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill256(const PrefillArgs& a, int dtype, int group, int64_t num_items, hipStream_t stream) {
  const int g = group / a.sub_groups;
  if (g < 1 || g > 8) return hipErrorNotSupported;
  if (dtype == PA_DTYPE_BF16) return launch_t<bf16_t>(a, num_items, stream);
  if (dtype == PA_DTYPE_F16) return launch_t<f16_t>(a, num_items, stream);
  return hipErrorNotSupported;
}

}  // namespace pa
