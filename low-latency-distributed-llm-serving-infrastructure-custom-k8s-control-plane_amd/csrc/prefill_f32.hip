// Causal chunked prefill over an fp32 paged cache, on the matrix cores.
//
// Masking follows the reference's block-diagonal causal mask
// (app/model/paged_attention.py:92-118 applied by SDPA,
// paged_attention.py:170-178): query token j of a sequence at position
// start + j attends context positions [0, start + j].  Context positions in
// a block outside the pool, and every position of a sequence whose table
// row is outside the table, take no weight.
//
#include <algorithm>

#include "pa_common.hpp"
#include "pa_launch.hpp"
#include "prefill_common.hpp"

namespace pa {

// Units and rows are those of the 16-bit kernel: a unit is (sequence, query
// tile, KV head, sub-group) and its 128 query rows are tile tokens x G query
// heads (row r = g * MTOK + tok).  The products run on
// v_mfma_f32_32x32x2_f32 (four fp32 products per lane per MFMA; fp32
// accumulation).  One workgroup of 8 waves per CU walks its share of the
// units (snake order over the units from the highest item down, as the
// 16-bit kernel).  Wave w owns query rows [32 (w%4), +32) and
// the 32-token half w/4 of every 64-token stage; the two waves of a row
// group merge (max, sum, acc) through LDS at the end.
//
//   S^T[t][row] = sum_d K[t][d] Q[row][d]:  A = K (lane l: token l%32, the
//     head-dim pair 4j + 2(l/32), +1 of an 8-byte LDS read, one per MFMA of
//     a pair), B = Q (the lane's own row, the same pairs, in 64 registers);
//   O^T[d][row] += sum_t V^T[d][t] P^T[t][row]:  the context of MFMA j is
//     taken in the order of the score layout, tokens 8(j/4) + 4(l/32) +
//     j%4, so that B is the lane's own probability s[j] (no repacking) and
//     A is V[that token][32 db + l%32], one 4-byte LDS read.
//
// Both sums run over every element of the head and of the tile, in another
// order than the 16-bit kernel (fp32 rounding, within the 1e-4 parity
// tolerance).  K and V go from HBM straight into LDS (global_load_lds_
// dwordx4) into unpadded rows with XOR-swizzled 16-byte chunks, two stages
// in flight (128 KB for heads of 128), one barrier per stage.  Per 32x32
// tile a wave runs 2 D / 2 MFMAs (64 + 64 for heads of 128) against about 80
// vector instructions of softmax, so the matrix cores set the pace.
constexpr int kFmThreads = 512;  // 4 row groups x 2 context halves
constexpr int kFmRows = 128;     // query rows per unit
constexpr int kFmTile = 32;      // context tokens per wave per stage
constexpr int kFmStage = 2 * kFmTile;

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// APPEND (pa_prefill_append): context positions at or after the chunk's
// start are copied from the step's new rows, and each unit of sub-group 0
// stores its own tile's rows from the stage buffers into the cache while
// each stage is in LDS (their block ids staged in LDS once per unit), so no
// unit reads a row another one writes.
template <int D, bool APPEND>
__global__ __launch_bounds__(kFmThreads) void prefill_f32_mfma_kernel(PrefillArgs a) {
  constexpr int ROWB = D * 4;                  // bytes of a K or V row
  constexpr int CH = D / 4;                    // 16-byte chunks of a row
  constexpr int DB = D / 32;                   // 32-wide d blocks of the output
  constexpr int RPC = kWave / CH;              // rows one copy covers
  constexpr int kWaves = kFmThreads / kWave;
  constexpr int kCopies = kFmStage / RPC / kWaves;  // copies per wave per tensor and stage
  constexpr int TBYTES = kFmStage * ROWB;     // one tensor's rows of a stage
  constexpr int kBufBytes = 2 * TBYTES;        // K, then V
  constexpr int kMerge = DB * 16 + 4;          // floats a lane hands over (acc, m, l, padding)
  static_assert(kCopies >= 1 && kCopies * RPC * kWaves == kFmStage, "stage / copy geometry");
  static_assert(4 * kWave * kMerge * 4 <= 2 * kBufBytes, "the merge fits the stage buffers");

  __shared__ __attribute__((aligned(16))) char s_lds[2 * kBufBytes];
  // Block id of every row of each stage buffer (-1 without a table row),
  // stored by the lanes that copy the row: the masks and the fused write read
  // them here instead of the table.
  __shared__ int32_t s_sid[2][kFmStage];

  const int G = a.group / a.sub_groups;
  const int MTOK = kFmRows / G;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rg = wave & 3;
  const int kh = wave >> 2;
  const int t = lane & 31;
  const int h = lane >> 5;
  const int row = rg * 32 + t;  // this lane's query row of a unit
  const int g = row / MTOK;
  const int tok = row - g * MTOK;
  const int hkv = a.num_kv_heads;
  const int units = hkv * a.sub_groups;
  const int log2_bs = a.log2_block_size;
  const int bs_mask = (1 << log2_bs) - 1;
  const int64_t row_bytes = static_cast<int64_t>(hkv) * ROWB;  // a cache row of one token
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_lds));
  const float scale = a.scale_log2e;
  const int hq = hkv * a.group;
  // Copies: wave w fills rows [8 w, 8 w + 8) of K and of V of a stage, RPC
  // rows per copy; lane i lands at chunk position i % CH of row i / CH and
  // fetches the chunk the swizzle puts there.
  const int crow = lane / CH;
  const int cpos = lane % CH;

  const int U = static_cast<int>(a.num_units);
  const int W = static_cast<int>(gridDim.x);
  const int wg = static_cast<int>(blockIdx.x);
  for (int r = 0;; ++r) {
    const int rank = (r & 1) ? (r + 1) * W - 1 - wg : r * W + wg;
    if (rank >= U) break;
    const int item = (U - 1 - rank) / units;
    const int unit = (U - 1 - rank) - item * units;
    const int kvh = unit / a.sub_groups;
    const int h0 = kvh * a.group + (unit - kvh * a.sub_groups) * G;  // first query head
    const int seq = a.items[2 * item];
    const int qt = a.items[2 * item + 1];
    const int64_t first = a.cu_seqlens[seq];
    const int count = static_cast<int>(a.cu_seqlens[seq + 1] - first);
    const int ctx = a.context_lens[seq];
    const int start = ctx - count;
    const int tok0 = qt * MTOK;
    const int ntok = min(MTOK, count - tok0);
    if (ntok <= 0) continue;  // (the whole workgroup)
    const int64_t trow = a.rows != nullptr ? a.rows[seq] : seq;
    const bool row_ok = trow >= 0 && trow < a.num_table_rows;
    const int32_t* bt = a.block_tables + (row_ok ? trow * a.block_table_stride : 0);
    const int bt_stride = row_ok ? a.block_table_stride : 1;
    const char* kbase = reinterpret_cast<const char*>(a.key_cache) + static_cast<int64_t>(kvh) * ROWB;
    const char* vbase = reinterpret_cast<const char*>(a.value_cache) + static_cast<int64_t>(kvh) * ROWB;
    // APPEND: this KV head's new rows, the row of position p (at or after
    // start) at nk0 + p * nkstride bytes (the host keeps strides below 2^24).
    const char* nk0 = nullptr;
    const char* nv0 = nullptr;
    uint32_t nkstride = 0, nvstride = 0;
    if constexpr (APPEND) {
      nkstride = static_cast<uint32_t>(a.new_key_token_stride * 4);
      nvstride = static_cast<uint32_t>(a.new_value_token_stride * 4);
      nk0 = reinterpret_cast<const char*>(a.new_key) + kvh * a.new_key_head_stride * 4 +
            (first - start) * static_cast<int64_t>(nkstride);
      nv0 = reinterpret_cast<const char*>(a.new_value) + kvh * a.new_value_head_stride * 4 +
            (first - start) * static_cast<int64_t>(nvstride);
    }
    const int kv_end = min(ctx, start + tok0 + ntok);  // exclusive
    // Positions that have a block-table column (the rest are never read).
    const int kv_read = static_cast<int>(
        min(static_cast<int64_t>(kv_end), static_cast<int64_t>(bt_stride) << log2_bs));
    const int kv_last = kv_read - 1;
    const int nstages = (kv_end + kFmStage - 1) / kFmStage;
    const bool live = tok < ntok && g < G;
    const int qpos = start + tok0 + tok;  // causal limit (inclusive)
    const int lim = min(qpos, kv_last);

    // Block ids of the rows this lane copies in stage x; -1 without a row.
    int ids[kCopies];
    auto load_ids = [&](int x) {
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int p = min(x * kFmStage + kWaves * 0 + 8 * wave + c * RPC + crow, kv_last);
        ids[c] = row_ok ? bt[p >> log2_bs] : -1;
      }
    };
    // Copies of stage x into buffer b.  Rows past the readable context
    // re-read its last row and an out-of-pool block reads block 0 (finite
    // values; their scores are masked).  APPEND: rows at or after the
    // chunk's start come from the new rows -- one path per stage (all rows
    // before the chunk, all in it, or the stage that holds its start), as
    // per-lane address selects in every stage spilled registers in the
    // stage loop.
    auto issue_rows = [&](int x, int b, auto src_of) {
      // (the lane's row and chunk are made opaque here, so that the copies'
      // per-lane terms are formed in each stage instead of being hoisted out
      // of the stage loop into registers)
      int cr = crow, cp = cpos;
      asm volatile("" : "+v"(cr), "+v"(cp));
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int R = 8 * wave + c * RPC + cr;
        const int pc = min(x * kFmStage + R, kv_last);
        const int piece = (cp ^ chunk_swizzle<CH>(R)) * 16;
        const uint32_t dst = lds0 + b * kBufBytes + (8 * wave + c * RPC) * ROWB;
        src_of(c, pc, piece, dst);
        if (cp == 0) s_sid[b][R] = ids[c];
      }
    };
    auto from_cache = [&](int c, int pc, int piece, uint32_t dst) {
      const int blk = static_cast<uint32_t>(ids[c]) < static_cast<uint32_t>(a.total_blocks) ? ids[c] : 0;
      const int64_t off = ((static_cast<int64_t>(blk) << log2_bs) + (pc & bs_mask)) * row_bytes + piece;
      dma16(dst, kbase + off);
      dma16(dst + TBYTES, vbase + off);
    };
    auto from_new = [&](int, int pc, int piece, uint32_t dst) {
      const uint64_t p = static_cast<uint32_t>(pc);
      dma16(dst, nk0 + (p * nkstride + piece));
      dma16(dst + TBYTES, nv0 + (p * nvstride + piece));
    };
    auto issue = [&](int x, int b) {
      if (!APPEND || x * kFmStage + kFmStage - 1 < start || kv_last < start) {
        issue_rows(x, b, from_cache);
      } else if (x * kFmStage >= start) {
        issue_rows(x, b, from_new);
      } else {
        issue_rows(x, b, [&](int c, int pc, int piece, uint32_t dst) {
          if (pc < start) from_cache(c, pc, piece, dst);
          else from_new(c, pc, piece, dst);
        });
      }
    };

    // ---- prologue: stage 0's copies, the query row, the table scan --------
    load_ids(0);
    issue(0, 0);
    if (nstages > 1) load_ids(1);
    float2 q[CH];  // the lane's row at head-dim pairs 4 j + 2 h, +1
    {
      const float* qrow = reinterpret_cast<const float*>(a.query) +
                          (first + tok0 + (live ? tok : 0)) * a.q_token_stride +
                          static_cast<int64_t>(h0 + (live ? g : 0)) * a.q_head_stride + 2 * h;
#pragma unroll
      for (int j = 0; j < CH; ++j)
        q[j] = live ? *reinterpret_cast<const float2*>(qrow + 4 * j) : make_float2(0.f, 0.f);
    }
    // APPEND: the unit writes positions [p_beg, p_end) of its tile (sub-group
    // 0 of the KV head, a table row inside the table; positions without a
    // table column are not written).
    const bool writer = APPEND && unit - kvh * a.sub_groups == 0 && row_ok;
    const int p_beg = start + tok0;
    const int p_end = max(p_beg, kv_read);
    // Positions whose block id lies outside the pool are skipped (as in
    // decode): every wave passes over the row's columns (cached reads) and
    // ballots whether there are any; such units take the masked path in
    // every tile.
    bool bad_ids;
    {
      const int ncols = (kv_read + bs_mask) >> log2_bs;
      bool bad = !row_ok;
      for (int col = lane; col < ncols && row_ok; col += kWave)
        bad |= static_cast<uint32_t>(bt[col]) >= static_cast<uint32_t>(a.total_blocks);
      bad_ids = __builtin_amdgcn_ballot_w64(bad) != 0;
    }
    wait_vmcnt<0>();
    __syncthreads();  // stage 0 has landed

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
    float m = kScoreFloor, l = 0.f;  // l: this lane's half of the row sum
    // The tile of a wave's stage: tokens kh * 32 + [0, 32) of the stage.
    const int k_row = kh * kFmTile + t;
    const int k_off = k_row * ROWB + 8 * h;
    const int k_swz = chunk_swizzle<CH>(k_row);

    for (int st = 0; st < nstages; ++st) {
      const int b = st & 1;
      if (st + 1 < nstages) {
        issue(st + 1, b ^ 1);
        if (st + 2 < nstages) load_ids(st + 2);
      }
      const int p0 = st * kFmStage + kh * kFmTile;  // the tile's first position
      if (p0 <= kv_last) {  // (wave-uniform: a tile past the context adds nothing)
        const char* kb = s_lds + b * kBufBytes + k_off;
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.f;
        // K reads one group of kKGroup pairs ahead of their MFMAs (the
        // scheduling barriers keep the compiler from hoisting every read,
        // which needs more registers than a wave has).
        constexpr int kKGroup = 2;
        float2 kc[kKGroup], kn[kKGroup];
#pragma unroll
        for (int u = 0; u < kKGroup; ++u) kc[u] = *reinterpret_cast<const float2*>(kb + ((u ^ k_swz) * 16));
#pragma unroll
        for (int jj = 0; jj < CH / kKGroup; ++jj) {
          if (jj + 1 < CH / kKGroup) {
#pragma unroll
            for (int u = 0; u < kKGroup; ++u)
              kn[u] = *reinterpret_cast<const float2*>(kb + ((((jj + 1) * kKGroup + u) ^ k_swz) * 16));
          }
#pragma unroll
          for (int u = 0; u < kKGroup; ++u) {
            s = mfma_f32(kc[u].x, q[jj * kKGroup + u].x, s);
            s = mfma_f32(kc[u].y, q[jj * kKGroup + u].y, s);
          }
#pragma unroll
          for (int u = 0; u < kKGroup; ++u) kc[u] = kn[u];
          __builtin_amdgcn_sched_barrier(0);
        }
        // Masks: past the row's causal limit or the readable context, or in
        // a block outside the pool (the stage's block id is checked in every
        // tile that takes masks: the diagonal and end tiles, and every tile
        // of a unit with such blocks).  The id test stays unconditional
        // here: gated as `p > lim || (bad_ids && ...)`, this ROCm's hipcc
        // emitted the -INF write on the `p > lim` path only, and positions in
        // out-of-pool blocks kept their scores.
        if (bad_ids || p0 + kFmTile - 1 > min(start + tok0, kv_last)) {
          // (every id read first, then one select per score)
          const int32_t* sid = s_sid[b] + kh * kFmTile + 4 * h;
          int4 idq[4];
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) idq[q4] = *reinterpret_cast<const int4*>(sid + 8 * q4);
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int tt = 8 * (i >> 2) + 4 * h + (i & 3);
            const int4 q = idq[i >> 2];
            const int id = (i & 3) == 0 ? q.x : (i & 3) == 1 ? q.y : (i & 3) == 2 ? q.z : q.w;
            const bool off = (p0 + tt > lim) | (static_cast<uint32_t>(id) >= static_cast<uint32_t>(a.total_blocks));
            s[i] = off ? -INFINITY : s[i];
          }
        }
        float tmax = s[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
        tmax = max_halves(tmax);
        // Lazy rescale: the reference maximum moves only when a tile's
        // maximum exceeds it by more than kLazyRescale (log2 units).
        const bool grow = (tmax - m) * scale > kLazyRescale;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          const float m_new = grow ? tmax : m;
          const float alpha = fast_exp2((m - m_new) * scale);
          l *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[db][i] *= alpha;
          m = m_new;
        }
        const float msc = m * scale;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[i] = fast_exp2(fmaf(s[i], scale, -msc));
          l += s[i];
        }
        const char* vb = s_lds + b * kBufBytes + TBYTES;
        // V^T operand of MFMA j: V[token of score j][32 db + t], read one j ahead.
        auto read_v = [&](int j, float (&v)[DB]) {
          const int R = kh * kFmTile + 8 * (j >> 2) + 4 * h + (j & 3);
          const int sv = chunk_swizzle<CH>(R);
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int d = db * 32 + t;
            v[db] = *reinterpret_cast<const float*>(vb + R * ROWB + (((d >> 2) ^ sv) * 16) + (d & 3) * 4);
          }
        };
        float vc[DB], vn[DB];
        read_v(0, vc);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          if (j + 1 < 16) read_v(j + 1, vn);
#pragma unroll
          for (int db = 0; db < DB; ++db) acc[db] = mfma_f32(vc[db], s[j], acc[db]);
#pragma unroll
          for (int db = 0; db < DB; ++db) vc[db] = vn[db];
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (writer && (st + 1) * kFmStage > p_beg && st * kFmStage < p_end) {
        // This stage's rows of the tile, stored from buffer b (stable until
        // the barrier that ends the stage).  Out-of-pool blocks are skipped.
        const int r0 = max(p_beg - st * kFmStage, 0);
        const int n = (min(p_end - st * kFmStage, kFmStage) - r0) * CH;  // pieces per tensor
        for (int i = tid; i < 2 * n; i += kFmThreads) {
          const bool is_v = i >= n;
          const int k = is_v ? i - n : i;
          const int r = r0 + k / CH;
          const int c = k % CH;
          const int p = st * kFmStage + r;
          const int blk = s_sid[b][r];
          if (static_cast<uint32_t>(blk) < static_cast<uint32_t>(a.total_blocks)) {
            const uint4 v = *reinterpret_cast<const uint4*>(s_lds + b * kBufBytes + (is_v ? TBYTES : 0) + r * ROWB +
                                                            ((c ^ chunk_swizzle<CH>(r)) * 16));
            char* dst = const_cast<char*>(is_v ? vbase : kbase) +
                        ((static_cast<int64_t>(blk) << log2_bs) + (p & bs_mask)) * row_bytes + c * 16;
            st16(dst, v);
          }
        }
      }
      // The next stage's copies have landed and every wave is done with
      // this stage's buffer (the copies after next refill it).
      wait_vmcnt<0>();
      __syncthreads();
    }
    l += __shfl_xor(l, 32, kWave);

    // ---- merge the two context halves of every row group -------------------
    {
      float* region = reinterpret_cast<float*>(s_lds) + (rg * kWave + lane) * kMerge;
      if (kh == 1) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            *reinterpret_cast<float4*>(region + db * 16 + 4 * q4) =
                make_float4(acc[db][4 * q4], acc[db][4 * q4 + 1], acc[db][4 * q4 + 2], acc[db][4 * q4 + 3]);
        *reinterpret_cast<float4*>(region + DB * 16) = make_float4(m, l, 0.f, 0.f);
      }
      __syncthreads();
      if (kh == 0) {
        const float4 ml = *reinterpret_cast<const float4*>(region + DB * 16);
        const float mm = fmaxf(m, ml.x);
        const float a1 = fast_exp2((m - mm) * scale);
        const float a2 = fast_exp2((ml.x - mm) * scale);
        const float lt = l * a1 + ml.y * a2;
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
        float* orow = reinterpret_cast<float*>(a.output) +
                      ((first + tok0 + tok) * hq + h0 + g) * static_cast<int64_t>(D) + 4 * h;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const float4 o2 = *reinterpret_cast<const float4*>(region + db * 16 + 4 * q4);
            const float4 o = make_float4((acc[db][4 * q4] * a1 + o2.x * a2) * inv,
                                         (acc[db][4 * q4 + 1] * a1 + o2.y * a2) * inv,
                                         (acc[db][4 * q4 + 2] * a1 + o2.z * a2) * inv,
                                         (acc[db][4 * q4 + 3] * a1 + o2.w * a2) * inv);
            // elements 32 db + 8 q4 + 4 h .. + 3 of the row
            if (live) *reinterpret_cast<float4*>(orow + db * 32 + 8 * q4) = o;
          }
      }
      // The next unit's copies overwrite the merge scratch.
      __syncthreads();
    }
  }
}

template <int D, bool APPEND>
static hipError_t launch_prefill_f32_mfma(const PrefillArgs& args, int group, int64_t num_items,
                                          hipStream_t s) {
  const int g = group / args.sub_groups;
  if (g < 1 || g > 8) return hipErrorNotSupported;
  PrefillArgs a = args;
  a.num_units = num_items * a.num_kv_heads * a.sub_groups;
  // Unit ranks are 32-bit and a workgroup's ranks reach about twice the count.
  if (a.num_units > (int64_t{1} << 30)) return hipErrorInvalidValue;
  // One workgroup per CU (the stage buffers hold one per CU), each looping
  // over its share of the units; fewer units than CUs run one each.
  const int cus = device_compute_units();
  const int64_t wgs = cus > 0 ? std::min<int64_t>(a.num_units, cus) : a.num_units;
  hipLaunchKernelGGL((prefill_f32_mfma_kernel<D, APPEND>), dim3(static_cast<uint32_t>(wgs)), dim3(kFmThreads), 0, s,
                     a);
  return hipGetLastError();
}

hipError_t launch_prefill_f32(const PrefillArgs& a, int head_dim, int group, int64_t num_items,
                              hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  const bool append = a.new_key != nullptr;
  if (head_dim == 128)
    return append ? launch_prefill_f32_mfma<128, true>(a, group, num_items, stream)
                  : launch_prefill_f32_mfma<128, false>(a, group, num_items, stream);
  if (head_dim == 64)
    return append ? launch_prefill_f32_mfma<64, true>(a, group, num_items, stream)
                  : launch_prefill_f32_mfma<64, false>(a, group, num_items, stream);
  return hipErrorNotSupported;
}

}  // namespace pa
