// Causal chunked prefill over the paged cache with gfx950 MFMA tiles.
//
// One workgroup (8 waves) per (sequence, query tile, KV head).  The tile
// holds 128 query rows = (128 / G) query tokens x the G query heads that
// share the KV head.  The context is walked in stages of 64 tokens; wave w
// owns rows [32 (w%4), 32 (w%4) + 32) and the 32-token half w/4 of every
// stage, with flash-style online softmax in fp32, so the two waves of a row
// group split the context and merge their partial results through LDS at
// the end (this halves the longest chain of a causal tile).
//
// Both products are computed transposed so that a lane owns one query row:
//   S^T[kv][row] = sum_d K[kv][d] Q[row][d]       (A = K regs, B = Q regs)
//   O^T[d][row] += sum_kv V^T[d][kv] P^T[kv][row]  (A = V^T regs, B = P^T regs)
// with v_mfma_f32_32x32x16_bf16 (or _f16 for fp16 caches).  In the 32x32
// accumulator lane l holds column l % 32 and rows 8*(i/4) + 4*(l/32) + (i%4),
// i = 0..15, so the softmax max/sum of a query row needs only its own 16
// values plus the partner lane l ^ 32, and the probabilities a lane holds
// are the B operand of the PV product with the context index of k-slot j
// being 8*(j/4) + 4*(l/32) + (j%4) inside each 16-token step.
//
// K and V go from HBM straight into LDS with the gfx950 direct loads
// (global_load_lds_dwordx4: lane i's 16 bytes land at M0 + 16 i), into
// unpadded rows whose 16-byte chunks are XOR-swizzled (chunk_swizzle) so that
// the operand reads below are free of bank conflicts.  The V^T operand is
// read with the gfx950 LDS transpose read ds_read_b64_tr_b16: inside each
// group of 16 lanes, lane i receives element j from the 8-byte word
// addressed by lane (i/4 + 4j), element i%4.  Lane i of a group therefore
// addresses V[kv0 + (i/4)][d0 + 4*(i%4)] and receives V[kv0 + j][d0 + i],
// j = 0..3: four context tokens of its own output column.
//
// Copies.  Waves 0-3 copy 16 rows each of every stage.  One copy covers 4
// rows (8 for 64-dim heads) of one cache block, so its source is a scalar
// base (block id, row offset) plus a fixed per-lane offset: no vector
// address arithmetic.  The block ids come from an LDS ring of table entries
// that wave 0 fills eight stages ahead, read one step ahead of their use.
// (Blocks smaller than one copy take the per-lane form of the address.)
// The copies are issued from
// inline assembly and each copying wave waits for its own copies with an
// exact s_waitcnt vmcnt before the barrier that publishes them: the compiler
// would otherwise drain every copy before each LDS read, as it cannot tell
// the buffers apart.
//
// Pipeline (one barrier per stage).  K and V have separate LDS rings: the K
// of stage st+2 is read into registers during step st and consumed by the
// QK MFMAs of step st+1, so every step starts its MFMAs right after the
// barrier; the V of stage st is read during step st.  A step is two phases,
// each interleaved at the instruction level (sched_group_barrier):
//   A: QK MFMAs of stage st+1  |  softmax of stage st (exp2, pack, row sum)
//                              |  V^T reads of stage st
//   B: PV MFMAs of stage st    |  row maxima of stage st+1  |  K reads of st+2
// so each wave alternates matrix and vector work instead of running long
// runs of one kind in lock-step with the other wave of its SIMD.
// The row sum is accumulated from the rounded probabilities the PV product
// uses (v_dot2 against ones), per lane half, and the halves are added once
// at the end.  Masking is applied only to tiles that cross the causal
// diagonal or the end of the context (or to every tile when some block id of
// the sequence lies outside the pool: those positions are skipped, as in
// decode), in a separate loop after the unmasked one, and the accumulator is
// rescaled only when some row's maximum grew by more than 2^8 over the
// reference maximum in use.
//
// Reference: the block-diagonal causal mask of app/model/paged_attention.py:
// 92-118 applied by SDPA (paged_attention.py:170-178); query token j of a
// sequence at position start + j attends context positions [0, start + j].
#include <type_traits>

#include "pa_common.hpp"
#include "pa_launch.hpp"
#include "prefill_common.hpp"

namespace pa {

constexpr int kPrefillThreads = 512;  // 4 row groups x 2 context halves
constexpr int kPrefillRows = 128;  // query rows per workgroup
constexpr int kKvTile = 32;        // context tokens per wave per stage
constexpr int kStage = 2 * kKvTile;  // context tokens per LDS stage
constexpr int kPrefillWaves = kPrefillThreads / 64;
constexpr int kCopyWaves = 4;  // waves 0-3 copy, one per SIMD
constexpr int kCopyRows = kStage / kCopyWaves;  // rows of a stage each copying wave copies
constexpr int kKBufs = 4;  // K ring: read in step st-2, consumed in st-1, refilled in st
constexpr int kVBufs = 4;  // V ring: landed in st-1, read in step st, refilled in st+2
constexpr int kIdSlots = 8;      // block-id ring slots
constexpr int kIdSlotBytes = 256;  // 64 table entries: every column of a stage
constexpr int kIdAhead = 8;      // stages between an id slot's copy and the stage's K copy + 4

// D: the head dim of the LDS rows and MFMA tiles; DM: the head dim in
// memory (80 and 96 run on rows of 128 whose pieces past DM are zero: the
// copies skip them, the query's are zero and the output's are not stored).
template <typename T, int D, int DM, bool LANE_IDS>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(PrefillArgs a) {
  static_assert(Elem<T>::kBytes == 2, "16-bit caches (bf16 or fp16)");
  static_assert(DM <= D && DM % 16 == 0, "memory head dim: a multiple of 16 up to D");
  constexpr bool MASKD = DM < D;
  constexpr int MEM_ROW = DM * 2;         // bytes of a head's row in memory
  constexpr int KS = D / 16;              // MFMA k-steps of QK^T
  constexpr int DB = D / 32;              // 32-wide d blocks of the output
  constexpr int CHUNKS = D / 8;           // 16-byte pieces per row
  constexpr int ROW_BYTES = D * 2;
  constexpr int kRowsPerDma = kWave / CHUNKS;          // rows one wave copy covers
  constexpr int kDmaPerWave = kCopyRows / kRowsPerDma;  // copies per tensor per stage
  constexpr int kRegion = kStage * ROW_BYTES;         // K (or V) rows of a stage
  constexpr int kVBase = kKBufs * kRegion;
  constexpr int kIdBase = (kKBufs + kVBufs) * kRegion;
  constexpr int kLdsBytes = kIdBase + kIdSlots * kIdSlotBytes;
  constexpr int kVReads = 2 * DB * 2;                 // V^T transpose reads per tile
  constexpr int kPerQk = 16 / KS;                     // probabilities per QK k-step
  static_assert(kDmaPerWave >= 1, "stage / wave mismatch");
  static_assert(kLdsBytes >= 4 * (16 * DB + 2) * kWave * 4, "merge scratch must fit");
  static_assert(kVReads % KS == 0, "V^T reads spread over the QK k-steps");

  // K ring, then V ring (rows swizzled); reused for the final merge.
  __shared__ __attribute__((aligned(16))) char s_lds[kLdsBytes];

  const int G = a.group / a.sub_groups;  // query heads of this workgroup
  const int MTOK = kPrefillRows / G;     // query tokens per workgroup
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // Wave-uniform (scalar): branches on it are whole-wave branches, and the
  // copy counts each wave waits on are exact.
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rg = wave & 3;   // row group
  const int kh = wave >> 2;  // context half of every stage
  const int hkv = a.num_kv_heads;
  // Highest item first: the last query tiles of a sequence see the most context.
  const int64_t blk_id = static_cast<int64_t>(gridDim.x) - 1 - blockIdx.x;
  // -> (item, KV head, sub-group of G of the head's a.group query heads).
  const int units = hkv * a.sub_groups;
  const int64_t item = blk_id / units;
  const int unit = static_cast<int>(blk_id - item * units);
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
  if (ntok <= 0) return;
  const int log2_bs = a.log2_block_size;
  const int bs_mask = (1 << log2_bs) - 1;
  // Byte strides of a cache row and a cache block (the host keeps a block
  // under 4 GiB, so a row offset is one 32 x 32 -> 64-bit multiply-add).
  const uint32_t row_bytes = static_cast<uint32_t>(hkv) * MEM_ROW;
  const uint32_t block_bytes = row_bytes << log2_bs;
  const int64_t trow = a.rows != nullptr ? a.rows[seq] : seq;
  const bool row_ok = trow >= 0 && trow < a.num_table_rows;
  const int32_t* bt = row_ok ? a.block_tables + trow * a.block_table_stride : kNoBlockRow;
  const int bt_stride = row_ok ? a.block_table_stride : 1;
  const char* kbase = reinterpret_cast<const char*>(a.key_cache) + kvh * MEM_ROW;
  const char* vbase = reinterpret_cast<const char*>(a.value_cache) + kvh * MEM_ROW;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_lds));

  // This lane's query row.
  const int row = rg * 32 + (lane & 31);
  const int half = lane >> 5;
  const int g = row / MTOK;
  const int tok = row - g * MTOK;
  // Rows past G * MTOK (when G does not divide 128) belong to no head.
  const bool row_live = tok < ntok && g < G;
  const int qpos = start + tok0 + tok;  // causal limit (inclusive)
  const int h = h0 + g;

  uint4 qreg[KS];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.query) +
                           (first + tok0 + tok) * a.q_token_stride + h * a.q_head_stride;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qreg[ks] = row_live && (2 * ks + half) * 8 < DM ? ld16(qrow + ks * 16 + half * 8) : make_uint4(0, 0, 0, 0);
  }

  const int kv_end = min(ctx, start + tok0 + ntok);  // exclusive
  // Positions that have a block-table column (the rest are never read); at
  // least one, as the host passes tables of one column or more.
  const int kv_read = static_cast<int>(
      min(static_cast<int64_t>(kv_end), static_cast<int64_t>(bt_stride) << log2_bs));
  const int kv_last = kv_read - 1;
  const int nstages = (kv_end + kStage - 1) / kStage;
  const float scale = a.scale_log2e;
  const int last_col = bt_stride - 1;
  // Positions whose block id lies outside the pool are skipped, as the
  // decode kernels skip them: one pass over the row's columns tells whether
  // there are any (then every tile takes the masked path below).  Its first
  // load is issued here and checked after the first copies have landed, so
  // the two memory round trips overlap.
  const int ncols = (kv_read + bs_mask) >> log2_bs;
  int scan0 = tid < ncols ? bt[tid] : 0;
  bool bad_ids = false;  // set once the scan is complete (before any tile is masked)

  // ---- copies ----------------------------------------------------------------
  // Wave cw < 4 copies rows [16 cw, 16 cw + 16) of a stage, kRowsPerDma rows
  // per copy: lane -> row delta = lane / CHUNKS of the copy, chunk position
  // lane % CHUNKS (fetching the chunk that the swizzle puts there).  Rows
  // past the readable context re-read its last row, and an out-of-pool block
  // id reads block 0 (finite values; their scores are masked).  Every copy is
  // issued unconditionally, so each wave's outstanding count is the same
  // every step.  (Copying from every wave instead raised each SIMD's scalar
  // work per step by a third and the step time with it.)
  const int cw = wave & (kCopyWaves - 1);
  const int delta = lane / CHUNKS;
  uint32_t chunk_off[kDmaPerWave];
  bool chunk_in[kDmaPerWave];  // the fetched piece lies inside the head in memory
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int r = cw * kCopyRows + j * kRowsPerDma + delta;
    const int c = (lane % CHUNKS) ^ chunk_swizzle<CHUNKS>(r);
    chunk_off[j] = static_cast<uint32_t>(c * 16);
    chunk_in[j] = c * 8 < DM;
  }
  // Per-lane offsets of a wave's copies when its 16 rows share one block.
  uint32_t row_off[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j)
    row_off[j] = __umul24(static_cast<uint32_t>(j * kRowsPerDma + delta), row_bytes) + chunk_off[j];
  const bool one_block = (1 << log2_bs) >= kCopyRows;
  auto valid_block = [&](int b) {
    return static_cast<uint32_t>(b) < static_cast<uint32_t>(a.total_blocks) ? static_cast<uint32_t>(b) : 0u;
  };
  // Block ids of the first stages come from scalar loads of the table
  // (constant address space: the table does not change during the launch).
  const_i32* btc = (const_i32*)(bt);
  // Block-id ring: slot x % kIdSlots holds the table entries of columns
  // [col0(x), col0(x) + 64) (clamped to the row): every column a stage's
  // positions use.  Wave 0 copies a stage's slot kIdAhead stages ahead, and
  // a copying wave reads the id of its next copies one step ahead, so no
  // copy waits on a table read and the loop issues no scalar loads (their
  // out-of-order returns would force every LDS wait to drain).
  auto col0 = [&](int x) { return min((x * kStage) >> log2_bs, last_col); };
  auto dma_ids = [&](int x) {
    const int c0 = col0(x);
    dma4_s(lds0 + kIdBase + (x & (kIdSlots - 1)) * kIdSlotBytes,
           static_cast<uint32_t>(min(lane, last_col - c0)) * 4u, bt + c0);
  };
  // Ring entry of position p of stage x (p inside the readable context and
  // the stage; other positions read some valid entry, which is not used).
  auto ring_id = [&](int x, int p) {
    const int idx = min(max((p >> log2_bs) - col0(x), 0), kWave - 1);
    return *reinterpret_cast<const int*>(s_lds + kIdBase + (x & (kIdSlots - 1)) * kIdSlotBytes + idx * 4);
  };
  // The ring entry of a copying wave's first row when its 16 rows share one
  // block and the stage lies inside the readable context (blocks of 16 or
  // more start on a stage boundary, or contain the whole stage).
  const int fast_idx4 = kIdBase + ((cw * kCopyRows) >> log2_bs) * 4;
  auto ring_fast = [&](int x) {
    return *reinterpret_cast<const int*>(s_lds + fast_idx4 + (x & (kIdSlots - 1)) * kIdSlotBytes);
  };
  const int id_last = btc[min(kv_last >> log2_bs, last_col)];  // block of the last readable row
  // Copies of this wave's rows of tensor stage x into LDS region `region`,
  // one per kRowsPerDma rows, with get_id(j, p): the block id of position p
  // (readable) of copy j.
  auto copy_each = [&](int x, uint32_t region, const char* base, auto get_id) {
    const int p0 = x * kStage + cw * kCopyRows;
    const uint32_t dst0 = lds0 + region + cw * kCopyRows * ROW_BYTES;
    if constexpr (!LANE_IDS) {
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) {
        const int p = p0 + j * kRowsPerDma;
        const int pc = min(p, kv_last);
        const uint32_t bb = valid_block(p <= kv_last ? get_id(j, p) : id_last);
        const char* src = base + (static_cast<uint64_t>(bb) * block_bytes +
                                  static_cast<uint32_t>(pc & bs_mask) * row_bytes);
        // Rows of the copy past the readable context re-read its last row
        // (same block: a copy never spans blocks here).
        const uint32_t voff =
            __umul24(min(static_cast<uint32_t>(delta), static_cast<uint32_t>(kv_last - pc)), row_bytes) +
            chunk_off[j];
        if (!MASKD || chunk_in[j]) dma16_s(dst0 + j * kRowsPerDma * ROW_BYTES, voff, src);
      }
    } else {
      // Blocks smaller than a copying wave's rows: each lane's row has its own
      // block, read from the ring for every copy of the tensor first (one
      // wait for all of them, not one per copy).
      int pos[kDmaPerWave], b[kDmaPerWave];
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) {
        pos[j] = min(p0 + j * kRowsPerDma + delta, kv_last);
        b[j] = pos[j] >= x * kStage ? ring_id(x, pos[j]) : id_last;
      }
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j)
        if (!MASKD || chunk_in[j])
          dma16(dst0 + j * kRowsPerDma * ROW_BYTES,
                base + (static_cast<uint64_t>(valid_block(b[j])) * block_bytes +
                        (static_cast<uint32_t>(pos[j] & bs_mask) * row_bytes + chunk_off[j])));
    }
  };

  // A loop step's copies: one scalar base for the wave's 16 rows when they
  // share a block and are readable (id_fast: their block id, read from the
  // ring a step ahead), else one copy at a time with ids from the ring.
  auto copy_step = [&](int x, uint32_t region, const char* base, int id_fast) {
    const int p0 = x * kStage + cw * kCopyRows;
    if (!LANE_IDS && one_block && p0 + kCopyRows - 1 <= kv_last) {
      const uint32_t bb = valid_block(__builtin_amdgcn_readfirstlane(id_fast));
      const char* src = base + (static_cast<uint64_t>(bb) * block_bytes +
                                static_cast<uint32_t>(p0 & bs_mask) * row_bytes);
      const uint32_t dst0 = lds0 + region + cw * kCopyRows * ROW_BYTES;
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j)
        if (!MASKD || chunk_in[j]) dma16_s(dst0 + j * kRowsPerDma * ROW_BYTES, row_off[j], src);
    } else {
      copy_each(x, region, base, [&](int, int p) { return __builtin_amdgcn_readfirstlane(ring_id(x, p)); });
    }
  };
  auto copy_prologue = [&](int x, uint32_t region, const char* base) {
    copy_each(x, region, base, [&](int, int p) { return btc[p >> log2_bs]; });
  };

  // ---- LDS operands --------------------------------------------------------------
  // Offsets inside slot 0 of the K ring and of the V ring; a slot adds a
  // multiple of kRegion (an immediate offset when the slot is static).
  const int k_row = kh * kKvTile + (lane & 31);
  int k_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    k_off[ks] = k_row * ROW_BYTES + (((half + 2 * ks) ^ chunk_swizzle<CHUNKS>(k_row)) * 16);
  const int li = lane & 15;
  int v_off[2][DB];  // [8-row half][d block]; +16 rows per k-step is added below
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
    const int r = kh * kKvTile + 4 * half + (li >> 2) + 8 * hi;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int col = 16 * ((lane >> 4) & 1) + 4 * (li & 3) + 32 * db;  // element
      v_off[hi][db] = kVBase + r * ROW_BYTES + (((col >> 3) ^ chunk_swizzle<CHUNKS>(r)) * 16) + (col & 7) * 2;
    }
  }
  auto read_k = [&](int slot, uint4* ka) {
    const char* buf = s_lds + slot * kRegion;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) ka[ks] = *reinterpret_cast<const uint4*>(buf + k_off[ks]);
  };
  // Transpose read r of V^T (r = (k-step, d block, 8-row half)).
  auto read_vt = [&](int slot, int r, uint4 (*va)[DB]) {
    const int kk = r / (2 * DB), db = (r / 2) % DB, hi = r % 2;
    const uint2 w = lds_read_tr16(
        reinterpret_cast<const uint16_t*>(s_lds + slot * kRegion + kk * 16 * ROW_BYTES + v_off[hi][db]));
    if (hi == 0) { va[kk][db].x = w.x; va[kk][db].y = w.y; }
    else { va[kk][db].z = w.x; va[kk][db].w = w.y; }
  };

  // Scores of tile t (positions [32 t, 32 t + 32)) masked for this lane's row:
  // past its causal limit or past the readable context (positions relative
  // to the tile, so each test is one compare) ...
  const int kv_lim = min(qpos, kv_last);  // last position this row attends
  auto mask_tile = [&](int t, f32x16& s) {
    const int lim = kv_lim - (t * kKvTile + 4 * half);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (8 * (i >> 2) + (i & 3) > lim) s[i] = -INFINITY;
    }
  };
  // ... and (bad_ids only) in a block outside the pool.  This one is applied
  // at the start of the step that turns the tile into probabilities, outside
  // the interleaved phases; the tile's maximum may then include such a
  // position's (finite) score, which only moves the reference maximum.
  auto mask_bad = [&](int t, f32x16& s) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kv = t * kKvTile + 8 * (i >> 2) + 4 * half + (i & 3);
      if (kv <= kv_lim && static_cast<uint32_t>(bt[kv >> log2_bs]) >= static_cast<uint32_t>(a.total_blocks))
        s[i] = -INFINITY;
    }
  };
  // Row maximum of a tile: v_max3 written out, because fmaxf makes the
  // compiler quiet each MFMA result first (a v_max x, x per input in IEEE
  // mode), which doubled the instructions; the scores are never NaN.
  auto max3 = [](float x, float y, float z) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(y), "v"(z));
    return r;
  };
  auto tile_max = [&](const f32x16& s) {
    const float a0 = max3(s[0], s[1], s[2]), a1 = max3(s[3], s[4], s[5]), a2 = max3(s[6], s[7], s[8]);
    const float a3 = max3(s[9], s[10], s[11]), a4 = max3(s[12], s[13], s[14]);
    const float b0 = max3(a0, a1, a2), b1 = max3(a3, a4, s[15]);
    const float t = max3(b0, b1, b1);
    return max_halves(t);
  };

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m = kScoreFloor, l = 0.f;  // l: this lane's half of the row sum
  // Lazy rescale: the reference maximum m of a row moves only when a tile's
  // maximum exceeds it by more than kLazyRescale (log2 units), so
  // p <= 2^kLazyRescale; l and acc use the same m, and the result is the
  // same softmax.
  auto rescale = [&](float tmax) {
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
  };

  // ---- prologue --------------------------------------------------------------
  // K of stages 0-2, V of stage 0 and the id ring of stages 0-7 landed, then
  // K 3 / V 1 in flight.
  if constexpr (MASKD) {
    // Row pieces past the head are never copied: zero them once, before any
    // copy lands.
    for (int i = tid; i < (kKBufs + kVBufs) * kRegion / 16; i += kPrefillThreads)
      st16(s_lds + 16 * i, make_uint4(0, 0, 0, 0));
    __syncthreads();
  }
  {
    if (wave == 0) {
#pragma unroll
      for (int x = 0; x < kIdAhead; ++x) dma_ids(x);
    }
    if constexpr (LANE_IDS) {
      // (these copies read their ids from the ring)
      wait_vmcnt<0>();
      __syncthreads();
    }
    if (wave < kCopyWaves) {
#pragma unroll
      for (int x = 0; x < 3; ++x) copy_prologue(x, x * kRegion, kbase);
      copy_prologue(0, kVBase, vbase);
    }
    wait_vmcnt<0>();
  }
  asm volatile("" : "+v"(scan0));  // the scan's first load is checked after the copies
  int bad_local = static_cast<uint32_t>(scan0) >= static_cast<uint32_t>(a.total_blocks) ? 1 : 0;
  for (int c = tid + kPrefillThreads; c < ncols; c += kPrefillThreads)
    bad_local |= static_cast<uint32_t>(bt[c]) >= static_cast<uint32_t>(a.total_blocks) ? 1 : 0;
  // (also publishes the first stages and the id ring)
  bad_ids = __syncthreads_or(bad_local) != 0;
  // Tiles below this index need no mask for any row of the workgroup.
  const int first_masked = bad_ids ? 0 : min(start + tok0 + 1, kv_read) / kKvTile;
  if (wave < kCopyWaves) {
    copy_prologue(3, 3 * kRegion, kbase);
    copy_prologue(1, kVBase + kRegion, vbase);
  }
  // Ids of step 0's copies (K of stage 4, V of stage 2), from the ring.
  int idk = 0, idv = 0;
  auto prefetch_ids = [&](int st) {
    if (wave < kCopyWaves) {
      idk = ring_fast(st + 4);
      idv = ring_fast(st + 2);
    }
  };
  prefetch_ids(0);
  f32x16 s0, s1;
  uint4 ka[KS];
  {
#pragma unroll
    for (int i = 0; i < 16; ++i) s0[i] = 0.f;
    read_k(0, ka);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s0 = mfma32<T>(ka[ks], qreg[ks], s0);
    read_k(1, ka);
    mask_tile(kh, s0);
    rescale(tile_max(s0));
  }
  // Every wave has read K of stage 0 before step 0 refills its buffer.
  stage_barrier();

  // 1.0 in both halves of a packed pair (bf16 0x3F80, fp16 0x3C00).
  constexpr uint32_t kOnes = Elem<T>::kDtype == PA_DTYPE_BF16 ? 0x3F803F80u : 0x3C003C00u;

  // One step: see the header comment.  s_cur holds the scores of this
  // wave's tile of stage st, s_nxt receives those of stage st + 1.  The K
  // and V rings have four slots each; stage x lives in slot x % 4 (SLOT, a
  // compile-time constant in both loops below).
  auto step = [&](int st, f32x16& s_cur, f32x16& s_nxt, auto masked, auto slot_c) {
    constexpr bool MASKED = decltype(masked)::value;
    constexpr int SLOT = decltype(slot_c)::value;
    const int slot = SLOT >= 0 ? SLOT : (st & (kKBufs - 1));
    if (wave < kCopyWaves) copy_step(st + 4, slot * kRegion, kbase, idk);
    const int idv_cur = idv;  // (the prefetch below replaces idv)
    if (bad_ids) mask_bad(2 * st + kh, s_cur);

    // ---- A: S_next = K_next Q^T | P = exp2(S - m) | V^T reads
    const float msc = m * scale;
    f32x16 sn;
#pragma unroll
    for (int i = 0; i < 16; ++i) sn[i] = 0.f;
    uint4 va[2][DB];
    uint4 pb[2];
    float rsum0 = 0.f, rsum1 = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      sn = mfma32<T>(ka[ks], qreg[ks], sn);
#pragma unroll
      for (int j = ks * kPerQk; j < (ks + 1) * kPerQk; ++j) s_cur[j] = fast_exp2(fmaf(s_cur[j], scale, -msc));
#pragma unroll
      for (int r = ks * (kVReads / KS); r < (ks + 1) * (kVReads / KS); ++r) read_vt(slot, r, va);
      if (((ks + 1) * kPerQk) % 8 == 0) {
        const int c = (ks + 1) * kPerQk / 8 - 1;
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
    // ---- B: O^T += V^T P^T | row maxima of S_next | K reads of stage st+2
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] = mfma32<T>(va[kk][db], pb[kk], acc[db]);
    read_k((slot + 2) & (kKBufs - 1), ka);
    prefetch_ids(st + 1);
    if constexpr (MASKED) mask_tile(2 * (st + 1) + kh, sn);
    const float tmax = tile_max(sn);
    l += rsum0 + rsum1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kVReads / KS, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 6 * 8 / KS, 0);
    }
#pragma unroll
    for (int i = 0; i < 2 * DB; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, (KS + 2) / (2 * DB), 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 2, 0);
    }
    rescale(tmax);
    s_nxt = sn;
    // The V copies and the id slot go out after the math, so that a copying
    // wave issues its copies in two short runs rather than one long one.
    if (wave < kCopyWaves) copy_step(st + 2, kVBase + ((slot + 2) & (kKBufs - 1)) * kRegion, vbase, idv_cur);
    if (wave == 0) dma_ids(st + kIdAhead);
    // K of stage st+3, V of stage st+1 and (wave 0) the id slot of stage
    // st+7, copied last step, must have landed before the barrier
    // publishes them.
    if (wave == 0) wait_vmcnt<2 * kDmaPerWave + 1>();
    else if (wave < kCopyWaves) wait_vmcnt<2 * kDmaPerWave>();
    stage_barrier();
  };

  // Every step runs a body with its ring slot (st % 4) and score registers
  // (st % 2) fixed at compile time: four unmasked steps per trip while both
  // tiles of stage st+1 lie below first_masked, then masked steps, four per
  // trip with an exit test after each (no step past the last stage).
  using U = std::false_type;
  using M = std::true_type;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  const int n_main = min(max(first_masked / 2 - 1, 0), nstages);
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
  // Let every copy land before the buffers are reused for the merge.
  wait_vmcnt<0>();
  __syncthreads();
  l += __shfl_xor(l, 32, kWave);

  // ---- merge the two context halves of every row group ---------------------
  float* scratch = reinterpret_cast<float*>(s_lds) + rg * (16 * DB + 2) * kWave;
  if (kh == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) scratch[(db * 16 + i) * kWave + lane] = acc[db][i];
    scratch[(16 * DB) * kWave + lane] = m;
    scratch[(16 * DB + 1) * kWave + lane] = l;
  }
  __syncthreads();
  if (kh == 1) return;
  {
    const float m2 = scratch[(16 * DB) * kWave + lane];
    const float l2 = scratch[(16 * DB + 1) * kWave + lane];
    const float mm = fmaxf(m, m2);
    const float a1 = fast_exp2((m - mm) * scale);
    const float a2 = fast_exp2((m2 - mm) * scale);
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc[db][i] = acc[db][i] * a1 + scratch[(db * 16 + i) * kWave + lane] * a2;
  }

  if (!row_live) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* orow = reinterpret_cast<uint16_t*>(a.output) +
                   ((first + tok0 + tok) * (hkv * a.group) + h) * static_cast<int64_t>(DM);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = db * 32 + 8 * q4 + 4 * half;
      if (MASKD && d >= DM) continue;
      uint2 w;
      w.x = pack_half2<T>(acc[db][4 * q4 + 0] * inv, acc[db][4 * q4 + 1] * inv);
      w.y = pack_half2<T>(acc[db][4 * q4 + 2] * inv, acc[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = w;
    }
}

bool prefill_fast_path_supported(int dtype, int head_dim, int group, int block_size) {
  // bf16 / fp16: the MFMA kernel below (heads of 80 and 96 on rows of 128)
  // and prefill256_kernel for heads of 256; fp32: prefill_f32_kernel (VALU),
  // heads of 64 and 128.
  if (dtype != PA_DTYPE_BF16 && dtype != PA_DTYPE_F16 && dtype != PA_DTYPE_F32) return false;
  const bool mfma_dim =
      head_dim == 64 || head_dim == 80 || head_dim == 96 || head_dim == 128 || head_dim == 256;
  if (dtype == PA_DTYPE_F32 ? head_dim != 64 && head_dim != 128 : !mfma_dim) return false;
  if (group < 1 || group > kMaxDecodeQueryGroup) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  return true;
}

// Query tokens per work item: 128 rows over the heads of one workgroup (a
// sub-group of at most 8 when the group is larger).
int prefill_tile_for(int group) {
  return group > 0 ? kPrefillRows / (group / decode_sub_groups(group)) : kPrefillRows;
}

template <typename T, int D, int DM>
static hipError_t launch_prefill_d(const PrefillArgs& a, int group, int64_t num_items, hipStream_t s) {
  const int g = group / a.sub_groups;
  if (g < 1 || g > 8) return hipErrorNotSupported;
  const dim3 grid(static_cast<uint32_t>(num_items * a.num_kv_heads * a.sub_groups));
  // A copying wave's 16 rows of a stage share one block from blocks of 16
  // up; smaller blocks take the per-lane copy addresses (ids read per lane
  // from the ring), which beat one scalar base per copy with its id read
  // just before it.
  if ((1 << a.log2_block_size) >= kCopyRows)
    hipLaunchKernelGGL((prefill_kernel<T, D, DM, false>), grid, dim3(kPrefillThreads), 0, s, a);
  else
    hipLaunchKernelGGL((prefill_kernel<T, D, DM, true>), grid, dim3(kPrefillThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int dtype, int head_dim, int group,
                          int64_t num_items, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  if (dtype == PA_DTYPE_F32) return launch_prefill_f32(a, head_dim, group, num_items, stream);
  if (head_dim == 256) return launch_prefill256(a, dtype, group, num_items, stream);
  if (dtype == PA_DTYPE_BF16) {
    if (head_dim == 128) return launch_prefill_d<bf16_t, 128, 128>(a, group, num_items, stream);
    if (head_dim == 96) return launch_prefill_d<bf16_t, 128, 96>(a, group, num_items, stream);
    if (head_dim == 80) return launch_prefill_d<bf16_t, 128, 80>(a, group, num_items, stream);
    if (head_dim == 64) return launch_prefill_d<bf16_t, 64, 64>(a, group, num_items, stream);
  } else if (dtype == PA_DTYPE_F16) {
    if (head_dim == 128) return launch_prefill_d<f16_t, 128, 128>(a, group, num_items, stream);
    if (head_dim == 96) return launch_prefill_d<f16_t, 128, 96>(a, group, num_items, stream);
    if (head_dim == 80) return launch_prefill_d<f16_t, 128, 80>(a, group, num_items, stream);
    if (head_dim == 64) return launch_prefill_d<f16_t, 64, 64>(a, group, num_items, stream);
  }
  return hipErrorNotSupported;
}

}  // namespace pa
