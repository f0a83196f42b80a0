// Causal chunked prefill over the paged cache with gfx950 MFMA tiles.
//
// A unit of work is (sequence, query tile, KV head).  The tile holds 128
// query rows = (128 / G) query tokens x the G query heads that share the KV
// head.  The launch runs one workgroup (8 waves) per CU, and each walks its
// share of the units in turn (longest first, snake order), so a unit's
// start costs no workgroup launch.  The context is walked in stages of 64
// tokens; wave w owns rows [32 (w%4), 32 (w%4) + 32) and the 32-token half
// w/4 of every stage, with flash-style online softmax in fp32, so the two
// waves of a row group split the context and merge their partial results
// through LDS at the end (this halves the longest chain of a causal tile).
// The query tile comes into LDS and the finished rows leave through it, in
// whole rows: a lane's own row in registers would take one 16-byte piece of
// 32 different rows per load or store.
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
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "pa_common.hpp"
#include "pa_launch.hpp"
#include "prefill_common.hpp"

namespace pa {

constexpr int kPrefillThreads = 512;  // 4 row groups x 2 context halves
constexpr int kPrefillRows = 128;  // query rows per unit
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
// APPEND (pa_prefill_append): context positions at or after the chunk's
// start are copied from the step's new rows instead of the cache, and after
// its last stage each unit of sub-group 0 stores its own tile's rows from
// the rings into the cache (the rings then hold the last four stages, which
// cover the tile's at most 128 tokens), so no unit reads a row another one
// writes.
template <typename T, int D, int DM, bool LANE_IDS, bool APPEND>
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
  constexpr int kQBase = kVBase + 2 * kRegion;       // query tile: V slots 2-3 during the prologue
  constexpr int kQRowsPerWave = kPrefillRows / kPrefillWaves;
  constexpr int kQDmaPerWave = kQRowsPerWave / kRowsPerDma;
  static_assert(kQRowsPerWave % kRowsPerDma == 0 && kPrefillRows * ROW_BYTES <= 2 * kRegion, "query tile");
  static_assert(DB % 2 == 0, "the two halves finish half of the d blocks each");
  constexpr int kHalfDB = DB / 2;                      // d blocks each half of a row group finishes
  constexpr int kMergeChunks = 4 * kHalfDB + 1;        // 16-byte pieces a lane hands over: acc + (m, l)
  constexpr int kOutBase = 8 * kMergeChunks * kWave * 16;  // finished rows, after the 8 merge regions
  static_assert(kOutBase + kPrefillRows * ROW_BYTES <= kIdBase, "merge scratch and finished rows must fit");
  static_assert(kVReads % KS == 0, "V^T reads spread over the QK k-steps");

  // K ring, then V ring (rows swizzled); reused for each unit's final merge.
  __shared__ __attribute__((aligned(16))) char s_lds[kLdsBytes];

  const int G = a.group / a.sub_groups;  // query heads of a unit
  const int MTOK = kPrefillRows / G;     // query tokens per unit
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // Wave-uniform (scalar): branches on it are whole-wave branches, and the
  // copy counts each wave waits on are exact.
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rg = wave & 3;   // row group
  const int kh = wave >> 2;  // context half of every stage
  const int hkv = a.num_kv_heads;
  const int units = hkv * a.sub_groups;  // units per item
  const int log2_bs = a.log2_block_size;
  const int bs_mask = (1 << log2_bs) - 1;
  // Byte strides of a cache row and a cache block (the host keeps a block
  // under 4 GiB, so a row offset is one 32 x 32 -> 64-bit multiply-add).
  const uint32_t row_bytes = static_cast<uint32_t>(hkv) * MEM_ROW;
  const uint32_t block_bytes = row_bytes << log2_bs;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_lds));
  const float scale = a.scale_log2e;

  // This lane's query row of a unit's tile.
  const int row = rg * 32 + (lane & 31);
  const int half = lane >> 5;
  const int g = row / MTOK;
  const int tok = row - g * MTOK;

  // ---- copy geometry ------------------------------------------------------------
  // Wave cw < 4 copies rows [16 cw, 16 cw + 16) of a stage, kRowsPerDma rows
  // per copy: lane -> row delta = lane / CHUNKS of the copy, chunk position
  // lane % CHUNKS (fetching the chunk that the swizzle puts there).  (Copying
  // from every wave instead raised each SIMD's scalar work per step by a
  // third and the step time with it.)
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
  // The ring entry of a copying wave's first row when its 16 rows share one
  // block (blocks of 16 or more start on a stage boundary, or contain the
  // whole stage).
  const int fast_idx4 = kIdBase + ((cw * kCopyRows) >> log2_bs) * 4;
  auto ring_fast = [&](int x) {
    return *reinterpret_cast<const int*>(s_lds + fast_idx4 + (x & (kIdSlots - 1)) * kIdSlotBytes);
  };

  // ---- LDS operands --------------------------------------------------------------
  // Offsets inside slot 0 of the K ring and of the V ring; a slot adds a
  // multiple of kRegion (an immediate offset when the slot is static).
  const int k_row = kh * kKvTile + (lane & 31);
  int k_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    k_off[ks] = k_row * ROW_BYTES + (((half + 2 * ks) ^ chunk_swizzle<CHUNKS>(k_row)) * 16);
  // This lane's query row in the staged tile: rows rg * 32 + (lane & 31) and
  // k_row share their low bits, hence their swizzle, so the offsets are
  // k_off plus a wave-uniform row shift.
  const int q_shift = kQBase + (rg - kh) * 32 * ROW_BYTES;
  const int li = lane & 15;
  // The waves of context half 1 keep their d blocks rotated by DB / 2:
  // register block b holds d block (b + kh DB / 2) mod DB, so that at the
  // merge blocks 0 .. DB / 2 - 1 are the ones a wave finishes itself, in
  // both halves, with indices fixed at compile time.
  int v_off[2][DB];  // [8-row half][register block]; +16 rows per k-step is added below
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
    const int r = kh * kKvTile + 4 * half + (li >> 2) + 8 * hi;
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      const int db = (b + kh * (DB / 2)) % DB;
      const int col = 16 * ((lane >> 4) & 1) + 4 * (li & 3) + 32 * db;  // element
      v_off[hi][b] = kVBase + r * ROW_BYTES + (((col >> 3) ^ chunk_swizzle<CHUNKS>(r)) * 16) + (col & 7) * 2;
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
  // 1.0 in both halves of a packed pair (bf16 0x3F80, fp16 0x3C00).
  constexpr uint32_t kOnes = Elem<T>::kDtype == PA_DTYPE_BF16 ? 0x3F803F80u : 0x3C003C00u;

  // ---- the workgroup's units ---------------------------------------------------
  // A unit is (item, KV head, sub-group); block id b = item * units + unit.
  // The launch runs W workgroups (one per CU) over U units: workgroup w takes
  // the units of rank w, 2W-1-w, 2W+w, 4W-1-w, ... in the order of block ids
  // from the highest down (the last query tiles of a sequence see the most
  // context), a snake that evens out each workgroup's total context.  Every
  // unit starts with a memory round trip for its table entries and one for
  // its first copies; the item and sequence records of the next unit are
  // loaded while the current one runs (one lane-indexed load into one
  // register), so they add none.
  const int U = static_cast<int>(a.num_units);
  const int W = static_cast<int>(gridDim.x);
  const int wg = static_cast<int>(blockIdx.x);
  auto rank_of = [&](int r) { return (r & 1) ? (r + 1) * W - 1 - wg : r * W + wg; };
  auto item_of = [&](int rk) { return (U - 1 - rk) / units; };
  int rank = rank_of(0);
  if (rank >= U) return;
  // The first unit's records, then the item of the second.
  int seq = a.items[2 * item_of(rank)];
  int qt = a.items[2 * item_of(rank) + 1];
  int first = static_cast<int>(a.cu_seqlens[seq]);  // token indices stay below 2^31
  int count = static_cast<int>(a.cu_seqlens[seq + 1]) - first;
  int ctx = a.context_lens[seq];
  int trow = a.rows != nullptr ? a.rows[seq] : seq;
  int rank_n = rank_of(1);
  int seq_n = 0, qt_n = 0;
  if (rank_n < U) {
    seq_n = a.items[2 * item_of(rank_n)];
    qt_n = a.items[2 * item_of(rank_n) + 1];
  }

  for (int r = 1;; ++r) {
    // Lane k of `pre` loads field k of the next unit's records: 0-1 the
    // (seq, query tile) of the unit after it, 2-3 the low words of
    // cu_seqlens[seq_n], cu_seqlens[seq_n + 1], 4 context_lens[seq_n], 5 the
    // table row of seq_n.  Read back when the next unit starts.
    const bool more = rank_n < U;
    const int rank_nn = rank_of(r + 1);
    int pre = 0;
    if (more) {
      const int it_nn = rank_nn < U ? item_of(rank_nn) : 0;
      const int32_t* p = a.items + 2 * it_nn + (lane & 1);
      if (lane == 2 || lane == 3) p = reinterpret_cast<const int32_t*>(a.cu_seqlens + seq_n + (lane - 2));
      if (lane == 4 || (lane == 5 && a.rows == nullptr)) p = a.context_lens + seq_n;
      if (lane == 5 && a.rows != nullptr) p = a.rows + seq_n;
      pre = *p;
    }

    const int unit = (U - 1 - rank) - item_of(rank) * units;
    const int kvh = unit / a.sub_groups;
    const int h0 = kvh * a.group + (unit - kvh * a.sub_groups) * G;  // first query head
    const int start = ctx - count;
    const int tok0 = qt * MTOK;
    const int ntok = min(MTOK, count - tok0);

    if (ntok > 0) {
      const bool row_ok = trow >= 0 && trow < a.num_table_rows;
      const int32_t* bt = row_ok ? a.block_tables + static_cast<int64_t>(trow) * a.block_table_stride : kNoBlockRow;
      global_i32* btg = (global_i32*)(bt);
      const int bt_stride = row_ok ? a.block_table_stride : 1;
      const char* kbase = reinterpret_cast<const char*>(a.key_cache) + kvh * MEM_ROW;
      const char* vbase = reinterpret_cast<const char*>(a.value_cache) + kvh * MEM_ROW;
      // APPEND: this KV head's new rows, the row of position p (at or after
      // start) at nkbase + p * nkstride bytes (the host keeps strides below
      // 2^24).
      const char* nkbase = nullptr;
      const char* nvbase = nullptr;
      uint32_t nkstride = 0, nvstride = 0;
      if constexpr (APPEND) {
        nkstride = static_cast<uint32_t>(a.new_key_token_stride * 2);
        nvstride = static_cast<uint32_t>(a.new_value_token_stride * 2);
        nkbase = reinterpret_cast<const char*>(a.new_key) + kvh * a.new_key_head_stride * 2 +
                 static_cast<int64_t>(first - start) * nkstride;
        nvbase = reinterpret_cast<const char*>(a.new_value) + kvh * a.new_value_head_stride * 2 +
                 static_cast<int64_t>(first - start) * nvstride;
      }

      // Rows past G * MTOK (when G does not divide 128) belong to no head.
      const bool row_live = tok < ntok && g < G;
      const int qpos = start + tok0 + tok;  // causal limit (inclusive)
      const int h = h0 + g;

      uint4 qreg[KS];  // this lane's query row, read from the staged tile below

      const int kv_end = min(ctx, start + tok0 + ntok);  // exclusive
      // Positions that have a block-table column (the rest are never read); at
      // least one, as the host passes tables of one column or more.
      const int kv_read = static_cast<int>(
          min(static_cast<int64_t>(kv_end), static_cast<int64_t>(bt_stride) << log2_bs));
      const int kv_last = kv_read - 1;
      const int nstages = (kv_end + kStage - 1) / kStage;  // >= 1
      const int last_col = bt_stride - 1;
      // Positions whose block id lies outside the pool are skipped, as the
      // decode kernels skip them: one pass over the row's columns tells whether
      // there are any (then every tile takes the masked path below).  Its first
      // load is issued here and checked after the first copies have landed, so
      // the two memory round trips overlap.
      const int ncols = (kv_read + bs_mask) >> log2_bs;
      int scan0 = tid < ncols ? btg[tid] : 0;
      bool bad_ids = false;  // set once the scan is complete (before any tile is masked)

      // ---- copies ------------------------------------------------------------
      // Rows past the readable context re-read its last row, and an
      // out-of-pool block id reads block 0 (finite values; their scores are
      // masked).  No stage past the last is copied: a step's copies, and the
      // count of them its wait allows in flight, depend on how many stages
      // remain.
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
      const int id_last = btc[min(kv_last >> log2_bs, last_col)];  // block of the last readable row
      // APPEND: the new row of position pos (at or after the chunk's start),
      // piece chunk_off[j].
      auto new_row = [&](const char* nbase, uint32_t nstride, int pos, int j) {
        return nbase + (static_cast<uint64_t>(static_cast<uint32_t>(pos)) * nstride + chunk_off[j]);
      };
      // Copies of this wave's rows of tensor stage x into LDS region `region`,
      // one per kRowsPerDma rows, with get_id(j, p): the block id of position p
      // (readable) of copy j.  (nbase, nstride): the tensor's new rows.
      auto copy_each = [&](int x, uint32_t region, const char* base, const char* nbase, uint32_t nstride,
                           auto get_id) {
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
            if (APPEND && p + kRowsPerDma - 1 >= start) {
              // Some of the copy's rows are new rows: per-lane addresses,
              // from a lane row made opaque here (hoisted out of the unit
              // loop, the per-copy terms spilled, and each reload's wait
              // drained the copies in flight).
              int dl = delta;
              asm volatile("" : "+v"(dl));
              const int pos = min(p + dl, kv_last);
              const char* lsrc = pos >= start ? new_row(nbase, nstride, pos, j) : src + voff;
              if (!MASKD || chunk_in[j]) dma16(dst0 + j * kRowsPerDma * ROW_BYTES, lsrc);
            } else {
              if (!MASKD || chunk_in[j]) dma16_s(dst0 + j * kRowsPerDma * ROW_BYTES, voff, src);
            }
          }
        } else {
          // Blocks smaller than a copying wave's rows: each lane's row has its own
          // block, read from the ring for every copy of the tensor first (one
          // wait for all of them, not one per copy).
          int pos[kDmaPerWave], b[kDmaPerWave];
          int dl = delta;
          if constexpr (APPEND) asm volatile("" : "+v"(dl));  // (as in the path above)
#pragma unroll
          for (int j = 0; j < kDmaPerWave; ++j) {
            pos[j] = min(p0 + j * kRowsPerDma + dl, kv_last);
            b[j] = pos[j] >= x * kStage ? ring_id(x, pos[j]) : id_last;
          }
#pragma unroll
          for (int j = 0; j < kDmaPerWave; ++j)
            if (!MASKD || chunk_in[j]) {
              const char* src = base + (static_cast<uint64_t>(valid_block(b[j])) * block_bytes +
                                        (static_cast<uint32_t>(pos[j] & bs_mask) * row_bytes + chunk_off[j]));
              if (APPEND && pos[j] >= start) src = new_row(nbase, nstride, pos[j], j);
              dma16(dst0 + j * kRowsPerDma * ROW_BYTES, src);
            }
        }
      };

      // A step's copies: one scalar base for the wave's 16 rows when they
      // share a block and are readable (id_fast: their block id) or are all
      // new rows, else one copy at a time with get_id (in the loop: ids from
      // the ring, read a step ahead).
      auto copy_step = [&](int x, uint32_t region, const char* base, const char* nbase, uint32_t nstride,
                           int id_fast, auto get_id) {
        const int p0 = x * kStage + cw * kCopyRows;
        // The wave's 16 rows: all new rows (APPEND), or all in one block of
        // the cache -- one scalar base either way, chosen by a select.
        const bool all_new = APPEND && p0 >= start && p0 + kCopyRows - 1 <= kv_last;
        const bool all_cache = !LANE_IDS && one_block && p0 + kCopyRows - 1 <= kv_last &&
                               (!APPEND || p0 + kCopyRows - 1 < start);
        if (all_new || all_cache) {
          const uint32_t bb = valid_block(__builtin_amdgcn_readfirstlane(id_fast));
          const char* src = base + (static_cast<uint64_t>(bb) * block_bytes +
                                    static_cast<uint32_t>(p0 & bs_mask) * row_bytes);
          if (APPEND && all_new) src = nbase + static_cast<uint64_t>(static_cast<uint32_t>(p0)) * nstride;
          const uint32_t dst0 = lds0 + region + cw * kCopyRows * ROW_BYTES;
#pragma unroll
          for (int j = 0; j < kDmaPerWave; ++j) {
            uint32_t voff = row_off[j];
            if (APPEND && all_new) voff = __umul24(static_cast<uint32_t>(j * kRowsPerDma + delta), nstride) + chunk_off[j];
            if (!MASKD || chunk_in[j]) dma16_s(dst0 + j * kRowsPerDma * ROW_BYTES, voff, src);
          }
        } else {
          copy_each(x, region, base, nbase, nstride, get_id);
        }
      };
      auto ring_ids = [&](int x) {
        return [&, x](int, int p) { return __builtin_amdgcn_readfirstlane(ring_id(x, p)); };
      };
      // The first stages' copies, with `id` the block of the wave's rows in
      // stage x (blocks of 16 or more: one block per copying wave and stage;
      // smaller blocks read their ids from the ring).
      auto copy_first = [&](int x, uint32_t region, const char* base, const char* nbase, uint32_t nstride,
                            int id) {
        copy_step(x, region, base, nbase, nstride, id, [&](int, int) { return id; });
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
          if (kv <= kv_lim && static_cast<uint32_t>(btg[kv >> log2_bs]) >= static_cast<uint32_t>(a.total_blocks))
            s[i] = -INFINITY;
        }
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

      // ---- prologue ----------------------------------------------------------
      // The query tile, the id ring of stages 0-7 and K of stage 0 land
      // before the first barrier; K of stages 1-2 and V of stage 0 land while
      // the first QK runs, before the second; K of stage 3 and V of stage 1
      // before the end of step 0 (only stages that exist are copied).
      if constexpr (MASKD) {
        // Row pieces past the head are never copied: zero them before any
        // copy lands (the previous unit's merge wrote over the rings).
        for (int i = tid; i < (kKBufs + kVBufs) * kRegion / 16; i += kPrefillThreads)
          st16(s_lds + 16 * i, make_uint4(0, 0, 0, 0));
        __syncthreads();
      }
      {
        // The query tile goes into V slots 2-3 (free until step 0 copies V of
        // stage 2) in whole rows, swizzled like the K rows: wave w copies rows
        // [w kQRowsPerWave, (w + 1) kQRowsPerWave), kRowsPerDma per copy.
        // Rows that belong to no head fetch the tile's first row (their
        // results are never stored).
        // (The row arithmetic is kept inside the unit loop: hoisted out of
        // it, its per-copy values would be held in registers for the whole
        // launch and spilled.)
        int qr = wave * kQRowsPerWave + delta;
        asm volatile("" : "+v"(qr));
        int qg = qr / MTOK;
        int qtok = qr - qg * MTOK;
#pragma unroll
        for (int j = 0; j < kQDmaPerWave; ++j) {
          const bool live = qtok < ntok && qg < G;
          const int c = (lane % CHUNKS) ^ chunk_swizzle<CHUNKS>(qr);
          const uint16_t* src = reinterpret_cast<const uint16_t*>(a.query) +
                                static_cast<int64_t>(first + tok0 + (live ? qtok : 0)) * a.q_token_stride +
                                static_cast<int64_t>(h0 + (live ? qg : 0)) * a.q_head_stride + c * 8;
          if (!MASKD || c * 8 < DM)
            dma16(lds0 + kQBase + (wave * kQRowsPerWave + j * kRowsPerDma) * ROW_BYTES, src);
          // next copy's row: kRowsPerDma further (less than a head's tokens)
          qr += kRowsPerDma;
          qtok += kRowsPerDma;
          if (qtok >= MTOK) { qtok -= MTOK; ++qg; }
        }
        if (wave == 0) {
#pragma unroll
          for (int x = 0; x < kIdAhead; ++x)
            if (x < nstages) dma_ids(x);
        }
        if constexpr (LANE_IDS) {
          // (these copies read their ids from the ring)
          wait_vmcnt<0>();
          __syncthreads();
        }
        if (wave < kCopyWaves) {
          // The block of this wave's rows in each of stages 0-3, all loaded
          // before the first copy (one round trip, not one per copy).
          int pid[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) pid[x] = btc[min(x * kStage + cw * kCopyRows, kv_last) >> log2_bs];
          copy_first(0, 0, kbase, nkbase, nkstride, pid[0]);
          if (nstages > 1) copy_first(1, kRegion, kbase, nkbase, nkstride, pid[1]);
          if (nstages > 2) copy_first(2, 2 * kRegion, kbase, nkbase, nkstride, pid[2]);
          copy_first(0, kVBase, vbase, nvbase, nvstride, pid[0]);
          // everything but K 1-2 and V 0 (issued last)
          wait_vmcnt_at_most<3 * kDmaPerWave>(kDmaPerWave * (1 + (nstages > 1 ? 1 : 0) + (nstages > 2 ? 1 : 0)));
        } else {
          wait_vmcnt<0>();
        }
      }
      __syncthreads();  // the query tile, K of stage 0 and the id ring
      f32x16 s0, s1;
      uint4 ka[KS];
#pragma unroll
      for (int i = 0; i < 16; ++i) s0[i] = 0.f;
      read_k(0, ka);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qreg[ks] = *reinterpret_cast<const uint4*>(s_lds + q_shift + k_off[ks]);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s0 = mfma32<T>(ka[ks], qreg[ks], s0);
      asm volatile("" : "+v"(scan0));  // the scan's first load is checked after all copies landed
      int bad_local = static_cast<uint32_t>(scan0) >= static_cast<uint32_t>(a.total_blocks) ? 1 : 0;
      for (int c = tid + kPrefillThreads; c < ncols; c += kPrefillThreads)
        bad_local |= static_cast<uint32_t>(btg[c]) >= static_cast<uint32_t>(a.total_blocks) ? 1 : 0;
      wait_vmcnt<0>();
      // (also publishes K of stages 1-2 and V of stage 0, and tells that every
      // wave has read K of stage 0 before step 0 refills its slot)
      bad_ids = __syncthreads_or(bad_local) != 0;
      // Tiles below this index need no mask for any row of the unit.
      const int first_masked = bad_ids ? 0 : min(start + tok0 + 1, kv_read) / kKvTile;
      if (wave < kCopyWaves) {
        if (nstages > 3) copy_step(3, 3 * kRegion, kbase, nkbase, nkstride, ring_fast(3), ring_ids(3));
        if (nstages > 1) copy_step(1, kVBase + kRegion, vbase, nvbase, nvstride, ring_fast(1), ring_ids(1));
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
      read_k(1, ka);
      mask_tile(kh, s0);
      rescale(tile_max(s0));

      // One step: see the header comment.  s_cur holds the scores of this
      // wave's tile of stage st, s_nxt receives those of stage st + 1.  The K
      // and V rings have four slots each; stage x lives in slot x % 4 (SLOT, a
      // compile-time constant in both loops below).
      auto step = [&](int st, f32x16& s_cur, f32x16& s_nxt, auto masked, auto slot_c) {
        constexpr bool MASKED = decltype(masked)::value;
        constexpr int SLOT = decltype(slot_c)::value;
        const int slot = SLOT >= 0 ? SLOT : (st & (kKBufs - 1));
        // Copies of this step: K of stage st+4, V of stage st+2 and (wave 0)
        // the id slot of stage st+8, each only if that stage exists.
        const bool cpk = st + 4 < nstages, cpv = st + 2 < nstages, cpi = st + kIdAhead < nstages;
        if (wave < kCopyWaves && cpk)
          copy_step(st + 4, slot * kRegion, kbase, nkbase, nkstride, idk, ring_ids(st + 4));
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
        if (wave < kCopyWaves && cpv)
          copy_step(st + 2, kVBase + ((slot + 2) & (kKBufs - 1)) * kRegion, vbase, nvbase, nvstride, idv_cur,
                    ring_ids(st + 2));
        if (wave == 0 && cpi) dma_ids(st + kIdAhead);
        // K of stage st+3, V of stage st+1 and (wave 0) the id slot of stage
        // st+7, copied last step, must have landed before the barrier
        // publishes them; this step's copies may stay in flight (copies
        // complete in issue order, so their count is the wait).
        if (wave < kCopyWaves) {
          const int n = (cpk ? kDmaPerWave : 0) + (cpv ? kDmaPerWave : 0) + (wave == 0 && cpi ? 1 : 0);
          wait_vmcnt_at_most<2 * kDmaPerWave + 1>(n);
        }
        stage_barrier();
      };

      // Every step runs a body with its ring slot (st % 4) and score registers
      // (st % 2) fixed at compile time: four unmasked steps per trip while both
      // tiles of stage st+1 lie below first_masked, then masked steps, four per
      // trip with an exit test after each (no step past the last stage).
      using U0 = std::false_type;
      using M1 = std::true_type;
      using S0 = std::integral_constant<int, 0>;
      using S1 = std::integral_constant<int, 1>;
      using S2 = std::integral_constant<int, 2>;
      using S3 = std::integral_constant<int, 3>;
      const int n_main = min(max(first_masked / 2 - 1, 0), nstages);
      int st = 0;
      for (; st + 3 < n_main; st += 4) {
        step(st, s0, s1, U0{}, S0{});
        step(st + 1, s1, s0, U0{}, S1{});
        step(st + 2, s0, s1, U0{}, S2{});
        step(st + 3, s1, s0, U0{}, S3{});
      }
      while (st < nstages) {
        step(st, s0, s1, M1{}, S0{});
        if (++st == nstages) break;
        step(st, s1, s0, M1{}, S1{});
        if (++st == nstages) break;
        step(st, s0, s1, M1{}, S2{});
        if (++st == nstages) break;
        step(st, s1, s0, M1{}, S3{});
        ++st;
      }
      // (the last step waited for every copy; no stage past the last is copied)
      l += __shfl_xor(l, 32, kWave);

      if constexpr (APPEND) {
        // The unit's share of the step's cache write (sub-group 0 of the KV
        // head): its tile's tokens, positions [start + tok0, + ntok), stored
        // from the rings as copied from the new rows -- stage x in slot x % 4
        // of each ring, which after the last step holds stages nstages - 4 ..
        // nstages - 1 (the tile's tokens lie in the last three), and its
        // table entries in id slot x % 8.  Positions without a table column
        // or in a block outside the pool are not written.
        if (unit - kvh * a.sub_groups == 0 && row_ok) {
          constexpr int MCH = DM / 8;  // 16-byte pieces of a head's row in memory
          const int p_beg = start + tok0;
          const int np = max(0, min(start + tok0 + ntok, kv_read) - p_beg);
          char* kdst = const_cast<char*>(kbase);
          char* vdst = const_cast<char*>(vbase);
          for (int i = tid; i < 2 * np * MCH; i += kPrefillThreads) {
            const bool is_v = i >= np * MCH;
            const int k = is_v ? i - np * MCH : i;
            const int p = p_beg + k / MCH;
            const int c = k - (k / MCH) * MCH;
            const int x = p / kStage;
            const int r = p - x * kStage;
            const int b = ring_id(x, p);
            if (static_cast<uint32_t>(b) < static_cast<uint32_t>(a.total_blocks)) {
              const uint4 v = *reinterpret_cast<const uint4*>(
                  s_lds + (is_v ? kVBase : 0) + (x & (kKBufs - 1)) * kRegion + r * ROW_BYTES +
                  ((c ^ chunk_swizzle<CHUNKS>(r)) * 16));
              st16((is_v ? vdst : kdst) + (static_cast<uint64_t>(b) * block_bytes +
                                           static_cast<uint32_t>(p & bs_mask) * row_bytes + c * 16),
                   v);
            }
          }
          __syncthreads();  // (the merge below writes over the rings)
        }
      }

      // ---- merge the two context halves of every row group -----------------
      // (after the last step's barrier no wave reads the rings any more)
      // Half kh of a row group finishes d blocks [kh DB/2, (kh + 1) DB/2) of
      // its rows: each wave hands the other half of its row group the blocks
      // that half finishes, and its (m, l), in 16-byte pieces (piece c of lane
      // i at (c * 64 + i) * 16 of its own region), reads the other's back a d
      // block (four pieces) at a time, and stores its half of every row.
      // With the rotated d blocks, register blocks 0 .. DB / 2 - 1 are the
      // ones a wave finishes and the rest are handed over, in both halves.
      {
        char* mine = s_lds + (rg * 2 + kh) * kMergeChunks * kWave * 16 + lane * 16;
        const char* other = s_lds + (rg * 2 + (kh ^ 1)) * kMergeChunks * kWave * 16 + lane * 16;
#pragma unroll
        for (int b = 0; b < kHalfDB; ++b) {
          const f32x16& x = acc[kHalfDB + b];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            st16(mine + (b * 4 + q) * kWave * 16,
                 make_uint4(__float_as_uint(x[4 * q + 0]), __float_as_uint(x[4 * q + 1]),
                            __float_as_uint(x[4 * q + 2]), __float_as_uint(x[4 * q + 3])));
          }
        }
        st16(mine + (4 * kHalfDB) * kWave * 16, make_uint4(__float_as_uint(m), __float_as_uint(l), 0u, 0u));
        __syncthreads();
        const uint4 ml = ld16(other + (4 * kHalfDB) * kWave * 16);
        const float m2 = __uint_as_float(ml.x);
        const float l2 = __uint_as_float(ml.y);
        const float mm = fmaxf(m, m2);
        const float a1 = fast_exp2((m - mm) * scale);
        const float a2 = fast_exp2((m2 - mm) * scale);
        // (the same sum, in the same order, in both halves)
        const float lt = kh == 0 ? l * a1 + l2 * a2 : l2 * a2 + l * a1;
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
        // The finished rows go through LDS (swizzled like the K rows) so that
        // each store writes whole 16-byte pieces of a row: lane i of half kh
        // stores piece kh CHUNKS/2 + i % (CHUNKS/2) of row k kRowsPerStore +
        // i / (CHUNKS/2) of the row group.
        char* stage_rows = s_lds + kOutBase + rg * 32 * ROW_BYTES;
        int r_lane = lane;  // (kept inside the unit loop, as the copies' rows above)
        asm volatile("" : "+v"(r_lane));
        const int r32w = r_lane & 31;
        const int sw_w = chunk_swizzle<CHUNKS>(r32w);
#pragma unroll
        for (int b = 0; b < kHalfDB; ++b) {
          const int db = kh * kHalfDB + b;
          const f32x16& x = acc[b];
          uint4 pv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) pv[q] = ld16(other + (b * 4 + q) * kWave * 16);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint2 w;
            w.x = pack_half2<T>((x[4 * q + 0] * a1 + __uint_as_float(pv[q].x) * a2) * inv,
                                (x[4 * q + 1] * a1 + __uint_as_float(pv[q].y) * a2) * inv);
            w.y = pack_half2<T>((x[4 * q + 2] * a1 + __uint_as_float(pv[q].z) * a2) * inv,
                                (x[4 * q + 3] * a1 + __uint_as_float(pv[q].w) * a2) * inv);
            *reinterpret_cast<uint2*>(stage_rows + r32w * ROW_BYTES + (((db * 4 + q) ^ sw_w) * 16) + half * 8) = w;
          }
        }
        constexpr int kHalfChunks = CHUNKS / 2;
        constexpr int kRowsPerStore = kWave / kHalfChunks;
        const int c = kh * kHalfChunks + r_lane % kHalfChunks;
        int r32 = r_lane / kHalfChunks;  // row of the row group this lane stores
        int og = (rg * 32 + r32) / MTOK;
        int otok = rg * 32 + r32 - og * MTOK;
        // All of the lane's pieces are read before the first store (one LDS
        // round trip, not one per store); they are this wave's own writes.
        uint4 piece[32 / kRowsPerStore];
#pragma unroll
        for (int k = 0; k < 32 / kRowsPerStore; ++k) {
          const int rk = r32 + k * kRowsPerStore;
          piece[k] = *reinterpret_cast<const uint4*>(stage_rows + rk * ROW_BYTES + ((c ^ chunk_swizzle<CHUNKS>(rk)) * 16));
        }
#pragma unroll
        for (int k = 0; k < 32 / kRowsPerStore; ++k) {
          const uint4 v = piece[k];
          if (otok < ntok && og < G && (!MASKD || c * 8 < DM)) {
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.output) +
                            (static_cast<int64_t>(first + tok0 + otok) * (hkv * a.group) + h0 + og) *
                                static_cast<int64_t>(DM) +
                            c * 8;
            st16(dst, v);
          }
          otok += kRowsPerStore;
          if (otok >= MTOK) { otok -= MTOK; ++og; }
        }
      }
      // The next unit's copies overwrite the merge scratch.
      if (more) __syncthreads();
    }

    if (!more) break;
    rank = rank_n;
    rank_n = rank_nn;
    seq = seq_n;
    qt = qt_n;
    first = __builtin_amdgcn_readlane(pre, 2);
    count = __builtin_amdgcn_readlane(pre, 3) - first;
    ctx = __builtin_amdgcn_readlane(pre, 4);
    trow = a.rows != nullptr ? __builtin_amdgcn_readlane(pre, 5) : seq;
    seq_n = __builtin_amdgcn_readlane(pre, 0);
    qt_n = __builtin_amdgcn_readlane(pre, 1);
  }
}

bool prefill_fast_path_supported(int dtype, int head_dim, int group, int block_size) {
  // bf16 / fp16: the MFMA kernel below (heads of 80 and 96 on rows of 128)
  // and prefill256_kernel for heads of 256; fp32: prefill_f32_mfma_kernel
  // (v_mfma_f32_32x32x2_f32), heads of 64 and 128.
  if (dtype != PA_DTYPE_BF16 && dtype != PA_DTYPE_F16 && dtype != PA_DTYPE_F32) return false;
  const bool mfma_dim =
      head_dim == 64 || head_dim == 80 || head_dim == 96 || head_dim == 128 || head_dim == 256;
  if (dtype == PA_DTYPE_F32 ? head_dim != 64 && head_dim != 128 : !mfma_dim) return false;
  if (group < 1 || group > kMaxDecodeQueryGroup) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  return true;
}

bool prefill_append_supported(int dtype, int head_dim) {
  // Every fast-path kernel but the one for heads of 256.
  if (dtype == PA_DTYPE_F32) return head_dim == 64 || head_dim == 128;
  return (dtype == PA_DTYPE_BF16 || dtype == PA_DTYPE_F16) &&
         (head_dim == 64 || head_dim == 80 || head_dim == 96 || head_dim == 128);
}

// Query tokens per work item: 128 rows over the heads of one workgroup (a
// sub-group of at most 8 when the group is larger).
int prefill_tile_for(int group) {
  return group > 0 ? kPrefillRows / (group / decode_sub_groups(group)) : kPrefillRows;
}

// Compute units of the current device (cached per device; 0 if unknown).
int device_compute_units() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 0) n = 0;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <typename T, int D, int DM, bool APPEND>
static hipError_t launch_prefill_d(const PrefillArgs& args, int group, int64_t num_items, hipStream_t s) {
  const int g = group / args.sub_groups;
  if (g < 1 || g > 8) return hipErrorNotSupported;
  PrefillArgs a = args;
  a.num_units = num_items * a.num_kv_heads * a.sub_groups;
  // Unit ranks are 32-bit and a workgroup's ranks reach about twice the count.
  if (a.num_units > (int64_t{1} << 30)) return hipErrorInvalidValue;
  // One workgroup per CU (the rings hold one per CU), each looping over its
  // share of the units; fewer units than CUs run one each.
  const int cus = device_compute_units();
  const int64_t wgs = cus > 0 ? std::min<int64_t>(a.num_units, cus) : a.num_units;
  const dim3 grid(static_cast<uint32_t>(wgs));
  // A copying wave's 16 rows of a stage share one block from blocks of 16
  // up; smaller blocks take the per-lane copy addresses (ids read per lane
  // from the ring), which beat one scalar base per copy with its id read
  // just before it.
  if ((1 << a.log2_block_size) >= kCopyRows)
    hipLaunchKernelGGL((prefill_kernel<T, D, DM, false, APPEND>), grid, dim3(kPrefillThreads), 0, s, a);
  else
    hipLaunchKernelGGL((prefill_kernel<T, D, DM, true, APPEND>), grid, dim3(kPrefillThreads), 0, s, a);
  return hipGetLastError();
}

template <typename T, int D, int DM>
static hipError_t launch_prefill_t(const PrefillArgs& a, int group, int64_t num_items, hipStream_t s) {
  return a.new_key != nullptr ? launch_prefill_d<T, D, DM, true>(a, group, num_items, s)
                              : launch_prefill_d<T, D, DM, false>(a, group, num_items, s);
}

hipError_t launch_prefill(const PrefillArgs& a, int dtype, int head_dim, int group,
                          int64_t num_items, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  if (dtype == PA_DTYPE_F32) return launch_prefill_f32(a, head_dim, group, num_items, stream);
  if (head_dim == 256)
    return a.new_key != nullptr ? hipErrorNotSupported : launch_prefill256(a, dtype, group, num_items, stream);
  if (dtype == PA_DTYPE_BF16) {
    if (head_dim == 128) return launch_prefill_t<bf16_t, 128, 128>(a, group, num_items, stream);
    if (head_dim == 96) return launch_prefill_t<bf16_t, 128, 96>(a, group, num_items, stream);
    if (head_dim == 80) return launch_prefill_t<bf16_t, 128, 80>(a, group, num_items, stream);
    if (head_dim == 64) return launch_prefill_t<bf16_t, 64, 64>(a, group, num_items, stream);
  } else if (dtype == PA_DTYPE_F16) {
    if (head_dim == 128) return launch_prefill_t<f16_t, 128, 128>(a, group, num_items, stream);
    if (head_dim == 96) return launch_prefill_t<f16_t, 128, 96>(a, group, num_items, stream);
    if (head_dim == 80) return launch_prefill_t<f16_t, 128, 80>(a, group, num_items, stream);
    if (head_dim == 64) return launch_prefill_t<f16_t, 64, 64>(a, group, num_items, stream);
  }
  return hipErrorNotSupported;
}

}  // namespace pa
