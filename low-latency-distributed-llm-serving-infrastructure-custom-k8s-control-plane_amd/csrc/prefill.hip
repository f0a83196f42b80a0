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
//   S^T[kv][row] = sum_d K[kv][d] Q[row][d]       (A = K from LDS, B = Q regs)
//   O^T[d][row] += sum_kv V^T[d][kv] P^T[kv][row]  (A = V^T, B = P^T regs)
// with v_mfma_f32_32x32x16_bf16 (or _f16 for fp16 caches).  In the 32x32
// accumulator lane l holds
// column l % 32 and rows 8*(i/4) + 4*(l/32) + (i%4), i = 0..15, so the
// softmax max/sum of a query row needs only its own 16 values plus the
// partner lane l ^ 32, and the probabilities a lane holds are the B operand
// of the PV product with the context index of k-slot j being
// 8*(j/4) + 4*(l/32) + (j%4) inside each 16-token step.
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
// Pipeline (one barrier per 64-token stage): four LDS stage buffers hold
// stage t (its V is read), stage t+1 (its K is read: the scores of the next
// tile are computed while this tile's exponentials run), stage t+2 (landed)
// and stage t+3 (being copied).  The block ids of a stage are copied into an
// LDS ring two stages before its rows.  The copies are issued from inline
// assembly, every step the same number per wave, and each wave waits for
// its own copies with an exact s_waitcnt vmcnt before the barrier that
// publishes them (the compiler would otherwise drain every copy before each
// LDS read, as it cannot tell the buffers apart).
// Masking is applied only to tiles that cross the causal diagonal or the end
// of the context (or to every tile when some block id of the sequence lies
// outside the pool: those positions are skipped, as in decode), and the
// accumulator is rescaled only when some row's maximum grew by more than 2^8
// over the reference maximum in use.
//
// Reference: the block-diagonal causal mask of app/model/paged_attention.py:
// 92-118 applied by SDPA (paged_attention.py:170-178); query token j of a
// sequence at position start + j attends context positions [0, start + j].
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4v __attribute__((ext_vector_type(4)));

constexpr int kPrefillThreads = 512;  // 4 row groups x 2 context halves
constexpr int kPrefillRows = 128;  // query rows per workgroup
constexpr int kKvTile = 32;        // context tokens per wave per stage
constexpr int kStage = 2 * kKvTile;  // context tokens per LDS stage
constexpr float kLazyRescale = 8.f;  // log2 headroom before the row maximum moves
constexpr int kStageBufs = 4;       // LDS stage buffers in flight
constexpr int kPrefillWaves = kPrefillThreads / 64;
constexpr int kIdRing = 8;          // block-id slots (one per stage in flight)
constexpr int kIdSlotBytes = 256;   // up to 64 table entries per stage

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

// ds_read_b64_tr_b16 at an LDS address (see the header comment).
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) i16x4v lds_i16x4;
  const i16x4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Direct global -> LDS loads.  Each lane's 16 (or 4) bytes land at
// lds_base + 16 * lane (4 * lane); lds_base must be wave-uniform.  They are
// issued from inline assembly so that the compiler, which cannot tell the
// stage buffers apart, does not drain them before every LDS read; the
// kernel waits for them itself (s_waitcnt vmcnt) before the barrier that
// publishes a stage.
__device__ __forceinline__ void dma16(uint32_t lds_base, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_base), "v"(src)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(uint32_t lds_base, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_base), "v"(src)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Swizzle of the 16-byte chunks of an unpadded LDS row: chunk c of row r sits
// at position c ^ chunk_swizzle(r).  It keeps the 16-byte K reads (16 rows,
// one chunk) and the transpose reads of V (4 rows x 4 chunks per 32 lanes)
// free of bank conflicts.
template <int CHUNKS>
__device__ __forceinline__ int chunk_swizzle(int r) {
  if constexpr (CHUNKS == 16) return 4 * (r & 3) + ((r >> 2) & 3);
  else return 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(PrefillArgs a) {
  static_assert(Elem<T>::kBytes == 2, "16-bit caches (bf16 or fp16)");
  constexpr int MTOK = kPrefillRows / G;  // query tokens per workgroup
  constexpr int KS = D / 16;              // MFMA k-steps of QK^T
  constexpr int DB = D / 32;              // 32-wide d blocks of the output
  constexpr int CHUNKS = D / 8;           // 16-byte pieces per row
  constexpr int ROW_BYTES = D * 2;
  constexpr int kRowsPerDma = kWave / CHUNKS;             // rows one wave load covers
  // The copies are issued by the waves of the first context half (0-3):
  // they reach the barrier earlier, and issuing from all eight waves bunched
  // the copies behind the barrier (59.6 -> 57.1 us median on the mixed
  // prefill + decode step).
  constexpr int kCopyWaves = kPrefillWaves / 2;
  constexpr int kDmaPerWave = kStage / kCopyWaves / kRowsPerDma;  // per tensor
  constexpr int kRegionBytes = kStage * ROW_BYTES;        // K (or V) rows of a stage
  constexpr int kStageBytes = 2 * kRegionBytes;
  constexpr int kIdsOff = kStageBufs * kStageBytes;       // block-id ring
  static_assert(kDmaPerWave >= 1, "stage / wave mismatch");
  static_assert(kStageBufs * kStageBytes >= 4 * (16 * DB + 2) * kWave * 4, "merge scratch must fit");

  // Four stage buffers (K rows, then V rows, swizzled) and the block-id ring;
  // the stage buffers are reused for the final merge.
  __shared__ __attribute__((aligned(16))) char s_lds[kIdsOff + kIdRing * kIdSlotBytes];

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
  const uint32_t row_bytes = static_cast<uint32_t>(hkv) * ROW_BYTES;
  const uint32_t block_bytes = row_bytes << log2_bs;
  const int64_t trow = a.rows != nullptr ? a.rows[seq] : seq;
  const bool row_ok = trow >= 0 && trow < a.num_table_rows;
  const int32_t* bt = row_ok ? a.block_tables + trow * a.block_table_stride : kNoBlockRow;
  const int bt_stride = row_ok ? a.block_table_stride : 1;
  const char* kbase = reinterpret_cast<const char*>(a.key_cache) + kvh * ROW_BYTES;
  const char* vbase = reinterpret_cast<const char*>(a.value_cache) + kvh * ROW_BYTES;
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
      qreg[ks] = row_live ? ld16(qrow + ks * 16 + half * 8) : make_uint4(0, 0, 0, 0);
  }

  const int kv_end = min(ctx, start + tok0 + ntok);  // exclusive
  // Positions that have a block-table column (the rest are never read).
  const int kv_read = static_cast<int>(
      min(static_cast<int64_t>(kv_end), static_cast<int64_t>(bt_stride) << log2_bs));
  const int ntiles = (kv_end + kKvTile - 1) / kKvTile;
  const int nstages = (kv_end + kStage - 1) / kStage;
  const float scale = a.scale_log2e;
  const int last_col = bt_stride - 1;
  // Positions whose block id lies outside the pool are skipped, as the
  // decode kernels skip them: one pass over the row's columns tells whether
  // there are any (then every tile takes the masked path below).
  int bad_local = 0;
  for (int c = tid; c < ((kv_read + bs_mask) >> log2_bs); c += kPrefillThreads)
    bad_local |= static_cast<uint32_t>(bt[c]) >= static_cast<uint32_t>(a.total_blocks) ? 1 : 0;
  const bool bad_ids = __syncthreads_or(bad_local) != 0;
  // Tiles below this index need no mask for any row of the workgroup.
  const int first_masked = bad_ids ? 0 : min(start + tok0 + 1, kv_read) / kKvTile;

  // ---- staging ---------------------------------------------------------------
  // Block ids: wave 0 copies the table entries a stage needs (at most 64)
  // into slot (stage & 7) of an LDS ring, five stages ahead of use.  K/V:
  // copying wave w copies rows [16 w, 16 w + 16) of a stage (lane -> row
  // lane / CHUNKS of its load, chunk position lane % CHUNKS, fetching the
  // chunk that the swizzle puts there), three stages ahead.  Rows past the
  // readable context re-read its last row, and an out-of-pool block id
  // reads block 0 (finite values; their scores are masked).  Every copy is
  // issued unconditionally, so each wave's outstanding count is the same
  // every step.
  auto dma_ids = [&](int stage) {
    const int col = min(((stage * kStage) >> log2_bs) + lane, last_col);
    dma4(lds0 + kIdsOff + (stage & (kIdRing - 1)) * kIdSlotBytes, bt + col);
  };
  auto stage_ids = [&](int stage) {
    return reinterpret_cast<const int*>(s_lds + kIdsOff + (stage & (kIdRing - 1)) * kIdSlotBytes);
  };
  const int dma_row0 = (wave % kCopyWaves) * (kStage / kCopyWaves) + lane / CHUNKS;  // + j * kRowsPerDma
  auto dma_kv = [&](int stage, int buf_off) {
    if (wave >= kCopyWaves) return;
    const int col0 = (stage * kStage) >> log2_bs;
    const int* ids = stage_ids(stage);
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int r = dma_row0 + j * kRowsPerDma;  // row inside the stage
      const int pos = min(stage * kStage + r, kv_read - 1);
      // (clamped: past the last stage pos may precede the stage's first column)
      const int b = ids[min(max((pos >> log2_bs) - col0, 0), kIdSlotBytes / 4 - 1)];
      const uint32_t bb = static_cast<uint32_t>(b) < static_cast<uint32_t>(a.total_blocks)
                              ? static_cast<uint32_t>(b) : 0u;
      const int chunk = (lane % CHUNKS) ^ chunk_swizzle<CHUNKS>(r);
      const uint64_t off = static_cast<uint64_t>(bb) * block_bytes +
                           (static_cast<uint32_t>(pos & bs_mask) * row_bytes + chunk * 16);
      const uint32_t dst = __builtin_amdgcn_readfirstlane(
          lds0 + buf_off + (r - lane / CHUNKS) * ROW_BYTES);
      dma16(dst, kbase + off);
      dma16(dst + kRegionBytes, vbase + off);
    }
  };
  // Outstanding copies a copying wave leaves behind the stage it must see
  // landed: its K/V copies of one stage plus, for wave 0, one id copy.
  auto wait_stage = [&]() {
    if (wave == 0) wait_vmcnt<2 * kDmaPerWave + 1>();
    else if (wave < kCopyWaves) wait_vmcnt<2 * kDmaPerWave>();
  };

  // Prologue: ids of stages 0-4, then K/V of stages 0-2 (the loop's step st
  // copies K/V of stage st+3 and ids of stage st+5).
  if (wave == 0) {
#pragma unroll
    for (int s = 0; s < 5; ++s) dma_ids(s);
    wait_vmcnt<0>();
  }
  __syncthreads();
  dma_kv(0, 0);
  dma_kv(1, kStageBytes);
  dma_kv(2, 2 * kStageBytes);
  if (wave < kCopyWaves) wait_vmcnt<2 * kDmaPerWave>();  // stages 0 and 1 landed
  __syncthreads();

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m = kScoreFloor, l = 0.f;

  // Per-lane byte offsets of the MFMA operands inside a stage buffer (this
  // wave's half of the stage; chunk positions follow the swizzle).
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
      v_off[hi][db] = kRegionBytes + r * ROW_BYTES +
                      (((col >> 3) ^ chunk_swizzle<CHUNKS>(r)) * 16) + (col & 7) * 2;
    }
  }
  auto read_k = [&](int buf_off, uint4* ka) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) ka[ks] = *reinterpret_cast<const uint4*>(s_lds + buf_off + k_off[ks]);
  };
  auto read_vt = [&](int buf_off, uint4 (*va)[DB]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const char* base = s_lds + buf_off + ks * 16 * ROW_BYTES;
        const uint2 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(base + v_off[0][db]));
        const uint2 hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(base + v_off[1][db]));
        va[ks][db] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
  };

  // The scores of stage st+1 are computed while stage st's are turned into
  // probabilities: the QK MFMAs of the next tile are interleaved with the
  // exponentials of this one, so the matrix pipe and the VALU overlap inside
  // a wave.  Stage buffers rotate through byte offsets kept in scalars:
  // stage st (V read), st+1 (K read), st+2 (landed), st+3 (being copied).
  // (computed unconditionally -- unused when the wave has no tile -- so the
  // query loads are complete on every path into the loop and the compiler
  // adds no memory-counter wait inside it)
  f32x16 s_cur;
#pragma unroll
  for (int i = 0; i < 16; ++i) s_cur[i] = 0.f;
  {
    uint4 ka[KS];
    read_k(0, ka);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s_cur = mfma32<T>(ka[ks], qreg[ks], s_cur);
  }
  int off_cur = 0, off_next = kStageBytes, off_land = 2 * kStageBytes, off_copy = 3 * kStageBytes;

  auto step = [&](int st, const f32x16& s_in) {
    dma_kv(st + 3, off_copy);
    if (wave == 0) dma_ids(st + 5);
    const int t = 2 * st + kh;  // this wave's 32-token tile
    f32x16 s_next = s_in;
    if (t < ntiles) {
      // LDS operands: V^T of this stage, K of the next one (read even when
      // there is no next tile: the stale scores are never used).
      uint4 va[2][DB], ka[KS];
      read_vt(off_cur, va);
      read_k(off_next, ka);

      // ---- online softmax of s_in (unscaled scores; exp2 folds the scale)
      f32x16 s = s_in;
      const int kv0 = t * kKvTile;
      if (t >= first_masked) {
        const int* ids = stage_ids(st);
        const int col0 = (st * kStage) >> log2_bs;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kv = kv0 + 8 * (i >> 2) + 4 * half + (i & 3);
          bool off = kv > qpos || kv >= kv_read;
          if (bad_ids)
            off = off || static_cast<uint32_t>(ids[(kv >> log2_bs) - col0]) >=
                             static_cast<uint32_t>(a.total_blocks);
          if (off) s[i] = -INFINITY;
        }
      }
      float tmax = s[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
      tmax = max_halves(tmax);
      // Lazy rescale: the reference maximum m of a row moves only when the
      // tile's maximum exceeds it by more than kLazyRescale (log2 units), so
      // p <= 2^kLazyRescale; l and acc use the same m, and the result is the
      // same softmax.
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

      // ---- interleaved: S_next = K_next Q^T | P = exp2(S - m) | O^T += V^T P^T
#pragma unroll
      for (int i = 0; i < 16; ++i) s_next[i] = 0.f;
      float rsum = 0.f;
      uint4 pb[2];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s_next = mfma32<T>(ka[ks], qreg[ks], s_next);
        // two (D = 128) or four (D = 64) probabilities per QK step
#pragma unroll
        for (int j = ks * 16 / KS; j < (ks + 1) * 16 / KS; ++j) {
          s[j] = fast_exp2(fmaf(s[j], scale, -msc));
          rsum += s[j];
        }
        if ((ks + 1) * 16 / KS % 8 == 0) {
          const int c = (ks + 1) * 16 / KS / 8 - 1;
          pb[c].x = pack_half2<T>(s[8 * c + 0], s[8 * c + 1]);
          pb[c].y = pack_half2<T>(s[8 * c + 2], s[8 * c + 3]);
          pb[c].z = pack_half2<T>(s[8 * c + 4], s[8 * c + 5]);
          pb[c].w = pack_half2<T>(s[8 * c + 6], s[8 * c + 7]);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[db] = mfma32<T>(va[ks][db], pb[ks], acc[db]);
      rsum = sum_halves(rsum);
      l += rsum;
    }  // t < ntiles
    const int o = off_cur;
    off_cur = off_next;
    off_next = off_land;
    off_land = off_copy;
    off_copy = o;
    // Stage st+2 (read as K next step) and the ids of stage st+4 must have
    // landed before the barrier publishes them.
    wait_stage();
    __syncthreads();
    return s_next;
  };

  // Two steps per trip (the compiler then keeps the scores in place).  A
  // trailing step past the last stage computes nothing and only copies
  // clamped rows into a free buffer.
  for (int st = 0; st < nstages; st += 2) {
    const f32x16 s_mid = step(st, s_cur);
    s_cur = step(st + 1, s_mid);
  }
  // Let every copy land before the buffers are reused for the merge.
  wait_vmcnt<0>();
  __syncthreads();

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
                   ((first + tok0 + tok) * (hkv * a.group) + h) * static_cast<int64_t>(D);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = db * 32 + 8 * q4 + 4 * half;
      uint2 w;
      w.x = pack_half2<T>(acc[db][4 * q4 + 0] * inv, acc[db][4 * q4 + 1] * inv);
      w.y = pack_half2<T>(acc[db][4 * q4 + 2] * inv, acc[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = w;
    }
}

bool prefill_fast_path_supported(int dtype, int head_dim, int group, int block_size) {
  // bf16 / fp16: the MFMA kernel below; fp32: prefill_f32_kernel (VALU).
  if (dtype != PA_DTYPE_BF16 && dtype != PA_DTYPE_F16 && dtype != PA_DTYPE_F32) return false;
  if (head_dim != 64 && head_dim != 128) return false;
  if (group < 1 || group > kMaxDecodeQueryGroup) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  return true;
}

// Query tokens per work item: 128 rows over the heads of one workgroup (a
// sub-group of at most 8 when the group is larger).
int prefill_tile_for(int group) {
  return group > 0 ? kPrefillRows / (group / decode_sub_groups(group)) : kPrefillRows;
}

template <typename T, int D>
static hipError_t launch_prefill_d(const PrefillArgs& a, int group, int64_t num_items,
                                   hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(num_items * a.num_kv_heads * a.sub_groups));
  switch (group / a.sub_groups) {
    case 1: hipLaunchKernelGGL((prefill_kernel<T, D, 1>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<T, D, 2>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 3: hipLaunchKernelGGL((prefill_kernel<T, D, 3>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<T, D, 4>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 5: hipLaunchKernelGGL((prefill_kernel<T, D, 5>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 6: hipLaunchKernelGGL((prefill_kernel<T, D, 6>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 7: hipLaunchKernelGGL((prefill_kernel<T, D, 7>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((prefill_kernel<T, D, 8>), grid, dim3(kPrefillThreads), 0, s, a); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int dtype, int head_dim, int group,
                          int64_t num_items, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  if (dtype == PA_DTYPE_F32) return launch_prefill_f32(a, head_dim, group, num_items, stream);
  if (dtype == PA_DTYPE_BF16) {
    if (head_dim == 128) return launch_prefill_d<bf16_t, 128>(a, group, num_items, stream);
    if (head_dim == 64) return launch_prefill_d<bf16_t, 64>(a, group, num_items, stream);
  } else if (dtype == PA_DTYPE_F16) {
    if (head_dim == 128) return launch_prefill_d<f16_t, 128>(a, group, num_items, stream);
    if (head_dim == 64) return launch_prefill_d<f16_t, 64>(a, group, num_items, stream);
  }
  return hipErrorNotSupported;
}

}  // namespace pa
