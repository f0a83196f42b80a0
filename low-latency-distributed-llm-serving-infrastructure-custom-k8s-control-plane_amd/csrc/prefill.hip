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
// with v_mfma_f32_32x32x16_bf16.  In the 32x32 accumulator lane l holds
// column l % 32 and rows 8*(i/4) + 4*(l/32) + (i%4), i = 0..15, so the
// softmax max/sum of a query row needs only its own 16 values plus the
// partner lane l ^ 32, and the probabilities a lane holds are the B operand
// of the PV product with the context index of k-slot j being
// 8*(j/4) + 4*(l/32) + (j%4) inside each 16-token step.
//
// K and V are staged row-major in LDS (16-byte stores).  The V^T operand is
// read with the gfx950 LDS transpose read ds_read_b64_tr_b16: inside each
// group of 16 lanes, lane i receives element j from the 8-byte word
// addressed by lane (i/4 + 4j), element i%4.  Lane i of a group therefore
// addresses V[kv0 + (i/4)][d0 + 4*(i%4)] and receives V[kv0 + j][d0 + i],
// j = 0..3: four context tokens of its own output column.
//
// Pipeline (one barrier per 64-token stage): three LDS stage buffers hold
// stage t (its V is read), stage t+1 (its K is read: the scores of the next
// tile are computed while this tile's exponentials run) and stage t+2 (being
// stored from registers).  Stages t+3 and t+4 are in flight in two register
// sets, and block ids are fetched two stages before their rows.  Every
// global load is unconditional, so the compiler's memory-counter waits are
// exact and never drain the younger stage.
// Masking is applied only to tiles that cross the causal diagonal or the end
// of the context, and the accumulator is rescaled only when some row's
// maximum grew by more than 2^8 over the reference maximum in use.
//
// Reference: the block-diagonal causal mask of app/model/paged_attention.py:
// 92-118 applied by SDPA (paged_attention.py:170-178); query token j of a
// sequence at position start + j attends context positions [0, start + j].
#include "pa_common.hpp"
#include "pa_launch.hpp"

namespace pa {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4v __attribute__((ext_vector_type(4)));

constexpr int kPrefillThreads = 512;  // 4 row groups x 2 context halves
constexpr int kPrefillRows = 128;  // query rows per workgroup
constexpr int kKvTile = 32;        // context tokens per wave per stage
constexpr int kStage = 2 * kKvTile;  // context tokens per LDS stage
constexpr float kLazyRescale = 8.f;  // log2 headroom before the row maximum moves
constexpr int kStageBufs = 3;       // LDS stage buffers in flight

__device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                 __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
}

// ds_read_b64_tr_b16 at an LDS address (see the header comment).
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) i16x4v lds_i16x4;
  const i16x4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

template <int D, int G>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(PrefillArgs a) {
  constexpr int MTOK = kPrefillRows / G;  // query tokens per workgroup
  constexpr int KS = D / 16;              // MFMA k-steps of QK^T
  constexpr int DB = D / 32;              // 32-wide d blocks of the output
  constexpr int CHUNKS = D / 8;           // 16-byte pieces per row
  constexpr int PIECES = kStage * CHUNKS / kPrefillThreads;  // per thread, K and V each
  // LDS row strides (elements): K rows 4 banks apart (conflict-free 16-byte
  // reads of 16 rows), V rows 16 banks apart (conflict-free transpose reads).
  constexpr int KSTR = D + 8;
  constexpr int VSTR = D + 32;
  static_assert(PIECES >= 1 && kStage * CHUNKS % kPrefillThreads == 0, "stage / thread mismatch");
  constexpr int kStageElems = kStage * (KSTR + VSTR);
  static_assert(kStageBufs * kStageElems * 2 >= 4 * (16 * (D / 32) + 2) * kWave * 4,
                "merge scratch must fit");

  // Three stage buffers (K rows then V rows); reused for the final merge.
  __shared__ __attribute__((aligned(16))) uint16_t s_lds[kStageBufs * kStageElems];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int rg = wave & 3;   // row group
  const int kh = wave >> 2;  // context half of every stage
  const int hkv = a.num_kv_heads;
  // Highest item first: the last query tiles of a sequence see the most context.
  const int64_t blk_id = static_cast<int64_t>(gridDim.x) - 1 - blockIdx.x;
  const int64_t item = blk_id / hkv;
  const int kvh = static_cast<int>(blk_id - item * hkv);
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
  const uint32_t row_bytes = static_cast<uint32_t>(hkv) * D * 2;
  const uint32_t block_bytes = row_bytes << log2_bs;
  const int32_t* bt = a.block_tables + static_cast<int64_t>(seq) * a.block_table_stride;
  const char* kbase = reinterpret_cast<const char*>(a.key_cache) + kvh * D * 2;
  const char* vbase = reinterpret_cast<const char*>(a.value_cache) + kvh * D * 2;

  // This lane's query row.
  const int row = rg * 32 + (lane & 31);
  const int half = lane >> 5;
  const int g = row / MTOK;
  const int tok = row - g * MTOK;
  // Rows past G * MTOK (when G does not divide 128) belong to no head.
  const bool row_live = tok < ntok && g < G;
  const int qpos = start + tok0 + tok;  // causal limit (inclusive)
  const int h = kvh * G + g;

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
      min(static_cast<int64_t>(kv_end), static_cast<int64_t>(a.block_table_stride) << log2_bs));
  const int ntiles = (kv_end + kKvTile - 1) / kKvTile;
  const int nstages = (kv_end + kStage - 1) / kStage;
  // Tiles below this index need no mask for any row of the workgroup.
  const int first_masked = min(start + tok0 + 1, kv_end) / kKvTile;
  const float scale = a.scale_log2e;

  // ---- staging: thread piece p covers stage row ld_row + p*kRowsPerPass,
  // 16 bytes at chunk ld_ch, of K and of V.  Every load is issued
  // unconditionally (no branch around a memory instruction), so the memory
  // counter waits stay exact and two stages are in flight in registers:
  //  - rows past the readable context re-read its last row (finite; their
  //    scores are masked);
  //  - an out-of-pool block id reads block 0 and is zeroed before it
  //    reaches LDS (the reference leaves such ids undefined).
  // Block ids are fetched two iterations before their rows are loaded.
  constexpr int kRowsPerPass = kPrefillThreads / CHUNKS;
  const int ld_row = tid / CHUNKS;
  const uint32_t lane_bytes = static_cast<uint32_t>(tid - ld_row * CHUNKS) * 16;
  const int ld_col = (tid - ld_row * CHUNKS) * 8;

  auto row_of = [&](int stage, int p) {
    return min(stage * kStage + ld_row + p * kRowsPerPass, kv_read - 1);
  };
  auto fetch_blocks = [&](int stage, int* out) {
#pragma unroll
    for (int p = 0; p < PIECES; ++p) out[p] = bt[row_of(stage, p) >> log2_bs];
  };
  auto load_tile = [&](int stage, const int* bl, uint4* kd, uint4* vd, uint32_t& bad) {
    bad = 0;
#pragma unroll
    for (int p = 0; p < PIECES; ++p) {
      const int pos = row_of(stage, p);
      const bool ok = static_cast<uint32_t>(bl[p]) < static_cast<uint32_t>(a.total_blocks);
      const uint32_t b = ok ? static_cast<uint32_t>(bl[p]) : 0u;
      const uint64_t off = static_cast<uint64_t>(b) * block_bytes +
                           (static_cast<uint32_t>(pos & bs_mask) * row_bytes + lane_bytes);
      kd[p] = ld16(kbase + off);
      vd[p] = ld16(vbase + off);
      bad |= ok ? 0u : (1u << p);
    }
  };
  auto store_tile = [&](int off, uint4* kd, uint4* vd, uint32_t bad) {
    if (__builtin_amdgcn_ballot_w64(bad != 0) != 0) {
#pragma unroll
      for (int p = 0; p < PIECES; ++p)
        if ((bad >> p) & 1u) kd[p] = vd[p] = make_uint4(0, 0, 0, 0);
    }
    uint16_t* sk = s_lds + off;
    uint16_t* sv = sk + kStage * KSTR;
#pragma unroll
    for (int p = 0; p < PIECES; ++p) {
      const int r = ld_row + p * kRowsPerPass;
      *reinterpret_cast<uint4*>(&sk[r * KSTR + ld_col]) = kd[p];
      *reinterpret_cast<uint4*>(&sv[r * VSTR + ld_col]) = vd[p];
    }
  };

  // Two register stages (X: even iterations, Y: odd) and their block ids.
  uint4 kx[PIECES], vx[PIECES], ky[PIECES], vy[PIECES];
  int bx[PIECES], by[PIECES];
  uint32_t badx, bady;

  // Prologue: stages 0 and 1 into LDS buffers 0 and 1, stages 2 and 3 in
  // registers, block ids of stages 4 and 5.
  fetch_blocks(0, bx);
  fetch_blocks(1, by);
  load_tile(0, bx, kx, vx, badx);
  load_tile(1, by, ky, vy, bady);
  fetch_blocks(2, bx);
  fetch_blocks(3, by);
  store_tile(0, kx, vx, badx);
  store_tile(kStageElems, ky, vy, bady);
  // (same issue order as the loop, so its memory counter waits hold on
  // entry too)
  load_tile(2, bx, kx, vx, badx);
  fetch_blocks(4, bx);
  load_tile(3, by, ky, vy, bady);
  fetch_blocks(5, by);
  __syncthreads();

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m = kScoreFloor, l = 0.f;

  // Per-lane LDS offsets of the MFMA operands (inside this wave's half).
  const int k_off = (kh * kKvTile + (lane & 31)) * KSTR + half * 8;
  const int li = lane & 15;
  const int v_off = kStage * KSTR + (kh * kKvTile + 4 * half + (li >> 2)) * VSTR +
                    16 * ((lane >> 4) & 1) + 4 * (li & 3);

  // The scores of stage st+1 are computed while stage st's are turned into
  // probabilities: the QK MFMAs of the next tile are interleaved with the
  // exponentials of this one, so the matrix pipe and the VALU overlap inside
  // a wave.  Stage buffers rotate through LDS offsets kept in scalars.
  f32x16 s_cur;
#pragma unroll
  for (int i = 0; i < 16; ++i) s_cur[i] = 0.f;
  int off_cur = 0, off_next = kStageElems, off_store = 2 * kStageElems;
  if (kh < ntiles) {
    uint4 ka[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      ka[ks] = *reinterpret_cast<const uint4*>(s_lds + k_off + ks * 16);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s_cur = mfma32(ka[ks], qreg[ks], s_cur);
  }

  // One pipeline step: stage st+2 registers -> LDS, stage st+4 loads issued
  // into the same registers, block ids of stage st+6, then the tile of
  // stage st.  Returns the scores of stage st+1.
  auto step = [&](int st, uint4* kd, uint4* vd, int* bl, uint32_t& bad, const f32x16& s_in) {
    store_tile(off_store, kd, vd, bad);
    load_tile(st + 4, bl, kd, vd, bad);
    fetch_blocks(st + 6, bl);
    const int t = 2 * st + kh;  // this wave's 32-token tile
    f32x16 s_next = s_in;
    if (t < ntiles) {
      // LDS operands: V^T of this stage, K of the next one (read even when
      // there is no next tile: the stale scores are never used).
      const uint16_t* sv = s_lds + off_cur + v_off;
      uint4 va[2][DB];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const uint16_t* p0 = sv + ks * 16 * VSTR + db * 32;
          const uint2 lo = lds_read_tr16(p0);
          const uint2 hi = lds_read_tr16(p0 + 8 * VSTR);
          va[ks][db] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
      const uint16_t* sk = s_lds + off_next + k_off;
      uint4 ka[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) ka[ks] = *reinterpret_cast<const uint4*>(sk + ks * 16);

      // ---- online softmax of s_in (unscaled scores; exp2 folds the scale)
      f32x16 s = s_in;
      const int kv0 = t * kKvTile;
      if (t >= first_masked) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kv = kv0 + 8 * (i >> 2) + 4 * half + (i & 3);
          if (kv > qpos || kv >= kv_end) s[i] = -INFINITY;
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
        s_next = mfma32(ka[ks], qreg[ks], s_next);
        // two (D = 128) or four (D = 64) probabilities per QK step
#pragma unroll
        for (int j = ks * 16 / KS; j < (ks + 1) * 16 / KS; ++j) {
          s[j] = fast_exp2(fmaf(s[j], scale, -msc));
          rsum += s[j];
        }
        if ((ks + 1) * 16 / KS % 8 == 0) {
          const int c = (ks + 1) * 16 / KS / 8 - 1;
          pb[c].x = pack_bf16x2(s[8 * c + 0], s[8 * c + 1]);
          pb[c].y = pack_bf16x2(s[8 * c + 2], s[8 * c + 3]);
          pb[c].z = pack_bf16x2(s[8 * c + 4], s[8 * c + 5]);
          pb[c].w = pack_bf16x2(s[8 * c + 6], s[8 * c + 7]);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[db] = mfma32(va[ks][db], pb[ks], acc[db]);
      rsum = sum_halves(rsum);
      l += rsum;
    }  // t < ntiles
    const int o = off_cur;
    off_cur = off_next;
    off_next = off_store;
    off_store = o;
    __syncthreads();
    return s_next;
  };

  // Two steps per trip so that the register stages and block-id sets
  // alternate by name.  A trailing step past the last stage computes
  // nothing (its tiles are past ntiles) and only reloads clamped rows.
  for (int st = 0; st < nstages; st += 2) {
    const f32x16 s_mid = step(st, kx, vx, bx, badx, s_cur);
    s_cur = step(st + 1, ky, vy, by, bady, s_mid);
  }

  // ---- merge the two context halves of every row group ---------------------
  // (the loop ended on a barrier, so the stage buffers are free)
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
                   ((first + tok0 + tok) * (hkv * G) + h) * static_cast<int64_t>(D);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = db * 32 + 8 * q4 + 4 * half;
      uint2 w;
      w.x = pack_bf16x2(acc[db][4 * q4 + 0] * inv, acc[db][4 * q4 + 1] * inv);
      w.y = pack_bf16x2(acc[db][4 * q4 + 2] * inv, acc[db][4 * q4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = w;
    }
}

bool prefill_fast_path_supported(int dtype, int head_dim, int group, int block_size) {
  if (dtype != PA_DTYPE_BF16) return false;
  if (head_dim != 64 && head_dim != 128) return false;
  if (group < 1 || group > 8) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  return true;
}

int prefill_tile_for(int group) { return group > 0 ? kPrefillRows / group : kPrefillRows; }

template <int D>
static hipError_t launch_prefill_d(const PrefillArgs& a, int group, int64_t num_items,
                                   hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(num_items * a.num_kv_heads));
  switch (group) {
    case 1: hipLaunchKernelGGL((prefill_kernel<D, 1>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<D, 2>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 3: hipLaunchKernelGGL((prefill_kernel<D, 3>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<D, 4>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 5: hipLaunchKernelGGL((prefill_kernel<D, 5>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 6: hipLaunchKernelGGL((prefill_kernel<D, 6>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 7: hipLaunchKernelGGL((prefill_kernel<D, 7>), grid, dim3(kPrefillThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((prefill_kernel<D, 8>), grid, dim3(kPrefillThreads), 0, s, a); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int dtype, int head_dim, int group,
                          int64_t num_items, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  if (dtype != PA_DTYPE_BF16) return hipErrorNotSupported;
  if (head_dim == 128) return launch_prefill_d<128>(a, group, num_items, stream);
  if (head_dim == 64) return launch_prefill_d<64>(a, group, num_items, stream);
  return hipErrorNotSupported;
}

}  // namespace pa
