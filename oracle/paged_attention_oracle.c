/*
 * ORACLE -- test infrastructure only.  Nothing in the product path links or
 * calls this file; only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py load it, and only to check the HIP path against.
 *
 * CPU restatement of the reference paged-attention kernel
 * (csrc/src/paged_kernels.cpp:7-105, ABI csrc/include/paged_kernels.h:11-34).
 * Written from the kernel's semantics; the floating-point operations are
 * issued in the same order as the reference so that the two agree bit for bit
 * when built with the reference flags (-O3 -fopenmp, no fast-math):
 *
 *   for every (query token q, query head h):                  [:49-50]
 *     h_kv  = h / (H_q / H_kv)                                 [:51]
 *     s_c   = (sum_d q[d]*k_c[d], d ascending) * scaling      [:66-70]
 *             or -inf where mask[q][c] == 0                    [:58-61]
 *     m     = max_c s_c, and 0 when every s_c is -inf          [:72,75]
 *     p_c   = expf(s_c - m) where s_c > -1e30, else 0          [:77-85]
 *     p_c  *= 1/sum_c p_c when the sum is positive             [:86-91]
 *     out[d]= sum_c p_c * v_c[d], c ascending                  [:94-102]
 *   num_context_tokens == 0  ->  output is all zeros           [:30-34]
 *
 * Layouts (element offsets):
 *   query   [1, H_q, T, D]      q + h*T*D + t*D               [:42,52]
 *   caches  (L, N, bs, H_kv, D) layer*N*bs*H_kv*D + slot*H_kv*D + h_kv*D
 *   mask    uint8 [T, C]        row-major                      [:58]
 *   output  [T, H_q, D]         token-major                    [:43,93]
 *   scratch fp32 [T, H_q, C]                                    [:44,53]
 *
 * Parity pinned by tests/test_oracle_attention.py: bit-identical to the
 * reference object built by oracle/Makefile (target `ref`), and within 1e-5
 * of a float64 closed-form softmax attention on ragged / GQA / causal cases.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

typedef struct {
    int32_t num_query_heads;
    int32_t num_query_tokens;
    int32_t head_dim;
    int32_t num_layers;
    int32_t total_blocks;
    int32_t block_size;
    int32_t num_kv_heads;
    int32_t num_context_tokens;
} OraclePagedAttentionDims;

static void attend_one_row(const float *qv, const float *kbase, const float *vbase,
                           int64_t row_stride, int32_t dim, int32_t nctx,
                           const int32_t *slots, const uint8_t *mask_row,
                           float scaling, float *scores, float *out)
{
    const float neg_inf = -INFINITY;
    float peak = neg_inf;
    for (int32_t c = 0; c < nctx; ++c) {
        if (mask_row[c] == 0) {
            scores[c] = neg_inf;
            continue;
        }
        const float *kr = kbase + (int64_t)slots[c] * row_stride;
        float acc = 0.0f;
        for (int32_t d = 0; d < dim; ++d)
            acc += qv[d] * kr[d];
        float s = acc * scaling;
        scores[c] = s;
        if (s > peak)
            peak = s;
    }
    if (peak == neg_inf)
        peak = 0.0f;

    float total = 0.0f;
    for (int32_t c = 0; c < nctx; ++c) {
        if (scores[c] > -1e30f) {
            scores[c] = expf(scores[c] - peak);
            total += scores[c];
        } else {
            scores[c] = 0.0f;
        }
    }
    if (total > 0.0f) {
        const float r = 1.0f / total;
        for (int32_t c = 0; c < nctx; ++c)
            scores[c] *= r;
    }

    for (int32_t d = 0; d < dim; ++d) {
        float acc = 0.0f;
        for (int32_t c = 0; c < nctx; ++c)
            acc += scores[c] * vbase[(int64_t)slots[c] * row_stride + d];
        out[d] = acc;
    }
}

void oracle_paged_attention(const float *query, const float *key_cache,
                            const float *value_cache, int32_t layer_idx,
                            OraclePagedAttentionDims dims,
                            const int32_t *gather_slots,
                            const uint8_t *attention_mask, float scaling,
                            float *output, float *scratch, void *stream)
{
    (void)stream;
    const int32_t hq = dims.num_query_heads;
    const int32_t nt = dims.num_query_tokens;
    const int32_t dim = dims.head_dim;
    const int32_t hkv = dims.num_kv_heads;
    const int32_t nctx = dims.num_context_tokens;

    if (nctx == 0) {
        memset(output, 0, (size_t)nt * hq * dim * sizeof(float));
        return;
    }
    const int64_t row_stride = (int64_t)hkv * dim;
    const int64_t layer_span = (int64_t)dims.total_blocks * dims.block_size * row_stride;
    const float *kl = key_cache + (int64_t)layer_idx * layer_span;
    const float *vl = value_cache + (int64_t)layer_idx * layer_span;
    const int32_t group = hq / hkv;

#pragma omp parallel for collapse(2)
    for (int32_t t = 0; t < nt; ++t) {
        for (int32_t h = 0; h < hq; ++h) {
            const int32_t g = h / group;
            attend_one_row(query + (int64_t)h * nt * dim + (int64_t)t * dim,
                           kl + (int64_t)g * dim, vl + (int64_t)g * dim,
                           row_stride, dim, nctx, gather_slots,
                           attention_mask + (int64_t)t * nctx, scaling,
                           scratch + ((int64_t)t * hq + h) * nctx,
                           output + (int64_t)t * hq * dim + (int64_t)h * dim);
        }
    }
}

/*
 * Per-sequence driver used for the large workloads, where the flat call's
 * T x C mask and T x H_q x C scratch do not fit: one attention call per
 * sequence with that sequence's own slots and a causal mask (decode = all
 * ones).  This is the call pattern of the CPU baseline for the long-context
 * decode and mixed-step workloads.  `fn` is the kernel to drive: either
 * oracle_paged_attention or the reference's own paged_attention symbol from
 * the library built by oracle/Makefile; both share the reference ABI.
 *
 *   query  [H_q, T_total, D] head-major (the reference layout)
 *   starts / counts: per-sequence start position and new-token count
 *   slot_offsets: exclusive prefix over (start+count) into `slots`
 *   output [T_total, H_q, D]
 *   mask / scratch / slot_buf / q_buf / o_buf: caller buffers of at least
 *   max_count*max_ctx bytes, max_count*H_q*max_ctx floats, max_ctx ints,
 *   max_count*H_q*D floats and max_count*H_q*D floats.
 *   kernel_seconds (out): steady-clock time spent inside `fn` only.
 */
#include <time.h>

typedef void (*paged_attention_fn)(const float *, const float *, const float *,
                                   int32_t, OraclePagedAttentionDims,
                                   const int32_t *, const uint8_t *, float,
                                   float *, float *, void *);

static double now_seconds(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

void oracle_paged_attention_per_sequence(
    paged_attention_fn fn, const float *query, const float *key_cache,
    const float *value_cache, int32_t layer_idx, OraclePagedAttentionDims dims,
    int32_t num_seqs, const int64_t *starts, const int64_t *counts,
    const int64_t *slots, const int64_t *slot_offsets, float scaling,
    float *output, uint8_t *mask, float *scratch, int32_t *slot_buf,
    float *q_buf, float *o_buf, double *kernel_seconds)
{
    const int32_t hq = dims.num_query_heads;
    const int32_t dim = dims.head_dim;
    const int32_t t_total = dims.num_query_tokens;
    int64_t qbase = 0;
    double spent = 0.0;
    if (fn == 0)
        fn = oracle_paged_attention;
    for (int32_t s = 0; s < num_seqs; ++s) {
        const int32_t n = (int32_t)counts[s];
        const int32_t ctx = (int32_t)(starts[s] + counts[s]);
        if (n == 0)
            continue;
        for (int32_t c = 0; c < ctx; ++c)
            slot_buf[c] = (int32_t)slots[slot_offsets[s] + c];
        for (int32_t i = 0; i < n; ++i)
            for (int32_t c = 0; c < ctx; ++c)
                mask[(int64_t)i * ctx + c] = (uint8_t)(c <= starts[s] + i);
        for (int32_t h = 0; h < hq; ++h)
            memcpy(q_buf + (int64_t)h * n * dim,
                   query + (int64_t)h * t_total * dim + qbase * dim,
                   (size_t)n * dim * sizeof(float));
        OraclePagedAttentionDims sd = dims;
        sd.num_query_tokens = n;
        sd.num_context_tokens = ctx;
        const double t0 = now_seconds();
        fn(q_buf, key_cache, value_cache, layer_idx, sd, slot_buf, mask,
           scaling, o_buf, scratch, 0);
        spent += now_seconds() - t0;
        memcpy(output + qbase * hq * dim, o_buf, (size_t)n * hq * dim * sizeof(float));
        qbase += n;
    }
    if (kernel_seconds)
        *kernel_seconds = spent;
}
