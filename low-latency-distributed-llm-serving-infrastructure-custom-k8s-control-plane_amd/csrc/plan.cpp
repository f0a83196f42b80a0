// Host-side step planning (pa_plan_step): sizes every buffer pa_pack fills
// from the host arrays the scheduler already holds, and chooses the decode
// split-K partition.  Plain C++: no HIP call, so the host can size and
// launch a step without reading anything back from the device.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "pa_error.hpp"
#include "paged_attention_amd.h"

namespace {

// The partition rule's bounds (tokens): largest and smallest partition and
// the smallest one a full-chip launch may take.
constexpr int64_t kMaxPartition = PA_DECODE_MAX_PARTITION;
constexpr int64_t kMinPartition = 64;
constexpr int64_t kMinFullChipPartition = 256;

// The latency model of a step that cannot fill the chip, measured on MI355X
// over 32-layer decode loops whose caches are read cold: one partition
// workgroup reads about 21 GB/s on its own (0.049 us per token of a 1 KB
// K+V row), about 310 of them saturate HBM (6.5 TB/s), and the split-K merge
// of a sequence costs about 2 us per batch of 8 partials (partial stores,
// the arrival atomic and the partial loads are dependent round trips).
constexpr double kUsPerToken = 0.049;
constexpr double kSaturatingWorkgroups = 310.0;
constexpr double kMergeUsPerBatch = 2.0;
constexpr int64_t kMergeBatch = 8;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct DecodeContexts {
  const int64_t* starts;
  const int64_t* counts;
  int32_t n;
  // Decode workgroups of the step at partition p (items x width).
  int64_t workgroups(int64_t p, int64_t width) const {
    int64_t items = 0;
    for (int32_t i = 0; i < n; ++i)
      if (counts[i] == 1) items += ceil_div(starts[i] + 1, p);
    return items * width;
  }
};

int64_t choose_partition(const DecodeContexts& d, const PaPlanParams& p, int64_t longest) {
  const int64_t hkv = p.num_kv_heads > 0 ? p.num_kv_heads : 1;
  const int64_t hq = p.num_query_heads > 0 ? p.num_query_heads : 4 * hkv;
  const int64_t group = hq / hkv > 0 ? hq / hkv : 1;
  const int64_t per_cu = p.workgroups_per_cu > 0 ? p.workgroups_per_cu : (group == 1 ? 5 : 4);
  const int64_t slots = (p.compute_units > 0 ? p.compute_units : 256) * per_cu;
  const int64_t width = p.workgroups_per_item > 0 ? p.workgroups_per_item : hkv;
  // A launch that fills the chip: every resident slot gets 1.5 workgroups.
  for (int64_t part = kMaxPartition; part > kMinFullChipPartition; part /= 2)
    if (d.workgroups(part, width) >= 3 * slots / 2) return part;
  // A latency-bound step: the partition of least modelled time -- the
  // longest workgroup's read (slowed by its share of HBM when more than the
  // saturating count run at once, times the waves of workgroups) plus the
  // merge of the longest sequence's partials.  Ties (two bandwidth-bound
  // launches read the same bytes) go to the shorter partition: its extra
  // workgroups measured faster.
  if (d.workgroups(kMinPartition, width) == 0) return kMinPartition;  // no decode
  int64_t best = kMinPartition;
  double best_us = -1.0;
  for (int64_t part = kMinPartition; part <= kMaxPartition; part *= 2) {
    const int64_t wgs = d.workgroups(part, width);
    const double active = static_cast<double>(wgs < slots ? wgs : slots);
    const double share = active > kSaturatingWorkgroups ? active / kSaturatingWorkgroups : 1.0;
    const double waves = static_cast<double>(ceil_div(wgs, slots));
    const int64_t parts = ceil_div(longest, part);
    const double merge = parts > 1 ? kMergeUsPerBatch * static_cast<double>(ceil_div(parts, kMergeBatch)) : 0.0;
    const double us = static_cast<double>(part) * kUsPerToken * share * waves + merge;
    if (best_us < 0.0 || us < best_us * (1.0 - 1e-9)) {
      best = part;
      best_us = us;
    }
  }
  return best;
}

int plan_fail(PaStepPlan* plan, int32_t seq, const char* what) {
  if (plan != nullptr) plan->bad_seq = seq;
  return pa::set_error(PA_ERR_INVALID_ARGUMENT, "pa_plan_step: %s", what);
}

}  // namespace

extern "C" {

int pa_plan_step(const int64_t* starts, const int64_t* counts, const int64_t* allocated, int32_t num_seqs,
                 PaPlanParams params, PaStepPlan* plan) {
  if (plan == nullptr) return plan_fail(nullptr, -1, "plan must not be NULL");
  memset(plan, 0, sizeof(*plan));
  plan->bad_seq = -1;
  if (num_seqs < 0) return plan_fail(plan, -1, "negative num_seqs");
  if (num_seqs > 0 && (starts == nullptr || counts == nullptr))
    return plan_fail(plan, -1, "start_positions and new_token_counts are required");
  if (params.block_size <= 0 || params.prefill_tile <= 0 || params.partition_size < 0)
    return plan_fail(plan, -1, "block_size and prefill_tile must be positive, partition_size non-negative");
  int64_t longest_decode = 0;
  for (int32_t i = 0; i < num_seqs; ++i) {
    const int64_t s = starts[i], c = counts[i];
    char what[160];
    if (s < 0 || c < 0) {
      snprintf(what, sizeof(what), "sequence %d: start_token (%lld) and token_count (%lld) must be non-negative",
               i, static_cast<long long>(s), static_cast<long long>(c));
      return plan_fail(plan, i, what);
    }
    if (allocated != nullptr && s + c > allocated[i]) {
      snprintf(what, sizeof(what), "sequence %d: tokens [%lld, %lld) exceed allocated tokens (%lld)", i,
               static_cast<long long>(s), static_cast<long long>(s + c), static_cast<long long>(allocated[i]));
      return plan_fail(plan, i, what);
    }
    const int64_t ctx = s + c;
    plan->num_query_tokens += c;
    plan->num_context_tokens += ctx;
    if (ctx > plan->max_context) plan->max_context = ctx;
    if (c > plan->max_new_tokens) plan->max_new_tokens = c < INT32_MAX ? static_cast<int32_t>(c) : INT32_MAX;
    const int64_t blocks = ceil_div(ctx, params.block_size);
    if (blocks > plan->max_blocks) plan->max_blocks = static_cast<int32_t>(blocks);
    if (c == 1) {
      ++plan->num_decode_seqs;
      if (ctx > longest_decode) longest_decode = ctx;
    } else if (c > 1) {
      ++plan->num_prefill_seqs;
      plan->num_prefill_items += ceil_div(c, params.prefill_tile);
    }
  }
  if (plan->num_context_tokens >= (int64_t(1) << 31))
    return plan_fail(plan, -1, "a step's context tokens must stay below 2^31");
  const DecodeContexts d{starts, counts, num_seqs};
  const int64_t part = params.partition_size > 0 ? params.partition_size
                                                 : choose_partition(d, params, longest_decode);
  plan->partition_size = static_cast<int32_t>(part);
  for (int32_t i = 0; i < num_seqs; ++i) {
    if (counts[i] != 1) continue;
    const int64_t ctx = starts[i] + 1;
    plan->num_decode_items += ceil_div(ctx, part);
    plan->num_merge_items += ctx > part ? 1 : 0;
  }
  return PA_OK;
}

}  // extern "C"
