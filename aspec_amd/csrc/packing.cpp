// Work-aware row packing: which pooled samples form the next packed rows, one row per
// data-parallel rank. Host code only (integer bookkeeping over a sample pool); compiled by the
// host compiler into the same library as the kernels, so a controller binds one C ABI.
//
//   aspec_count_eligible_anchor_starts  count_eligible_anchor_starts (aspec/controller/packing.py:43-67)
//   aspec_pack_work_aware_rows          pack_work_aware_rows         (aspec/controller/packing.py:87-167)
//
// Placement follows the reference's policy step for step: the first `dp_size` samples seed one row
// each, the rest are visited by useful-work density (ratio as an IEEE double quotient, then work,
// then length, all descending, then index) and each goes to the fitting row with the least slack
// left (ties: lower row index), until `max_selected` samples are taken. Rows are then ordered by
// token count, descending (ties: lower row index). The best-fit query is an ordered-set lookup,
// O(log dp) per sample, so a pool of n samples packs in O(n log n).
#include <stdint.h>

#include <algorithm>
#include <numeric>
#include <set>
#include <utility>
#include <vector>

#include "../../include/aspec_amd.h"

namespace aspec {
int set_error(int code, const char* fmt, ...);  // status.hip
}  // namespace aspec

namespace {

// Integers that a double holds exactly: the density ratio must equal Python's int / int quotient.
constexpr int64_t kExactDouble = int64_t{1} << 53;

}  // namespace

extern "C" int aspec_count_eligible_anchor_starts(const int64_t* runs, const int64_t* run_offsets,
                                                  const int64_t* sample_lengths, int64_t num_samples,
                                                  int64_t block_size, int64_t* counts_out) {
  using aspec::set_error;
  if (num_samples < 0) return set_error(ASPEC_ERR_INVALID, "count_eligible_anchor_starts: num_samples < 0");
  if (num_samples == 0) return ASPEC_OK;
  if (!run_offsets || !sample_lengths || !counts_out)
    return set_error(ASPEC_ERR_INVALID, "count_eligible_anchor_starts: null pointer");
  if (run_offsets[0] != 0) return set_error(ASPEC_ERR_INVALID, "count_eligible_anchor_starts: run_offsets[0] != 0");
  for (int64_t s = 0; s < num_samples; ++s) {
    const int64_t begin = run_offsets[s], end = run_offsets[s + 1];
    if (end < begin) return set_error(ASPEC_ERR_INVALID, "count_eligible_anchor_starts: run_offsets decrease at %lld",
                                      static_cast<long long>(s));
    if (end > begin && !runs) return set_error(ASPEC_ERR_INVALID, "count_eligible_anchor_starts: null runs");
    for (int64_t r = begin; r < end; ++r)
      if (runs[r] < 0)
        return set_error(ASPEC_ERR_INVALID, "packed_loss_mask run lengths must be non-negative");
  }
  for (int64_t s = 0; s < num_samples; ++s) {
    const int64_t length = sample_lengths[s];
    if (length <= 0 || block_size <= 0) {
      counts_out[s] = 0;
      continue;
    }
    // Anchors start at positions [0, length - block_size]; runs alternate unsupervised/supervised,
    // starting with an unsupervised run, so odd runs are the supervised spans.
    const int64_t prefix = std::max<int64_t>(length - block_size + 1, 0);
    int64_t cursor = 0, count = 0;
    for (int64_t r = run_offsets[s]; r < run_offsets[s + 1]; ++r) {
      const int64_t stop = cursor + runs[r];
      if ((r - run_offsets[s]) & 1) count += std::max<int64_t>(0, std::min(stop, prefix) - std::min(cursor, prefix));
      cursor = stop;
    }
    counts_out[s] = count;
  }
  return ASPEC_OK;
}

extern "C" int aspec_pack_work_aware_rows(const int64_t* lengths, const int64_t* useful_work, int64_t count,
                                          int64_t dp_size, int64_t max_seq_length, int64_t max_selected,
                                          int64_t* row_offsets, int64_t* row_samples, int64_t* row_tokens_out) {
  using aspec::set_error;
  if (dp_size <= 0 || max_seq_length <= 0)
    return set_error(ASPEC_ERR_INVALID, "dp_size and max_seq_length must be positive");
  if (max_selected >= 0 && max_selected < dp_size)
    return set_error(ASPEC_ERR_INVALID, "max_selected must be at least dp_size");
  if (count < 0) return set_error(ASPEC_ERR_INVALID, "pack_work_aware_rows: count < 0");
  if (!row_offsets || !row_tokens_out || (count > 0 && (!lengths || !useful_work || !row_samples)))
    return set_error(ASPEC_ERR_INVALID, "pack_work_aware_rows: null pointer");
  for (int64_t i = 0; i < count; ++i) {
    if (lengths[i] <= 0 || lengths[i] > max_seq_length)
      return set_error(ASPEC_ERR_INVALID,
                       "Packing received work that can never fit a row: %lld:%lld; max_seq_length=%lld",
                       static_cast<long long>(i), static_cast<long long>(lengths[i]),
                       static_cast<long long>(max_seq_length));
    if (lengths[i] >= kExactDouble || useful_work[i] >= kExactDouble || useful_work[i] <= -kExactDouble)
      return set_error(ASPEC_ERR_INVALID, "pack_work_aware_rows: sample %lld exceeds 2^53", static_cast<long long>(i));
  }
  std::fill(row_offsets, row_offsets + dp_size + 1, int64_t{0});
  std::fill(row_tokens_out, row_tokens_out + dp_size, int64_t{0});
  if (count < dp_size) return ASPEC_OK;  // not enough work for one row per rank: nothing packed

  // Candidate order: density, work, length (descending), index (ascending).
  std::vector<int64_t> order(static_cast<size_t>(count - dp_size));
  std::iota(order.begin(), order.end(), dp_size);
  std::vector<double> density(static_cast<size_t>(count));
  for (int64_t i = 0; i < count; ++i)
    density[i] = static_cast<double>(useful_work[i]) / static_cast<double>(lengths[i]);
  std::sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
    if (density[a] != density[b]) return density[a] > density[b];
    if (useful_work[a] != useful_work[b]) return useful_work[a] > useful_work[b];
    if (lengths[a] != lengths[b]) return lengths[a] > lengths[b];
    return a < b;
  });

  std::vector<int64_t> tokens(lengths, lengths + dp_size);
  std::vector<std::vector<int64_t>> rows(static_cast<size_t>(dp_size));
  for (int64_t r = 0; r < dp_size; ++r) rows[r].push_back(r);
  // Rows keyed by (tokens, -row): the fitting row with the least slack is the largest key whose
  // tokens stay within max_seq_length - length; among equal tokens the largest key is the lowest row.
  std::set<std::pair<int64_t, int64_t>> by_fill;
  for (int64_t r = 0; r < dp_size; ++r) by_fill.emplace(tokens[r], -r);
  int64_t selected = dp_size;
  for (const int64_t i : order) {
    if (max_selected >= 0 && selected >= max_selected) break;
    const int64_t limit = max_seq_length - lengths[i];
    auto it = by_fill.upper_bound({limit, INT64_MAX});
    if (it == by_fill.begin()) continue;  // no row has room
    --it;
    const int64_t r = -it->second;
    by_fill.erase(it);
    tokens[r] += lengths[i];
    by_fill.emplace(tokens[r], -r);
    rows[r].push_back(i);
    ++selected;
  }

  std::vector<int64_t> rank(static_cast<size_t>(dp_size));
  std::iota(rank.begin(), rank.end(), 0);
  std::sort(rank.begin(), rank.end(), [&](int64_t a, int64_t b) {
    return tokens[a] != tokens[b] ? tokens[a] > tokens[b] : a < b;
  });
  int64_t at = 0;
  for (int64_t k = 0; k < dp_size; ++k) {
    const auto& row = rows[rank[k]];
    row_offsets[k] = at;
    std::copy(row.begin(), row.end(), row_samples + at);
    at += static_cast<int64_t>(row.size());
    row_tokens_out[k] = tokens[rank[k]];
  }
  row_offsets[dp_size] = at;
  return ASPEC_OK;
}
