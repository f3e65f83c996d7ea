// Host-side launch model of the decode split (no device code): the modelled finish time of a
// v2 launch at each candidate partition size, and the v2 work list. Python's choose_split and
// work_list (ayaka_amd/hip/attention.py) call these once per planned step or graph update, so
// their cost is host time on the engine thread; the pure-Python statement of the same model is
// kept beside the tests, which check the two agree.

#include <algorithm>
#include <climits>
#include <cstdint>
#include <functional>
#include <queue>
#include <vector>

#include "ayaka_hip.h"


namespace {

// One candidate partition size over the rows: its work items and the data to schedule them.
struct Candidate {
  uint32_t size = 0;
  int64_t full = 0;           // full partitions
  std::vector<uint32_t> rest; // the rows' partial last partitions, longest first
  int64_t items() const { return full + (int64_t)rest.size(); }
};

struct Model {
  int groups, xcds, per_xcd;
  int64_t cost;
  std::vector<uint32_t> lengths;  // rows with context, as 32-bit counts
  std::vector<uint32_t> counts;   // counting-sort buckets
  std::vector<uint32_t> sorted;
  std::vector<int64_t> loads;

  void split(Candidate& c, uint32_t size) {
    c.size = size;
    c.full = 0;
    c.rest.clear();
    // n / size through a double reciprocal, corrected by one step (n < 2^31: the estimate is
    // off by at most one); an integer division per row costs several times more here
    const double inv = 1.0 / size;
    for (uint32_t n : lengths) {
      int64_t q = (int64_t)((double)n * inv);
      int64_t r = (int64_t)n - q * size;
      if (r < 0) {
        --q;
        r += size;
      } else if (r >= (int64_t)size) {
        ++q;
        r -= size;
      }
      c.full += q;
      if (r) c.rest.push_back((uint32_t)r);
    }
    // longest first: a counting sort when the value range is small against the count
    if (size <= 8 * c.rest.size() + 64) {
      counts.assign(size, 0);
      for (uint32_t r : c.rest) ++counts[r];
      sorted.clear();
      for (uint32_t v = size; v-- > 1;)
        for (uint32_t k = counts[v]; k; --k) sorted.push_back(v);
      c.rest.swap(sorted);
    } else {
      std::sort(c.rest.begin(), c.rest.end(), std::greater<uint32_t>());
    }
  }

  // Items are dealt to XCD i mod xcds in order: first the full partitions (all alike, so an
  // XCD's units share them evenly: q or q + 1 each), then the partial ones, each repeated
  // `groups` times in a row; partial item k has index full * groups + k. With `exact` false,
  // a lower bound of the finish time instead (per XCD: its busiest unit before the partial
  // items, its least busy one plus its longest partial item, and its mean load).
  int64_t finish(const Candidate& c, bool exact) {
    const int64_t unit = (int64_t)c.size + cost;
    const int64_t full_items = c.full * groups;
    const int64_t n_rest = (int64_t)c.rest.size() * groups;
    if (full_items + n_rest == 0) return 0;
    int64_t finish = 0;
    for (int x = 0; x < xcds; ++x) {
      const int64_t mine = full_items > x ? (full_items - x + xcds - 1) / xcds : 0;
      const int64_t q = mine / per_xcd, r = mine % per_xcd;
      const int64_t first = ((x - full_items) % xcds + xcds) % xcds;  // its first partial item
      const int64_t top = (q + (r ? 1 : 0)) * unit;
      if (first >= n_rest) {
        finish = std::max(finish, top);
        continue;
      }
      if (!exact) {
        int64_t total = mine * unit;
        for (int64_t k = first; k < n_rest; k += xcds) total += (int64_t)c.rest[k / groups] + cost;
        const int64_t longest = q * unit + (int64_t)c.rest[first / groups] + cost;
        finish = std::max({finish, top, longest, (total + per_xcd - 1) / per_xcd});
        continue;
      }
      for (int u = 0; u < per_xcd; ++u) loads[u] = (q + (u < r ? 1 : 0)) * unit;
      std::make_heap(loads.begin(), loads.end(), std::greater<int64_t>());
      for (int64_t k = first; k < n_rest; k += xcds) {
        std::pop_heap(loads.begin(), loads.end(), std::greater<int64_t>());
        loads.back() += (int64_t)c.rest[k / groups] + cost;
        std::push_heap(loads.begin(), loads.end(), std::greater<int64_t>());
      }
      finish = std::max(finish, *std::max_element(loads.begin(), loads.end()));
    }
    return finish;
  }
};

bool make_model(Model& m, const int64_t* lengths, int32_t n_lengths, int32_t groups, int32_t cost,
                int32_t compute_units, int32_t xcds) {
  if (n_lengths < 0 || groups < 1 || cost < 0 || xcds < 1 || compute_units < xcds || compute_units % xcds != 0 ||
      (n_lengths && !lengths))
    return false;
  m.groups = groups;
  m.xcds = xcds;
  m.per_xcd = compute_units / xcds;
  m.cost = cost;
  m.loads.resize(m.per_xcd);
  m.lengths.clear();
  m.lengths.reserve(n_lengths);
  for (int32_t i = 0; i < n_lengths; ++i)
    if (lengths[i] > 0) m.lengths.push_back((uint32_t)std::min<int64_t>(lengths[i], INT32_MAX));
  return true;
}

}  // namespace

extern "C" {

int ayk_split_model(const int64_t* lengths, int32_t n_lengths, const int32_t* sizes, int32_t n_sizes,
                    int32_t groups, int32_t cost, int32_t compute_units, int32_t xcds, int64_t* makespans,
                    int64_t* item_counts) {
  Model m;
  if (n_sizes < 0 || (n_sizes && (!sizes || !makespans)) ||
      !make_model(m, lengths, n_lengths, groups, cost, compute_units, xcds))
    return AYK_ERR_ARGUMENT;
  Candidate c;
  for (int32_t i = 0; i < n_sizes; ++i) {
    if (sizes[i] <= 0) return AYK_ERR_ARGUMENT;
    m.split(c, (uint32_t)sizes[i]);
    if (item_counts) item_counts[i] = c.items();
    makespans[i] = m.finish(c, true);
  }
  return AYK_OK;
}

int ayk_best_split(const int64_t* lengths, int32_t n_lengths, const int32_t* sizes, int32_t n_sizes, int32_t groups,
                   int32_t cost, int32_t compute_units, int32_t xcds, int64_t max_items, int64_t round_items,
                   int32_t* best) {
  Model m;
  if (n_sizes < 1 || !sizes || !best || !make_model(m, lengths, n_lengths, groups, cost, compute_units, xcds))
    return AYK_ERR_ARGUMENT;
  std::vector<Candidate> cands(n_sizes);
  std::vector<int32_t> eligible;
  for (int32_t i = 0; i < n_sizes; ++i) {
    if (sizes[i] <= 0) return AYK_ERR_ARGUMENT;
    m.split(cands[i], (uint32_t)sizes[i]);
    if (max_items <= 0 || cands[i].items() <= max_items) eligible.push_back(i);
  }
  *best = -1;
  if (eligible.empty()) return AYK_OK;
  // candidates past the round limit are left out, except the last eligible one
  std::vector<std::pair<int64_t, int32_t>> order;  // (lower bound, candidate)
  for (size_t e = 0; e < eligible.size(); ++e) {
    const int32_t i = eligible[e];
    if (e + 1 < eligible.size() && cands[i].items() * groups > round_items) continue;
    order.emplace_back(m.finish(cands[i], false), i);
  }
  // exact finish times in order of their bounds; a candidate whose bound exceeds the best
  // found (or equals it, for a later candidate: ties go to the first) cannot win
  std::sort(order.begin(), order.end());
  int64_t best_time = INT64_MAX;
  for (const auto& [bound, i] : order) {
    if (bound > best_time || (bound == best_time && i > *best)) continue;
    const int64_t t = m.finish(cands[i], true);
    if (t < best_time || (t == best_time && i < *best)) {
      best_time = t;
      *best = i;
    }
  }
  return AYK_OK;
}

int64_t ayk_work_list(const int64_t* lengths, int32_t n_lengths, int32_t partition_size, int32_t* out) {
  if (n_lengths < 0 || partition_size <= 0 || (n_lengths && !lengths)) return -1;
  int64_t n = 0;
  for (int32_t i = 0; i < n_lengths; ++i)
    n += lengths[i] > 0 ? (lengths[i] + partition_size - 1) / partition_size : 1;
  if (!out) return n;
  int32_t* w = out;
  // full partitions, by row then partition
  for (int32_t i = 0; i < n_lengths; ++i)
    for (int64_t p = 0; p < (lengths[i] > 0 ? lengths[i] / partition_size : 0); ++p) {
      *w++ = i;
      *w++ = (int32_t)p;
    }
  // the partial last partitions, longest first (ties by row)
  std::vector<std::pair<int64_t, int32_t>> rest;
  for (int32_t i = 0; i < n_lengths; ++i)
    if (lengths[i] > 0 && lengths[i] % partition_size) rest.emplace_back(-(lengths[i] % partition_size), i);
  std::sort(rest.begin(), rest.end());
  for (const auto& [neg, i] : rest) {
    *w++ = i;
    *w++ = (int32_t)(lengths[i] / partition_size);
  }
  // partition 0 of every row without context (it writes the row's zeros)
  for (int32_t i = 0; i < n_lengths; ++i)
    if (lengths[i] <= 0) {
      *w++ = i;
      *w++ = 0;
    }
  return n;
}

// The multi-row launch model's schedule: durations sorted longest first, each started in the
// slot that frees up first (a min-heap of slot loads); equal durations fill whole rounds.
int ayk_dispatch_makespan(const double* durations, int64_t n, int32_t slots, double* makespan) {
  if (n < 0 || slots < 1 || !makespan || (n > 0 && !durations)) return AYK_ERR_ARGUMENT;
  std::vector<double> d(durations, durations + n);
  std::sort(d.begin(), d.end(), std::greater<double>());
  if (n <= slots) {
    *makespan = n ? d[0] : 0.0;
    return AYK_OK;
  }
  if (d[0] == d[n - 1]) {
    *makespan = (double)((n + slots - 1) / slots) * d[0];
    return AYK_OK;
  }
  std::priority_queue<double, std::vector<double>, std::greater<double>> loads(d.begin(), d.begin() + slots);
  for (int64_t i = slots; i < n; ++i) {
    const double least = loads.top();
    loads.pop();
    loads.push(least + d[i]);
  }
  double last = 0.0;
  while (!loads.empty()) {
    last = std::max(last, loads.top());
    loads.pop();
  }
  *makespan = last;
  return AYK_OK;
}

}  // extern "C"
