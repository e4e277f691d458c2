// Host-side plumbing of the C ABI: per-thread error messages, launch checks,
// and the host route planner that mirrors routing.plan_routes.
#include <vector>

#include "common.hpp"

namespace lm {

static thread_local std::string g_last_error;

int set_error(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(LM_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return LM_OK;
}

}  // namespace lm

extern "C" const char *lm_version(void) { return "localmoe35ba3b-amd 0.3 gfx950"; }

extern "C" const char *lm_last_error(void) { return lm::g_last_error.c_str(); }

// Stable counting sort of the flat routes by expert id (routing.py:5-20).
// positions is [2, tokens*top_k]; the segment arrays need `experts` entries.
extern "C" int lm_plan_routes_host(const int64_t *ids, int64_t tokens, int64_t top_k,
                                   int64_t experts, int64_t *positions, int64_t *seg_expert,
                                   int64_t *seg_start, int64_t *seg_stop, int64_t *n_segments) {
  const int64_t routes = tokens * top_k;
  LM_REQUIRE(tokens > 0 && top_k > 0 && ids != nullptr, LM_EINVAL,
             "Expected nonempty CPU [tokens,top_k] IDs");
  LM_REQUIRE(experts > 0, LM_EINVAL, "Out-of-range expert ID");
  for (int64_t i = 0; i < routes; ++i)
    LM_REQUIRE(ids[i] >= 0 && ids[i] < experts, LM_EINVAL, "Out-of-range expert ID");
  std::vector<int64_t> offset(experts + 1, 0);
  for (int64_t i = 0; i < routes; ++i) offset[ids[i] + 1]++;
  int64_t n = 0;
  for (int64_t e = 0; e < experts; ++e) {
    const int64_t count = offset[e + 1];
    offset[e + 1] += offset[e];
    if (count) {
      seg_expert[n] = e;
      seg_start[n] = offset[e];
      seg_stop[n] = offset[e + 1];
      ++n;
    }
  }
  *n_segments = n;
  for (int64_t i = 0; i < routes; ++i) {
    const int64_t p = offset[ids[i]]++;
    positions[p] = i / top_k;
    positions[routes + p] = i % top_k;
  }
  return LM_OK;
}

// Host twin of lm_route_plan for callers that already hold the routing ids
// on the CPU (the reference's host-planned prefill path, prefill.py:52-85):
// one stable counting sort gives every route its row in expert order; the
// tile table lists only the bm-row tiles of non-empty experts (the
// reference's host path launches exactly those); each token's routes are
// ordered by (expert id, slot) with an insertion sort of its top_k ids.
extern "C" int lm_route_plan_host(const int64_t *ids, int64_t tokens, int64_t top_k,
                                  int64_t experts, int64_t bm, int64_t *pos, int64_t *table,
                                  int64_t max_tiles, int64_t *ordered, int64_t *slots,
                                  int64_t *n_tiles, int64_t *n_active) {
  LM_REQUIRE(tokens > 0 && top_k > 0 && top_k <= 64 && ids != nullptr, LM_EINVAL,
             "Expected nonempty CPU [tokens,top_k] IDs");
  LM_REQUIRE(experts > 0 && bm >= 1, LM_EINVAL, "invalid expert count or tile height");
  LM_REQUIRE(pos && table && ordered && slots && n_tiles && n_active, LM_EINVAL, "null pointer");
  const int64_t routes = tokens * top_k;
  LM_REQUIRE(max_tiles >= (routes + bm - 1) / bm + experts, LM_EINVAL,
             "max_tiles must be at least cdiv(routes, bm) + experts");
  for (int64_t i = 0; i < routes; ++i)
    LM_REQUIRE(ids[i] >= 0 && ids[i] < experts, LM_EINVAL, "Out-of-range expert ID");
  std::vector<int64_t> first(experts + 1, 0);  // first row of each expert
  for (int64_t i = 0; i < routes; ++i) first[ids[i] + 1]++;
  int64_t active = 0, tiles = 0;
  for (int64_t e = 0; e < experts; ++e) {
    const int64_t count = first[e + 1];
    first[e + 1] += first[e];
    if (!count) continue;
    ++active;
    for (int64_t start = first[e]; start < first[e + 1]; start += bm, ++tiles) {
      table[tiles * 3] = e;
      table[tiles * 3 + 1] = start;
      table[tiles * 3 + 2] = first[e + 1];
    }
  }
  std::vector<int64_t> row_of(routes);
  std::vector<int64_t> next(first.begin(), first.end() - 1);
  for (int64_t i = 0; i < routes; ++i) {
    const int64_t p = next[ids[i]]++;
    pos[p] = i / top_k;
    row_of[i] = p;
  }
  for (int64_t t = 0; t < tokens; ++t) {
    const int64_t *tid = ids + t * top_k;
    int64_t *ts = slots + t * top_k;
    for (int64_t j = 0; j < top_k; ++j) {  // stable: equal ids keep slot order
      int64_t i = j;
      while (i > 0 && tid[ts[i - 1]] > tid[j]) {
        ts[i] = ts[i - 1];
        --i;
      }
      ts[i] = j;
    }
    for (int64_t j = 0; j < top_k; ++j) ordered[t * top_k + j] = row_of[t * top_k + ts[j]];
  }
  *n_tiles = tiles;
  *n_active = active;
  return LM_OK;
}
