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

extern "C" const char *lm_version(void) { return "localmoe35ba3b-amd 0.1 gfx950"; }

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
