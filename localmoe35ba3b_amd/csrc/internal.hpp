// Host-side launch helpers shared between translation units of the library.
#pragma once
#include "common.hpp"

namespace lm {

int router_logits(const uint16_t *x, const uint16_t *w, const float *bias, float *logits,
                  int64_t T, int64_t E, int64_t H, hipStream_t st);
int router_topk(const float *logits, int64_t T, int64_t E, int64_t K, int64_t *ids,
                uint16_t *weights, hipStream_t st);
// shared_rows > 0 appends cdiv(shared_rows, bm) tiles (E, R + j*bm, R + shared_rows)
// after the max_tiles plan rows and pos[R + t] = t for the always-on shared expert.
int route_plan(const int64_t *ids, int64_t T, int64_t K, int64_t E, int64_t bm, int64_t *pos,
               int64_t *table, int64_t max_tiles, int64_t *ordered, int64_t *slots,
               int64_t shared_rows, hipStream_t st);
int routed_gemm(const void *x, const int8_t *q, const float *s, const int64_t *pos,
                const int64_t *table, int64_t n_tiles, int64_t bm, void *y, int64_t n, int64_t k,
                bool gather, bool swiglu, int64_t q_es, int64_t s_es, int64_t ldx,
                hipStream_t st);

}  // namespace lm
