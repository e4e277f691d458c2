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
// One routed grouped W8A16 GEMM (gate_up with gather + optional SwiGLU
// epilogue, or down over contiguous rows) over a (expert, start, stop) tile
// table.  Table experts are clamped into [0, experts), starts and stops into
// [0, y_rows], gathered row indices into [0, x_rows).
struct RoutedGemm {
  const void *x;
  int64_t ldx, x_rows;
  const int8_t *q;
  const float *s;
  int64_t q_es, s_es, experts;
  const int64_t *pos;
  const int64_t *table;
  int64_t n_tiles, bm;
  void *y;
  int64_t y_rows, n, k;
  bool gather, swiglu;
  int dtype;
  const int8_t *q_tiles = nullptr;  // q in the lm_w8_tile_rows layout, or null
  // Non-null: x holds fp16 rows fp16(row r * 2^x_exp[r]) (exact) and q_tiles
  // is in the LM_TILES_F16 format; the output is bf16.
  const int *x_exp = nullptr;
  // Gathered GEMMs on q_tiles: the token of row r of table tile i at
  // ptile[i * bm + r] (any value for rows past the tile's end), read with the
  // table row instead of through pos; required with q_tiles and gather.
  const int *ptile = nullptr;
};
int routed_gemm(const RoutedGemm &r, hipStream_t st);

}  // namespace lm
