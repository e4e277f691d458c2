// Index guards of the MoE kernels, shared by the device code and the
// host-compiled bounds test (tests/native/test_bounds.cpp builds this header
// with g++ alone).  Every expert id, route position and tile-table entry that
// a kernel turns into an address passes through one of these functions, so a
// malformed value (an unwritten workspace word, a garbage table row, an id
// out of range) can give a wrong result but never an address outside the
// bank, the activations or the workspace.
#pragma once

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define LM_HD __host__ __device__ __forceinline__
#else
#define LM_HD inline
#endif

namespace lm {

// i clamped into [0, n); n >= 1.
LM_HD int64_t clamp_index(int64_t i, int64_t n) { return i < 0 ? 0 : (i >= n ? n - 1 : i); }
LM_HD int clamp_index32(int i, int n) { return i < 0 ? 0 : (i >= n ? n - 1 : i); }

LM_HD uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
LM_HD float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// Order-preserving selection keys: a larger key is a larger logit, then a
// smaller expert index.  -0 is folded onto +0.  key64 holds any fp32 value
// (NaN and infinities included: they order by their bit patterns); key32
// holds a value whose low 16 bits are zero (a bf16 value) in half the bits.
// The index field is 16 bits wide, so an index decoded from any key lies in
// [0, 65535]; callers clamp it to the expert count.
LM_HD unsigned long long key64_make(float v, int idx) {
  uint32_t b = f32_bits(v + 0.0f);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (uint32_t)(0xFFFFu - ((uint32_t)idx & 0xFFFFu));
}
LM_HD int key64_index(unsigned long long k) { return (int)(0xFFFFu - (uint32_t)(k & 0xFFFFu)); }
LM_HD float key64_value(unsigned long long k) {
  const uint32_t b = (uint32_t)(k >> 32);
  return bits_f32((b & 0x80000000u) ? (b & 0x7FFFFFFFu) : ~b);
}
LM_HD uint32_t key32_make(float v, int idx) {
  uint32_t b = f32_bits(v + 0.0f) >> 16;
  b = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return (b << 16) | (0xFFFFu - ((uint32_t)idx & 0xFFFFu));
}
LM_HD int key32_index(uint32_t k) { return (int)(0xFFFFu - (k & 0xFFFFu)); }
LM_HD float key32_value(uint32_t k) {
  const uint32_t b = k >> 16;
  return bits_f32(((b & 0x8000u) ? (b & 0x7FFFu) : (~b & 0xFFFFu)) << 16);
}

// Combine slot of selected route t among the K selected expert ids: its rank
// in ascending id order, ties broken by route index.  For any ids (distinct,
// duplicated or out of range) the K slots are a permutation of 0..K-1, so
// every slot of the decode expert list is written on every call.
LM_HD int combine_slot(const int64_t *ids, int K, int t) {
  const int64_t id = ids[t];
  int rank = 0;
  for (int j = 0; j < K; ++j) rank += (ids[j] < id || (ids[j] == id && j < t)) ? 1 : 0;
  return rank;
}

// Expert of decode-down row r: rows [cols * s, cols * (s + 1)) belong to
// selected slot s < K (expert ex[s], clamped into [0, experts)), rows past
// K * cols to the always-on shared expert `experts`.
LM_HD int decode_row_expert(const int *ex, int K, int cols, int experts, int r) {
  const int s = r / cols;
  int e = experts;
  for (int j = 0; j < K; ++j)
    if (s == j) e = clamp_index32(ex[j], experts);
  return e;
}

// One row of a route-plan tile table, (expert, start, stop), made safe to
// address with: the expert clamped into [0, experts), start into
// [0, row_limit], stop into [start, row_limit], and the tile's row count
// capped at tile_rows.  rows == 0 means "skip the tile".
struct TileBounds {
  int64_t expert;
  int64_t start;
  int rows;
};
LM_HD TileBounds tile_bounds(int64_t e, int64_t start, int64_t stop, int64_t experts,
                             int64_t row_limit, int tile_rows) {
  TileBounds t;
  t.expert = clamp_index(e, experts);
  t.start = start < 0 ? 0 : (start > row_limit ? row_limit : start);
  const int64_t sp = stop < t.start ? t.start : (stop > row_limit ? row_limit : stop);
  const int64_t n = sp - t.start;
  t.rows = (int)(n < tile_rows ? n : tile_rows);
  return t;
}

}  // namespace lm
