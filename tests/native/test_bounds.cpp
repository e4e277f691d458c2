// Host-compiled check of the index guards the MoE kernels use before they
// form an address (localmoe35ba3b_amd/csrc/bounds.hpp).  Every guard is fed
// garbage - random bit patterns, NaN payloads, infinities, signed zeros,
// denormals, duplicated and out-of-range ids, unwritten workspace words -
// and every address it leads to is checked against the buffer it indexes:
//   decode top-k   logits -> selection keys -> expert ids -> combine slots
//   decode down    slot expert -> down-bank row and scale addresses
//   decode gate_up slot expert -> gate_up-bank row addresses
//   grouped GEMM   tile-table row -> expert, rows, gathered activation rows
//   combines       route and slot indices
// Exit status 0 and a summary line on success; the first violation aborts.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <random>
#include <vector>

#include "bounds.hpp"

using namespace lm;

static long checks = 0;
#define REQUIRE(cond)                                                        \
  do {                                                                       \
    ++checks;                                                                \
    if (!(cond)) {                                                           \
      std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      std::abort();                                                          \
    }                                                                        \
  } while (0)

constexpr int kE = 256, kTopK = 8, kH = 2048, kI = 512, kDnCols = 8, kGuPairs = 8;
// bank geometry of one layer (elements): E + 1 experts, index E = shared
constexpr int64_t kGuQes = 2LL * kI * kH, kGuSes = 2LL * kI * (kH / 128);
constexpr int64_t kDnQes = (int64_t)kH * kI, kDnSes = (int64_t)kH * (kI / 128);

static float garbage_float(std::mt19937_64 &rng, int kind) {
  switch (kind) {
    case 0: return bits_f32((uint32_t)rng());                       // any bit pattern
    case 1: return bits_f32(0x7F800001u | ((uint32_t)rng() & 0x7FFFFFu));  // NaN payloads
    case 2: return (rng() & 1) ? INFINITY : -INFINITY;
    case 3: return (rng() & 1) ? 0.0f : -0.0f;
    case 4: return bits_f32((uint32_t)rng() & 0x807FFFFFu);         // denormals
    case 5: return bits_f32(((uint32_t)rng()) & 0xFFFF0000u);       // bf16 values (key32)
    default: return std::normal_distribution<float>(0.f, 1.f)(rng);
  }
}

// The decode top-k's selection, restated on the host over the same keys:
// the 8 largest keys (key32 when every logit is a bf16 value, as on the
// device), their decoded expert ids and combine slots.
static void check_topk(const std::vector<float> &lg) {
  bool bf16_only = true;
  for (float v : lg) bf16_only = bf16_only && (f32_bits(v) & 0xFFFFu) == 0;
  std::vector<int64_t> ids(kTopK);
  if (bf16_only) {
    std::vector<uint32_t> keys(kE);
    for (int e = 0; e < kE; ++e) keys[e] = key32_make(lg[e], e);
    std::sort(keys.begin(), keys.end(), std::greater<uint32_t>());
    REQUIRE(std::adjacent_find(keys.begin(), keys.end()) == keys.end());  // distinct keys
    for (int i = 0; i < kTopK; ++i) ids[i] = key32_index(keys[i]);
  } else {
    std::vector<unsigned long long> keys(kE);
    for (int e = 0; e < kE; ++e) keys[e] = key64_make(lg[e], e);
    std::sort(keys.begin(), keys.end(), std::greater<unsigned long long>());
    REQUIRE(std::adjacent_find(keys.begin(), keys.end()) == keys.end());
    for (int i = 0; i < kTopK; ++i) ids[i] = key64_index(keys[i]);
  }
  int sel[kTopK];
  bool written[kTopK] = {};
  for (int t = 0; t < kTopK; ++t) {
    REQUIRE(ids[t] >= 0 && ids[t] < kE);
    const int slot = combine_slot(ids.data(), kTopK, t);
    REQUIRE(slot >= 0 && slot < kTopK && !written[slot]);
    written[slot] = true;
    sel[slot] = (int)clamp_index(ids[t], kE);
  }
  for (int s = 1; s < kTopK; ++s) REQUIRE(sel[s - 1] < sel[s]);  // ascending, distinct
}

// Decode gate_up and down address ranges for an arbitrary expert list (the
// workspace words the down kernel reads, possibly never written).
static void check_decode_addresses(const int *ex) {
  const int64_t gu_bank = (kE + 1) * kGuQes, dn_bank = (kE + 1) * kDnQes;
  const int64_t gu_sbank = (kE + 1) * kGuSes, dn_sbank = (kE + 1) * kDnSes;
  for (int slot = 0; slot <= kTopK; ++slot) {
    const int e = slot == kTopK ? kE : clamp_index32(ex[slot], kE);
    REQUIRE(e >= 0 && e <= kE);
    for (int n0 = 0; n0 < kI; n0 += kGuPairs) {  // gate rows n0.., up rows kI + n0..
      const int64_t last_row = kI + n0 + kGuPairs - 1;
      REQUIRE(e * kGuQes + last_row * kH + kH - 1 < gu_bank);
      REQUIRE(e * kGuSes + last_row * (kH / 128) + kH / 128 - 1 < gu_sbank);
    }
  }
  constexpr int R = (kTopK + 1) * kDnCols;
  for (int c0 = 0; c0 < kH; c0 += kDnCols) {
    for (int r = 0; r < R; ++r) {
      const int e = decode_row_expert(ex, kTopK, kDnCols, kE, r);
      REQUIRE(e >= 0 && e <= kE);
      REQUIRE(r < kTopK * kDnCols || e == kE);
      const int64_t row = c0 + r % kDnCols;
      REQUIRE(e * kDnQes + row * kI >= 0 && e * kDnQes + row * kI + kI - 1 < dn_bank);
      REQUIRE(e * kDnSes + row * (kI / 128) + kI / 128 - 1 < dn_sbank);
    }
  }
}

// Grouped GEMM tile rows: every row a tile touches lies inside y, every
// gathered activation row inside x, the expert inside the bank.
static void check_tile(int64_t e, int64_t start, int64_t stop, int64_t experts, int64_t y_rows,
                       int tile_rows, const std::vector<int64_t> &pos, int64_t x_rows) {
  const TileBounds tb = tile_bounds(e, start, stop, experts, y_rows, tile_rows);
  REQUIRE(tb.expert >= 0 && tb.expert < experts);
  REQUIRE(tb.rows >= 0 && tb.rows <= tile_rows);
  REQUIRE(tb.start >= 0 && tb.start <= y_rows);
  REQUIRE(tb.start + tb.rows <= y_rows);
  for (int r = 0; r < tb.rows; ++r) {
    const int64_t p = tb.start + r;
    REQUIRE(p >= 0 && p < (int64_t)pos.size());
    const int64_t xr = clamp_index(pos[p], x_rows);
    REQUIRE(xr >= 0 && xr < x_rows);
  }
  // the kernels' unconditional loads re-read the tile's last row past `rows`
  if (tb.rows > 0) REQUIRE(tb.start + tb.rows - 1 < y_rows);
}

int main() {
  std::mt19937_64 rng(20261202);
  // 1. key codecs: value round trip and index range over garbage
  for (int it = 0; it < 200000; ++it) {
    const float v = garbage_float(rng, it % 7);
    const int idx = (int)(rng() % 70000) - 1000;  // also out of [0, 65536)
    const int i64 = key64_index(key64_make(v, idx));
    const int i32 = key32_index(key32_make(v, idx));
    REQUIRE(i64 >= 0 && i64 <= 0xFFFF && i32 >= 0 && i32 <= 0xFFFF);
    if (idx >= 0 && idx <= 0xFFFF) REQUIRE(i64 == idx && i32 == idx);
    if (!std::isnan(v)) {
      REQUIRE(key64_value(key64_make(v, idx)) == v);
      REQUIRE((f32_bits(key64_value(key64_make(v, 0))) == f32_bits(v + 0.0f)));
    }
  }
  // 2. decode top-k over garbage logit vectors
  for (int it = 0; it < 4000; ++it) {
    std::vector<float> lg(kE);
    const int mode = it % 9;
    for (int e = 0; e < kE; ++e)
      lg[e] = mode < 7 ? garbage_float(rng, mode) : garbage_float(rng, (int)(rng() % 7));
    if (it % 13 == 0) std::fill(lg.begin(), lg.end(), lg[0]);  // all ties
    check_topk(lg);
  }
  // 3. combine slots and decode addresses for arbitrary id lists
  const int64_t specials[] = {0, 1, 255, 256, 257, -1, -256, 65535, 65536,
                              std::numeric_limits<int32_t>::max(),
                              std::numeric_limits<int32_t>::min(),
                              std::numeric_limits<int64_t>::max(),
                              std::numeric_limits<int64_t>::min()};
  for (int it = 0; it < 20000; ++it) {
    int64_t ids[kTopK];
    int ex[kTopK];
    for (int t = 0; t < kTopK; ++t) {
      const int kind = (int)(rng() % 4);
      ids[t] = kind == 0 ? (int64_t)rng() : kind == 1 ? specials[rng() % 13]
               : kind == 2 ? (int64_t)(rng() % 4) : (int64_t)(rng() % kE);
      ex[t] = (int)(uint32_t)rng();  // an unwritten workspace word
    }
    bool written[kTopK] = {};
    for (int t = 0; t < kTopK; ++t) {
      const int slot = combine_slot(ids, kTopK, t);
      REQUIRE(slot >= 0 && slot < kTopK && !written[slot]);
      written[slot] = true;
    }
    if (it % 50 == 0) check_decode_addresses(ex);
    for (int t = 0; t < kTopK; ++t) ex[t] = (int)clamp_index(ids[t], 1LL << 40);
    if (it % 50 == 1) check_decode_addresses(ex);
  }
  // 4. grouped GEMM tile rows: the fused prefill's geometry (E + 1 experts,
  // R + T rows, T activation rows) and the routed entry points'
  for (int it = 0; it < 20000; ++it) {
    const int64_t T = 1 + (int64_t)(rng() % 3000);
    const bool fused = it % 2 == 0;
    const int64_t experts = fused ? kE + 1 : 1 + (int64_t)(rng() % 300);
    const int64_t y_rows = fused ? T * (kTopK + 1) : (int64_t)(rng() % 5000);
    const int64_t x_rows = fused ? T : 1 + (int64_t)(rng() % 5000);
    const int tile_rows = 1 + (int)(rng() % 128);
    std::vector<int64_t> pos((size_t)y_rows);
    for (auto &p : pos) p = (rng() & 1) ? (int64_t)rng() : specials[rng() % 13];
    for (int j = 0; j < 8; ++j) {
      const int64_t e = (rng() & 1) ? (int64_t)rng() : specials[rng() % 13];
      const int64_t s = (rng() & 1) ? (int64_t)rng() : (int64_t)(rng() % (y_rows + 200)) - 100;
      const int64_t p = (rng() & 1) ? (int64_t)rng() : s + (int64_t)(rng() % 300) - 50;
      check_tile(e, s, p, experts, y_rows, tile_rows, pos, x_rows);
    }
  }
  // 5. combine indices: routes into [0, tokens * K), slots into [0, K)
  for (int it = 0; it < 100000; ++it) {
    const int64_t tokens = 1 + (int64_t)(rng() % 65535);
    const int64_t v = (rng() & 1) ? (int64_t)rng() : specials[rng() % 13];
    const int64_t route = clamp_index(v, tokens * kTopK);
    const int64_t slot = clamp_index(v, kTopK);
    REQUIRE(route >= 0 && route < tokens * kTopK && slot >= 0 && slot < kTopK);
    const int r32 = clamp_index32((int)(uint32_t)rng(), (int)(tokens * kTopK));
    REQUIRE(r32 >= 0 && r32 < tokens * kTopK);
  }
  std::printf("bounds ok: %ld checks\n", checks);
  return 0;
}
