// Streaming int8-weight GEMV core for decode (M <= 8 activation rows).
//
// A block streams R weight rows of K int8 each.  The (row, 128-group) pairs
// are flattened to f = r * G + g (G = K / 128); one wave instruction loads
// 8 consecutive pairs = 1 KB with one 16-byte load per lane, lane octet
// j = lane / 8 covering pair 8 i + j.  Each wave owns a contiguous run of
// instructions and issues a whole batch of loads before consuming any of
// them, so a block keeps LOADS * 4 KB of weights in flight.  Per-pair
// partial dot products are reduced across the octet with DPP and parked in
// LDS; the per-row epilogue then walks the groups in ascending order, which
// is what the W8A8 reference epilogue requires (w8a8.py:40).
#pragma once
#include "common.hpp"

namespace lm {

// Row index -> weight row.  `split` > 0 maps rows [0, split) to
// first + r and rows [split, 2 split) to second + (r - split): the gate / up
// halves of a fused gate_up matrix.
struct RowMap {
  int first;
  int second;
  int split;
  __device__ __forceinline__ int operator()(int r) const {
    return (split > 0 && r >= split) ? second + (r - split) : first + r;
  }
};

// Walks this wave's instructions in batches of LOADS.  `body(w, r, g, f, ok)`
// receives each lane's 16 bytes of row r, group g (flattened index f); ok is
// false for lanes past the end (their w is zero).  All lanes of the wave
// call body together, so body may use cross-lane DPP.  Weight rows are read
// once per call and not again before the rest of a decode step's weights
// (far more than the caches hold) have passed, so they are loaded
// non-temporally: the loads stream past the caches, which reads HBM faster.
template <int LOADS, typename RowPtr, typename Body>
__device__ __forceinline__ void stream_rows(int R, int G, RowPtr row_ptr, Body body) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int oct = lane >> 3;
  const int sub = lane & 7;
  const int total = R * G;
  const int ninstr = (total + 7) >> 3;
  const int ipw = (ninstr + nwaves - 1) / nwaves;
  const int ibeg = wave * ipw;
  const int iend = min(ibeg + ipw, ninstr);
  int f = ibeg * 8 + oct;
  int r = f / G;
  int g = f - r * G;
  for (int i = ibeg; i < iend; i += LOADS) {
    u32x4 w[LOADS];
    int rs[LOADS], gs[LOADS], fs[LOADS];
    bool ok[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      ok[u] = (i + u < iend) && (f < total);
      rs[u] = r;
      gs[u] = g;
      fs[u] = f;
      if (ok[u]) {
        w[u] = ldg16_nt(row_ptr(r) + g * 128 + sub * 16);
      } else {
        w[u] = u32x4{0u, 0u, 0u, 0u};
      }
      f += 8;
      g += 8;
      while (g >= G) {
        g -= G;
        ++r;
      }
    }
#pragma unroll
    for (int u = 0; u < LOADS; ++u) body(w[u], rs[u], gs[u], fs[u], ok[u]);
  }
}

// One-batch form of stream_rows for kernels whose waves own at most LOADS
// instructions: issue() starts every load of the wave, consume() runs the
// body afterwards, so a prologue placed between the two overlaps the HBM
// latency.  Every lane issues exactly LOADS loads without branches: slots
// past the end read pair 0 again (a valid address) and are flagged !ok.
// All lanes of an octet share one (row, group) pair and hence one ok flag.
// Branch-free issue keeps the compiler's wait counts exact, so code that
// needs only older loads does not wait for these.  THREADS is the
// workgroup size the kernel is launched with (a constant, so the issue does
// not wait for the block-size kernel argument).
template <int LOADS, int THREADS = 256>
struct RowLoads {
  u32x4 w[LOADS];
  int r[LOADS], g[LOADS], f[LOADS];
  bool ok[LOADS];

  template <typename RowPtr>
  __device__ __forceinline__ void issue(int R, int G, RowPtr row_ptr) {
    static_assert(THREADS % 64 == 0, "whole waves");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    constexpr int nwaves = THREADS >> 6;
    const int sub = lane & 7;
    const int total = R * G;
    const int ninstr = (total + 7) >> 3;
    const int ipw = (ninstr + nwaves - 1) / nwaves;
    const int ibeg = wave * ipw;
    const int iend = min(ibeg + ipw, ninstr);
    int ff = ibeg * 8 + (lane >> 3);
    int rr = ff / G;
    int gg = ff - rr * G;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      ok[u] = (ibeg + u < iend) && (ff < total);
      r[u] = ok[u] ? rr : 0;
      g[u] = ok[u] ? gg : 0;
      f[u] = ok[u] ? ff : 0;
      w[u] = ldg16_nt(row_ptr(r[u]) + g[u] * 128 + sub * 16);
      ff += 8;
      gg += 8;
      while (gg >= G) {
        gg -= G;
        ++rr;
      }
    }
  }

  template <typename Body>
  __device__ __forceinline__ void consume(Body body) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) body(w[u], r[u], g[u], f[u], ok[u]);
  }
};

// Two-phase forms of the activation staging below, for kernels that issue
// their weight loads in between: load() requests the activations, store()
// writes them (quantized, for QuantStage) to LDS.  The memory counter
// completes in issue order, so the wait before store() covers only these
// older loads, not the weights.  Loads are branch-free (pieces or jobs past
// the end re-read the last one); only the stores are guarded.
// RowStage: `rows` rows of `row_bytes` bytes (a multiple of 16), at most N
// 16-byte pieces per thread (rows * row_bytes <= N * 16 * blockDim.x).
template <int N>
struct RowStage {
  u32x4 v[N];
  int n;
  __device__ __forceinline__ void load(const unsigned char *src, int64_t pitch, int rows,
                                       int row_bytes) {
    const int per_row = row_bytes >> 4;
    n = rows * per_row;
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int i = min((int)(threadIdx.x + u * blockDim.x), n - 1);
      const int m = i / per_row, c = i - (i / per_row) * per_row;
      v[u] = ldg16(src + m * pitch + c * 16);
    }
  }
  // Branch-free as well: pieces past the end rewrite the last piece with the
  // value it already holds (a store under a branch would make the compiler
  // wait for every load in flight, the weights included).
  __device__ __forceinline__ void store(unsigned char *dst) const {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int i = min((int)(threadIdx.x + u * blockDim.x), n - 1);
      *reinterpret_cast<u32x4 *>(dst + (int64_t)i * 16) = v[u];
    }
  }
};

// Absmax of a 128-group held as 4 values per lane by one half-wave: four DPP
// steps inside each 16-lane row, then v_permlane16_swap, which exchanges the
// two rows of each row pair (both results hold one row each, so their max is
// the pair's max whichever way round they come back).  All VALU: no LDS
// counter wait, so the groups of several jobs interleave.
__device__ __forceinline__ float halfwave_max(float a) {
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0xB1, 0xF, 0xF, false)));
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x4E, 0xF, 0xF, false)));
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x141, 0xF, 0xF, false)));
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x140, 0xF, 0xF, false)));
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Quantizes one 128-group (4 values per lane of a half-wave, w8a8.py:8-14)
// into xq[g * 128 + 4 l ..] and, from lane 0, its scale.  Callers pass the
// destination of a real job; surplus lanes redo the last job and store the
// same bytes to it again, so no store is under a branch.
template <typename T>
__device__ __forceinline__ void quantize_group(uint2 raw, int l, int8_t *xq_group,
                                               float *xs_slot) {
  const float inv127 = (float)(1.0 / 127.0);
  float v[4] = {T::to_f32(raw.x & 0xFFFFu), T::to_f32(raw.x >> 16), T::to_f32(raw.y & 0xFFFFu),
                T::to_f32(raw.y >> 16)};
  const float a =
      halfwave_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  const float sc = fmaxf(a, 1e-10f) * inv127;
  const float r = 1.0f / sc;
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    packed |= ((uint32_t)(uint8_t)(int8_t)(int)rintf(quant_div(v[i], sc, r))) << (8 * i);
  *reinterpret_cast<uint32_t *>(xq_group + l * 4) = packed;
  if (l == 0) *xs_slot = sc;
}

// QuantStage: a half-wave owns (row, group) jobs half, half + nhalf, ... (at
// most J of them: rows * (K / 128) <= J * blockDim.x / 32).
template <typename T, int J>
struct QuantStage {
  uint2 raw[J];
  int jobs, G;
  __device__ __forceinline__ void load(const uint16_t *x, int64_t ldx, int rows, int K) {
    G = K >> 7;
    jobs = rows * G;
    const int half = threadIdx.x >> 5, nhalf = blockDim.x >> 5, l = threadIdx.x & 31;
#pragma unroll
    for (int u = 0; u < J; ++u) {
      const int job = min(half + u * nhalf, jobs - 1);
      const int m = job / G, g = job - (job / G) * G;
      raw[u] = ldg_u2(x + m * ldx + g * 128 + l * 4);
    }
  }
  __device__ __forceinline__ void store(int K, int8_t *xq, float *xs) const {
    const int half = threadIdx.x >> 5, nhalf = blockDim.x >> 5, l = threadIdx.x & 31;
#pragma unroll
    for (int u = 0; u < J; ++u) {
      const int job = min(half + u * nhalf, jobs - 1);
      const int m = job / G, g = job - (job / G) * G;
      quantize_group<T>(raw[u], l, xq + m * K + g * 128, xs + m * G + g);
    }
  }
};

// Absmax over aligned runs of LPG lanes (8, 16 or 32): the DPP steps of
// halfwave_max that stay inside such a run.
template <int LPG>
__device__ __forceinline__ float group_max(float a) {
  static_assert(LPG == 8 || LPG == 16 || LPG == 32, "lanes per group");
  if constexpr (LPG == 32) {
    return halfwave_max(a);
  } else {
    a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0xB1, 0xF, 0xF, false)));
    a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x4E, 0xF, 0xF, false)));
    a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x141, 0xF, 0xF, false)));
    if constexpr (LPG == 16)
      a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x140, 0xF, 0xF, false)));
    return a;
  }
}

// QuantStage for a compile-time geometry: K = 128 G, TH threads, and LPG
// lanes per 128-group (VPL = 128 / LPG values per lane, loaded as 8-byte
// pieces like QuantStage's).  Group slot t (lanes LPG t ..) always takes
// group t % G, of rows t / G + (TH / LPG / G) u, u < J, so the group offset
// is fixed and each job adds one row stride: the generic stage's per-job
// index division and 64-bit row products are gone.  Fewer lanes per group
// give each lane more values, which spreads the per-group work (absmax,
// scale, reciprocal) over fewer lanes' instructions: with 8 rows of 2048 a
// 1024-thread block quantizes every group in one pass of 8-lane slots
// instead of four passes of half-waves.  Rows past `rows` redo the last row
// (the same bytes as its owner stores; no store is under a branch).  The
// arithmetic per value is quantize_group's (w8a8.py:8-14), so the bytes and
// scales are identical.  Covers up to J * TH / LPG / G rows.
template <typename T, int J, int G, int TH, int LPG>
struct QuantRows {
  static constexpr int VPL = 128 / LPG, NSLOT = TH / LPG, STEP = NSLOT / G;
  static_assert(NSLOT % G == 0 && VPL % 4 == 0, "whole rows per sweep of the group slots");
  uint2 raw[J][VPL / 4];
  int rows;
  __device__ __forceinline__ void load(const uint16_t *x, int64_t ldx, int nrows, int) {
    rows = nrows;
    const int t = threadIdx.x / LPG, l = threadIdx.x % LPG;
    const uint16_t *base = x + (t % G) * 128 + l * VPL;
    const int m0 = t / G;
#pragma unroll
    for (int u = 0; u < J; ++u) {
      const uint16_t *p = base + (int64_t)min(m0 + STEP * u, rows - 1) * ldx;
#pragma unroll
      for (int i = 0; i < VPL / 4; ++i) raw[u][i] = ldg_u2(p + 4 * i);
    }
  }
  __device__ __forceinline__ void store(int, int8_t *xq, float *xs) const {
    const int t = threadIdx.x / LPG, l = threadIdx.x % LPG;
    const int g = t % G, m0 = t / G;
    const float inv127 = (float)(1.0 / 127.0);
#pragma unroll
    for (int u = 0; u < J; ++u) {
      const int m = min(m0 + STEP * u, rows - 1);
      float v[VPL];
#pragma unroll
      for (int i = 0; i < VPL / 4; ++i) {
        v[4 * i] = T::to_f32(raw[u][i].x & 0xFFFFu);
        v[4 * i + 1] = T::to_f32(raw[u][i].x >> 16);
        v[4 * i + 2] = T::to_f32(raw[u][i].y & 0xFFFFu);
        v[4 * i + 3] = T::to_f32(raw[u][i].y >> 16);
      }
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) a = fmaxf(a, fabsf(v[i]));
      a = group_max<LPG>(a);
      const float sc = fmaxf(a, 1e-10f) * inv127;
      const float r = 1.0f / sc;
      uint32_t packed[VPL / 4];
#pragma unroll
      for (int i = 0; i < VPL / 4; ++i) {
        packed[i] = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          packed[i] |= ((uint32_t)(uint8_t)(int8_t)(int)rintf(quant_div(v[4 * i + k], sc, r)))
                       << (8 * k);
      }
      int8_t *dst = xq + m * (G * 128) + g * 128 + l * VPL;
      if constexpr (VPL == 4) {
        *reinterpret_cast<uint32_t *>(dst) = packed[0];
      } else if constexpr (VPL == 8) {
        *reinterpret_cast<uint2 *>(dst) = uint2{packed[0], packed[1]};
      } else {
        static_assert(VPL == 16, "values per lane");
        *reinterpret_cast<u32x4 *>(dst) = u32x4{packed[0], packed[1], packed[2], packed[3]};
      }
      if (l == 0) xs[m * G + g] = sc;
    }
  }
};

// Per-row dynamic quantization of `rows` activation rows of K 16-bit values
// into LDS (w8a8.py:8-14).  Each 128-group is handled by 32 lanes.
template <typename T>
__device__ __forceinline__ void quantize_rows_to_lds(const uint16_t *x, int64_t ldx, int rows,
                                                     int K, int8_t *xq, float *xs) {
  const int G = K >> 7;
  const int half = threadIdx.x >> 5;
  const int nhalf = blockDim.x >> 5;
  const int l = threadIdx.x & 31;
  // Jobs (row m, group g) in batches of B per half-wave.  Every load of a
  // batch is issued before the first is used, and the jobs are computed
  // branch-free (jobs past the end redo the last one; only the stores are
  // guarded), so their dependency chains interleave: a batch costs about one
  // load latency, not one per job.  The group absmax is four DPP steps inside
  // each 16-lane row and one shuffle across the two rows of the half-wave.
  constexpr int B = 8;
  const int jobs = rows * G;
  for (int base = half; base < jobs; base += nhalf * B) {
    uint2 raw[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int job = min(base + u * nhalf, jobs - 1);
      const int m = job / G, g = job - (job / G) * G;
      raw[u] = ldg_u2(x + m * ldx + g * 128 + l * 4);
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int job = min(base + u * nhalf, jobs - 1);
      const int m = job / G, g = job - (job / G) * G;
      quantize_group<T>(raw[u], l, xq + m * K + g * 128, xs + m * G + g);
    }
  }
}

// Sixteen int8 weights against sixteen int8 activations: exact int32.
__device__ __forceinline__ int dot16_i8(u32x4 w, u32x4 x) {
  int p = __builtin_amdgcn_sdot4((int)w[0], (int)x[0], 0, false);
  p = __builtin_amdgcn_sdot4((int)w[1], (int)x[1], p, false);
  p = __builtin_amdgcn_sdot4((int)w[2], (int)x[2], p, false);
  p = __builtin_amdgcn_sdot4((int)w[3], (int)x[3], p, false);
  return p;
}

// Sixteen dequantized weights (8 packed words) against sixteen 16-bit
// activations (two 16-byte vectors), fp32 accumulate.
template <typename T>
__device__ __forceinline__ float dot16_w16(const uint32_t wd[8], u32x4 x0, u32x4 x1) {
  float a = 0.0f;
  a = T::dot2(wd[0], x0[0], a);
  a = T::dot2(wd[1], x0[1], a);
  a = T::dot2(wd[2], x0[2], a);
  a = T::dot2(wd[3], x0[3], a);
  a = T::dot2(wd[4], x1[0], a);
  a = T::dot2(wd[5], x1[1], a);
  a = T::dot2(wd[6], x1[2], a);
  a = T::dot2(wd[7], x1[3], a);
  return a;
}

// The W8A8 reference epilogue over one row's group partials (w8a8.py:40):
// acc = acc + (float(p_g) * xs_g) * ws_g for g ascending, no FMA.
// The terms of eight groups are formed together (their LDS reads in flight
// at once) and then added in ascending order, which leaves the sum unchanged.
__device__ __forceinline__ float w8a8_epilogue(const int *p, const float *xs, const float *ws,
                                               int G) {
  float acc = 0.0f;
  int g = 0;
  for (; g + 8 <= G; g += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = mul_rn(mul_rn((float)p[g + u], xs[g + u]), ws[g + u]);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = add_rn(acc, t[u]);
  }
  for (; g < G; ++g) acc = add_rn(acc, mul_rn(mul_rn((float)p[g], xs[g]), ws[g]));
  return acc;
}

// Ascending-order fp32 sum of G values, eight reads in flight at a time.
__device__ __forceinline__ float ordered_sum8(const float *v, int G) {
  float acc = 0.0f;
  int g = 0;
  for (; g + 8 <= G; g += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = v[g + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += t[u];
  }
  for (; g < G; ++g) acc += v[g];
  return acc;
}

}  // namespace lm
