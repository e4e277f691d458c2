// Routing side of the MoE block:
//   router logits (fp64 accumulation, bf16-rounded) + top-k + softmax renorm
//                                                   (HF:768-776)
//   device route plan: stable token sort / permute  (gpu_routes.py:17-63)
//   ordered combines for decode and prefill         (int8.py:240-250, prefill.py:37-49)
//   SwiGLU glue, RMSNorm                            (HF:715, HF:801-815)
#include <type_traits>

#include "internal.hpp"

namespace lm {

// ============================================================ router logits
// logit[t, e] = f32(bf16(f32(sum_k f64(x[t,k]) * f64(w[e,k])))) (+ bias[e]).
// Products of two bf16 values are exact in fp64 and the fp64 sum of 2048 of
// them is exact unless operands span more than ~37 binary orders of
// magnitude, so the result does not depend on the summation order; the
// kernels below may therefore permute k freely.

// Small token counts (decode): one wave per (expert, token-block), VALU fp64.
template <int MT>
__global__ __launch_bounds__(256) void router_logits_gemv(const uint16_t *__restrict__ x,
                                                          const uint16_t *__restrict__ w,
                                                          const float *__restrict__ bias,
                                                          float *__restrict__ logits, int T,
                                                          int E, int H) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  double acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0;
  const uint16_t *wr = w + (int64_t)e * H;
  for (int k0 = lane * 8; k0 < H; k0 += 512) {
    const u32x4 wv = ldg16(wr + k0);
    double wd[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wd[2 * j] = (double)bf16_bits_to_f32(wv[j] & 0xFFFFu);
      wd[2 * j + 1] = (double)bf16_bits_to_f32(wv[j] >> 16);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < T) {
        const u32x4 xv = ldg16(x + (int64_t)m * H + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[m] = __builtin_fma((double)bf16_bits_to_f32(xv[j] & 0xFFFFu), wd[2 * j], acc[m]);
          acc[m] = __builtin_fma((double)bf16_bits_to_f32(xv[j] >> 16), wd[2 * j + 1], acc[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m < T) {
      const double s = wave_sum_f64_dpp(acc[m]);
      if (lane == 0) {
        float l = round_bf16((float)s);
        if (bias) l = l + bias[e];
        logits[(int64_t)m * E + e] = l;
      }
    }
  }
}

// Large token counts (prefill): v_mfma_f64_16x16x4f64.  Block = 4 waves,
// tile 16 tokens x 128 experts, each wave 16 x 32.  Lane quad q supplies
// k = k0 + 8 q + j at MFMA step j (the same permutation for both operands),
// so one 16-byte load per operand row feeds 8 MFMA steps.
template <int D>
__global__ __launch_bounds__(256) void router_logits_mfma(const uint16_t *__restrict__ x,
                                                          const uint16_t *__restrict__ w,
                                                          const float *__restrict__ bias,
                                                          float *__restrict__ logits, int T,
                                                          int E, int H) {
  // One wave = 16 tokens x 32 experts; K in 32-wide stages held in a
  // D-stage register ring (D - 1 stages in flight while one is consumed;
  // H must be a multiple of 32 D).  Even and odd K-steps accumulate into
  // separate fp64 tiles, added at the end, so four independent MFMA chains
  // are in flight.
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t0 = blockIdx.x * 16;
  const int e0 = blockIdx.y * 128 + wave * 32;
  if (e0 >= E) return;
  const int q = lane >> 4;
  const int r = lane & 15;
  const uint16_t *xa = x + (int64_t)min(t0 + r, T - 1) * H + q * 8;
  const uint16_t *wb0 = w + (int64_t)min(e0 + r, E - 1) * H + q * 8;
  const uint16_t *wb1 = w + (int64_t)min(e0 + 16 + r, E - 1) * H + q * 8;
  f64x4 acc[2][2] = {{{0.0, 0.0, 0.0, 0.0}, {0.0, 0.0, 0.0, 0.0}},
                     {{0.0, 0.0, 0.0, 0.0}, {0.0, 0.0, 0.0, 0.0}}};
  u32x4 ra[D], rb0[D], rb1[D];
  const int last = H - 32;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int k = min(32 * d, last);
    ra[d] = ldg16(xa + k);
    rb0[d] = ldg16(wb0 + k);
    rb1[d] = ldg16(wb1 + k);
  }
  for (int k0 = 0; k0 < H; k0 += 32 * D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const u32x4 av = ra[u], bv0 = rb0[u], bv1 = rb1[u];
      // refill the slot with the stage D ahead (clamped: past the end the
      // last stage is re-read and never consumed)
      const int kn = min(k0 + 32 * (u + D), last);
      ra[u] = ldg16(xa + kn);
      rb0[u] = ldg16(wb0 + kn);
      rb1[u] = ldg16(wb1 + kn);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sh = (j & 1) ? 16u : 0u;
        const double a = (double)bf16_bits_to_f32((av[j >> 1] >> sh) & 0xFFFFu);
        const double b0 = (double)bf16_bits_to_f32((bv0[j >> 1] >> sh) & 0xFFFFu);
        const double b1 = (double)bf16_bits_to_f32((bv1[j >> 1] >> sh) & 0xFFFFu);
        acc[j & 1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b0, acc[j & 1][0], 0, 0, 0);
        acc[j & 1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b1, acc[j & 1][1], 0, 0, 0);
      }
    }
  }
  // D layout of the f64 16x16x4 MFMA: lane holds column (lane & 15) and
  // rows (lane >> 4) + 4 i, i = 0..3 (unlike the 4 (lane >> 4) + i rows of the
  // 32-bit-output 16x16 MFMAs).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + q + 4 * i;
    if (t >= T) continue;
    const int ea = e0 + r, eb = e0 + 16 + r;
    if (ea < E) {
      float l = round_bf16((float)(acc[0][0][i] + acc[1][0][i]));
      if (bias) l = l + bias[ea];
      logits[(int64_t)t * E + ea] = l;
    }
    if (eb < E) {
      float l = round_bf16((float)(acc[0][1][i] + acc[1][1][i]));
      if (bias) l = l + bias[eb];
      logits[(int64_t)t * E + eb] = l;
    }
  }
}

// ============================================================ top-k
__global__ __launch_bounds__(256) void topk_kernel(const float *__restrict__ logits, int T, int E,
                                                   int K, int64_t *__restrict__ ids,
                                                   uint16_t *__restrict__ weights) {
  __shared__ unsigned long long scratch[4][kTopkScratch];
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  topk_wave(logits + (int64_t)t * E, E, K, lane, scratch[threadIdx.x >> 6], ids + (int64_t)t * K,
            weights + (int64_t)t * K);
}

int router_logits(const uint16_t *x, const uint16_t *w, const float *bias, float *logits,
                  int64_t T, int64_t E, int64_t H, hipStream_t st) {
  if (T <= 8) {
    const unsigned g = cdiv(E, 4);
    if (T == 1)
      router_logits_gemv<1><<<g, 256, 0, st>>>(x, w, bias, logits, (int)T, (int)E, (int)H);
    else
      router_logits_gemv<8><<<g, 256, 0, st>>>(x, w, bias, logits, (int)T, (int)E, (int)H);
  } else {
    const dim3 grid(cdiv(T, 16), cdiv(E, 128));
    if (H % 128 == 0)
      router_logits_mfma<4><<<grid, 256, 0, st>>>(x, w, bias, logits, (int)T, (int)E, (int)H);
    else
      router_logits_mfma<1><<<grid, 256, 0, st>>>(x, w, bias, logits, (int)T, (int)E, (int)H);
  }
  return check_launch("router_logits");
}

int router_topk(const float *logits, int64_t T, int64_t E, int64_t K, int64_t *ids,
                uint16_t *weights, hipStream_t st) {
  topk_kernel<<<cdiv(T, 4), 256, 0, st>>>(logits, (int)T, (int)E, (int)K, ids, weights);
  return check_launch("topk_kernel");
}

// ============================================================ route plan
// Stable counting sort of the flat route ids by expert, one 1024-thread block.
// Wave w owns a contiguous slice of the routes and walks it 64 at a time:
// lanes holding the same expert id find each other with eight ballots over
// the id bits, so a route's rank among equal ids inside the slice is the
// wave's running count for that expert plus the equal ids in lower lanes.
// A column scan over the 16 per-wave counts and a scan over experts turn
// these slice ranks into positions of the stable order - three block
// barriers in total.  ids are clamped into [0, E), so a malformed id can
// never index out of bounds.
constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
// Routes per call whose ids and ranks are staged in LDS (ids as bytes,
// ranks as 16-bit); larger calls keep the ranks in the `ordered` output.
constexpr int kPlanLdsRoutes = 40960;

// Exclusive scan of one value per thread over the first 256 threads of a
// 1024-thread block (the others pass 0); returns the prefix, *total = sum.
__device__ int block_scan_256(int v, int *scratch, int *total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  if (lane == 63 && wave < 4) scratch[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < wave && i < 4; ++i) base += scratch[i];
  const int all = scratch[0] + scratch[1] + scratch[2] + scratch[3];
  __syncthreads();
  *total = all;
  return base + incl - v;
}

// Stable sort of up to N (id, slot, value) triples by id with an odd-even
// transposition network (static register indices only).
template <int N>
__device__ __forceinline__ void sort_triples(int (&id)[N], int (&sl)[N], int (&v)[N]) {
#pragma unroll
  for (int pass = 0; pass < N; ++pass) {
#pragma unroll
    for (int i = pass & 1; i + 1 < N; i += 2) {
      if (id[i] > id[i + 1]) {
        const int a = id[i], b = sl[i], c = v[i];
        id[i] = id[i + 1];
        sl[i] = sl[i + 1];
        v[i] = v[i + 1];
        id[i + 1] = a;
        sl[i + 1] = b;
        v[i + 1] = c;
      }
    }
  }
}

template <bool LDS>
__global__ __launch_bounds__(1024) void route_plan_kernel(const int64_t *__restrict__ ids, int T,
                                                          int K, int E, int bm,
                                                          int64_t *__restrict__ pos,
                                                          int64_t *__restrict__ table,
                                                          int max_tiles,
                                                          int64_t *__restrict__ ordered,
                                                          int64_t *__restrict__ slots,
                                                          int shared_rows) {
  __shared__ int offs[257], tends[256], scratch[4];
  __shared__ int wcnt[kPlanWaves][256];
  __shared__ uint8_t sid8[LDS ? kPlanLdsRoutes : 1];
  __shared__ uint16_t srank[LDS ? kPlanLdsRoutes : 1];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int R = T * K;
  const unsigned long long lt = (1ull << lane) - 1ull;
  auto load_eid = [&](int i) -> int {
    const int64_t e = ids[i];
    return (int)(e < 0 ? 0 : (e >= E ? E - 1 : e));
  };
  auto eid = [&](int i) -> int {
    if constexpr (LDS) return sid8[i];
    else return load_eid(i);
  };
  auto rank_get = [&](int r) -> int {
    if constexpr (LDS) return srank[r];
    else return (int)ordered[r];
  };
  auto rank_set = [&](int r, int v) {
    if constexpr (LDS) srank[r] = (uint16_t)v;
    else ordered[r] = v;
  };
  if constexpr (LDS) {
#pragma unroll 8
    for (int r = t; r < R; r += kPlanThreads) sid8[r] = (uint8_t)load_eid(r);
  }
  if (t < 256)
    for (int w = 0; w < kPlanWaves; ++w) wcnt[w][t] = 0;
  __syncthreads();

  // Pass 1: rank of every route among equal ids of its wave's slice.
  const int slice = ((R + kPlanWaves - 1) / kPlanWaves + 63) & ~63;
  const int lo = wave * slice, hi = min(lo + slice, R);
  for (int base = lo; base < hi; base += 64) {
    const int r = base + lane;
    const bool valid = r < hi;
    const int e = valid ? eid(r) : 0;
    unsigned long long same = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const unsigned long long bit = __ballot(valid && ((e >> b) & 1));
      same &= ((e >> b) & 1) ? bit : ~bit;
    }
    const int in_chunk = __popcll(same & lt);
    const int before = valid ? wcnt[wave][e] : 0;
    if (valid) rank_set(r, before + in_chunk);
    if (valid && in_chunk == 0) wcnt[wave][e] = before + __popcll(same);
  }
  __syncthreads();
  // Column scan: wcnt[w][e] becomes the count of e in slices before w.
  int total_e = 0;
  if (t < 256) {
    for (int w = 0; w < kPlanWaves; ++w) {
      const int c = wcnt[w][t];
      wcnt[w][t] = total_e;
      total_e += c;
    }
  }
  int all;
  const int ex = block_scan_256(t < E ? total_e : 0, scratch, &all);
  if (t < 256) offs[t] = ex;
  if (t == 0) offs[256] = all;
  __syncthreads();

  // Pass 2: sorted position p of every route; pos[p] = its token.
  for (int r = t; r < R; r += kPlanThreads) {
    const int e = eid(r);
    const int p = offs[e] + wcnt[r / slice][e] + rank_get(r);
    pos[p] = r / K;
    rank_set(r, p);
  }

  // Tile table (gpu_routes._table): tiles of bm rows, expert by expert.
  const int nt = t < E ? (offs[t + 1] - offs[t] + bm - 1) / bm : 0;
  int ntot;
  const int tex = block_scan_256(nt, scratch, &ntot);
  if (t < 256) tends[t] = tex + nt;
  __syncthreads();
  for (int i = t; i < max_tiles; i += kPlanThreads) {
    int64_t ex_ = 0, st_ = 0, sp_ = 0;
    if (i < ntot) {
      int l = 0, h = E;
      while (l < h) {
        const int mid = (l + h) >> 1;
        if (tends[mid] <= i) l = mid + 1;
        else h = mid;
      }
      const int prior = l > 0 ? tends[l - 1] : 0;
      ex_ = l;
      st_ = offs[l] + (int64_t)(i - prior) * bm;
      sp_ = offs[l + 1];
    }
    table[i * 3] = ex_;
    table[i * 3 + 1] = st_;
    table[i * 3 + 2] = sp_;
  }
  // Always-on shared expert: its rows follow the R routed rows, gathered in
  // token order, as extra tiles of expert E after the plan's max_tiles rows.
  if (shared_rows > 0) {
    const int nst = (shared_rows + bm - 1) / bm;
    for (int j = t; j < nst; j += kPlanThreads) {
      table[(int64_t)(max_tiles + j) * 3] = E;
      table[(int64_t)(max_tiles + j) * 3 + 1] = R + (int64_t)j * bm;
      table[(int64_t)(max_tiles + j) * 3 + 2] = R + shared_rows;
    }
    for (int tok = t; tok < shared_rows; tok += kPlanThreads) pos[R + tok] = tok;
  }
  __threadfence_block();
  __syncthreads();

  // slots = argsort(ids, dim=1, stable); ordered[t, i] = inverse[t*K + slots[t, i]].
  auto token_order = [&](auto n_tag) {
    constexpr int N = decltype(n_tag)::value;
    for (int tok = t; tok < T; tok += kPlanThreads) {
      int id[N], sl[N], iv[N];
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const bool in = j < K;
        id[j] = in ? eid(tok * K + j) : 0x7FFFFFFF;
        sl[j] = j;
        iv[j] = in ? rank_get(tok * K + j) : 0;
      }
      sort_triples<N>(id, sl, iv);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        if (j < K) {
          slots[(int64_t)tok * K + j] = sl[j];
          ordered[(int64_t)tok * K + j] = iv[j];
        }
      }
    }
  };
  if (K <= 8) token_order(std::integral_constant<int, 8>{});
  else token_order(std::integral_constant<int, 16>{});
}

int route_plan(const int64_t *ids, int64_t T, int64_t K, int64_t E, int64_t bm, int64_t *pos,
               int64_t *table, int64_t max_tiles, int64_t *ordered, int64_t *slots,
               int64_t shared_rows, hipStream_t st) {
  if (T * K <= kPlanLdsRoutes)
    route_plan_kernel<true><<<1, kPlanThreads, 0, st>>>(ids, (int)T, (int)K, (int)E, (int)bm, pos,
                                                        table, (int)max_tiles, ordered, slots,
                                                        (int)shared_rows);
  else
    route_plan_kernel<false><<<1, kPlanThreads, 0, st>>>(ids, (int)T, (int)K, (int)E, (int)bm,
                                                         pos, table, (int)max_tiles, ordered,
                                                         slots, (int)shared_rows);
  return check_launch("route_plan_kernel");
}

// ============================================================ combines
__device__ __forceinline__ float load_weight(const void *w, int dtype, int64_t i) {
  if (dtype == LM_FP32) return static_cast<const float *>(w)[i];
  const uint16_t b = static_cast<const uint16_t *>(w)[i];
  return dtype == LM_FP16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b);
}

// int8._ordered_reduce: ascending table order, rounding to the output dtype T
// at every step.  A table slot outside [0, E) is clamped into it.
template <typename T>
__global__ __launch_bounds__(256) void ordered_reduce_kernel(const uint16_t *__restrict__ v,
                                                             const int64_t *__restrict__ table,
                                                             const void *w, int w_dtype,
                                                             uint16_t *__restrict__ y, int N,
                                                             int E) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float acc = 0.0f;
  for (int e = 0; e < E; ++e) {
    const int64_t slot = clamp_index(table[e * 5 + 4], E);
    const float wt = load_weight(w, w_dtype, slot);
    const float val = T::round(T::to_f32(v[(int64_t)e * N + n]) * wt);
    acc = T::round(acc + val);
  }
  y[n] = T::from_f32(acc);
}

// prefill._reduce: per token, routes in ascending expert order, rounding to
// T at every step.  Routes are clamped into [0, tokens * K), slots into [0, K).
template <typename T>
__global__ __launch_bounds__(256) void routed_reduce_kernel(const uint16_t *__restrict__ v,
                                                            const int64_t *__restrict__ ordered,
                                                            const int64_t *__restrict__ slots,
                                                            const void *w, int w_dtype,
                                                            uint16_t *__restrict__ y, int N,
                                                            int K, int64_t routes) {
  const int tok = blockIdx.y;
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float acc = 0.0f;
  for (int i = 0; i < K; ++i) {
    const int64_t route = clamp_index(ordered[(int64_t)tok * K + i], routes);
    const int64_t slot = clamp_index(slots[(int64_t)tok * K + i], K);
    const float wt = load_weight(w, w_dtype, (int64_t)tok * K + slot);
    const float val = T::round(T::to_f32(v[route * N + n]) * wt);
    acc = T::round(acc + val);
  }
  y[(int64_t)tok * N + n] = T::from_f32(acc);
}

// SwiGLU glue on a [rows, 2*half] gate_up tensor of dtype T.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *__restrict__ gu,
                                                     uint16_t *__restrict__ h, int64_t rows,
                                                     int64_t half) {
  const int64_t total = rows * half;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / half, c = i - r * half;
    const float g = T::to_f32(gu[r * 2 * half + c]);
    const float u = T::to_f32(gu[r * 2 * half + half + c]);
    h[i] = T::from_f32(T::round(silu_f32(g)) * u);
  }
}

// RMSNorm (HF:807-815) on rows of n bf16 values; one block per row.  The sum
// of squares uses a fixed tree - thread t sums its contiguous chunk of
// ceil(n/256) elements in order, a 64-lane xor butterfly per wave, then the
// four wave sums left to right - and r = 1 / sqrt(mean + eps) with IEEE
// sqrt and division, so the result is reproducible bit for bit.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t *__restrict__ x,
                                                      const float *__restrict__ w,
                                                      uint16_t *__restrict__ y, int n,
                                                      float eps) {
  __shared__ float red[4];
  const uint16_t *xr = x + (int64_t)blockIdx.x * n;
  uint16_t *yr = y + (int64_t)blockIdx.x * n;
  const int per = (n + 255) / 256;
  const int lo = min(threadIdx.x * per, n), hi = min(lo + per, n);
  float ss = 0.0f;
  for (int i = lo; i < hi; ++i) {
    const float v = bf16_bits_to_f32(xr[i]);
    ss += v * v;
  }
  ss = wave_sum_f32(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float r = 1.0f / sqrtf(tot / (float)n + eps);
  for (int i = lo; i < hi; ++i) {
    float v = bf16_bits_to_f32(xr[i]) * r;
    if (w) v = v * (1.0f + w[i]);
    yr[i] = f32_to_bf16_bits(v);
  }
}

}  // namespace lm

using namespace lm;

extern "C" int lm_router_topk(const void *x, const void *w, const float *bias, float *logits,
                              int64_t *ids, void *weights, int64_t tokens, int64_t experts,
                              int64_t hidden, int64_t top_k, void *stream) {
  LM_REQUIRE(experts >= 1 && experts <= 256, LM_EINVAL, "router supports 1..256 experts");
  LM_REQUIRE(top_k >= 1 && top_k <= 16 && top_k <= experts, LM_EINVAL, "invalid top_k");
  LM_REQUIRE(hidden > 0 && hidden % 32 == 0, LM_EINVAL, "hidden must be a multiple of 32");
  LM_REQUIRE(tokens >= 0, LM_EINVAL, "invalid token count");
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && w && logits && ids && weights, LM_EINVAL, "null pointer");
  hipStream_t st = as_stream(stream);
  if (int rc = router_logits(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(w),
                             bias, logits, tokens, experts, hidden, st))
    return rc;
  return router_topk(logits, tokens, experts, top_k, ids, static_cast<uint16_t *>(weights), st);
}

extern "C" int lm_route_plan(const int64_t *ids, int64_t tokens, int64_t top_k, int64_t experts,
                             int64_t bm, int64_t *pos, int64_t *table, int64_t max_tiles,
                             int64_t *ordered, int64_t *slots, void *stream) {
  LM_REQUIRE(tokens >= 1 && top_k >= 1 && top_k <= 16, LM_EINVAL,
             "Expected contiguous CUDA [tokens,top_k] routing IDs");
  LM_REQUIRE(experts >= 1 && experts <= 256, LM_EINVAL, "route plan supports 1..256 experts");
  LM_REQUIRE(bm >= 1, LM_EINVAL, "tile height must be positive");
  LM_REQUIRE(tokens * top_k < (1LL << 30), LM_EINVAL, "too many routes");
  LM_REQUIRE(max_tiles == (tokens * top_k + bm - 1) / bm + experts, LM_EINVAL,
             "max_tiles must be cdiv(routes, bm) + experts");
  LM_REQUIRE(ids && pos && table && ordered && slots, LM_EINVAL, "null pointer");
  return route_plan(ids, tokens, top_k, experts, bm, pos, table, max_tiles, ordered, slots, 0,
                    as_stream(stream));
}

extern "C" int lm_ordered_reduce(const void *v, const int64_t *table, const void *w, int w_dtype,
                                 void *y, int64_t n, int64_t experts, int dtype, void *stream) {
  LM_REQUIRE(n > 0 && experts >= 0, LM_EINVAL, "invalid reduce geometry");
  LM_REQUIRE(w_dtype == LM_BF16 || w_dtype == LM_FP16 || w_dtype == LM_FP32, LM_EINVAL,
             "weights must be bf16, fp16 or fp32");
  LM_REQUIRE(dtype == LM_BF16 || dtype == LM_FP16, LM_EINVAL, "values must be bf16 or fp16");
  LM_REQUIRE(v && table && w && y, LM_EINVAL, "null pointer");
  const unsigned g = cdiv(n, 256);
  const uint16_t *vp = static_cast<const uint16_t *>(v);
  uint16_t *yp = static_cast<uint16_t *>(y);
  if (dtype == LM_BF16)
    ordered_reduce_kernel<BF16><<<g, 256, 0, as_stream(stream)>>>(vp, table, w, w_dtype, yp,
                                                                  (int)n, (int)experts);
  else
    ordered_reduce_kernel<FP16><<<g, 256, 0, as_stream(stream)>>>(vp, table, w, w_dtype, yp,
                                                                  (int)n, (int)experts);
  return check_launch("ordered_reduce_kernel");
}

extern "C" int lm_routed_reduce(const void *v, const int64_t *ordered, const int64_t *slots,
                                const void *w, int w_dtype, void *y, int64_t tokens, int64_t n,
                                int64_t top_k, int dtype, void *stream) {
  LM_REQUIRE(n > 0 && tokens >= 0 && top_k >= 1, LM_EINVAL, "invalid reduce geometry");
  LM_REQUIRE(w_dtype == LM_BF16 || w_dtype == LM_FP16 || w_dtype == LM_FP32, LM_EINVAL,
             "weights must be bf16, fp16 or fp32");
  LM_REQUIRE(dtype == LM_BF16 || dtype == LM_FP16, LM_EINVAL, "values must be bf16 or fp16");
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(tokens < 65536, LM_EINVAL, "too many tokens for one launch");
  LM_REQUIRE(v && ordered && slots && w && y, LM_EINVAL, "null pointer");
  const dim3 grid(cdiv(n, 256), (unsigned)tokens);
  const uint16_t *vp = static_cast<const uint16_t *>(v);
  uint16_t *yp = static_cast<uint16_t *>(y);
  if (dtype == LM_BF16)
    routed_reduce_kernel<BF16><<<grid, 256, 0, as_stream(stream)>>>(
        vp, ordered, slots, w, w_dtype, yp, (int)n, (int)top_k, tokens * top_k);
  else
    routed_reduce_kernel<FP16><<<grid, 256, 0, as_stream(stream)>>>(
        vp, ordered, slots, w, w_dtype, yp, (int)n, (int)top_k, tokens * top_k);
  return check_launch("routed_reduce_kernel");
}

extern "C" int lm_swiglu(const void *gu, void *h, int64_t rows, int64_t half, int dtype,
                         void *stream) {
  LM_REQUIRE(rows >= 0 && half > 0, LM_EINVAL, "invalid SwiGLU geometry");
  LM_REQUIRE(dtype == LM_BF16 || dtype == LM_FP16, LM_EINVAL, "SwiGLU input must be bf16 or fp16");
  if (rows == 0) return LM_OK;
  LM_REQUIRE(gu && h, LM_EINVAL, "null pointer");
  int64_t blocks = (rows * half + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  const uint16_t *gp = static_cast<const uint16_t *>(gu);
  uint16_t *hp = static_cast<uint16_t *>(h);
  if (dtype == LM_BF16)
    swiglu_kernel<BF16><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(gp, hp, rows, half);
  else
    swiglu_kernel<FP16><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(gp, hp, rows, half);
  return check_launch("swiglu_kernel");
}

extern "C" int lm_rmsnorm(const void *x, const float *w, void *y, int64_t rows, int64_t n,
                          float eps, void *stream) {
  LM_REQUIRE(rows >= 0 && n > 0, LM_EINVAL, "invalid RMSNorm geometry");
  if (rows == 0) return LM_OK;
  LM_REQUIRE(rows < (1LL << 31) && x && y, LM_EINVAL, "null pointer");
  rmsnorm_kernel<<<(unsigned)rows, 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t *>(x), w, static_cast<uint16_t *>(y), (int)n, eps);
  return check_launch("rmsnorm_kernel");
}
