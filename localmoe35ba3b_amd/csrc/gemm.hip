// W8A16 MFMA GEMM for prefill (gfx950, v_mfma_f32_16x16x32_{bf16,f16}).
//
// Used three ways:
//   dense   y = x . dequant(q)^T                 lm_w8a16_linear, m > 8 (int8.py:9-37)
//   routed  per tile (e, start, stop) of a route-plan table, rows gathered
//           through pos (gate_up) or contiguous (down)   (prefill.py:12-34)
//   swiglu  the gate_up variant with bf16(bf16(silu(gate)) * up) fused in the
//           epilogue                                     (prefill.py:75-78)
//
// Block = 256 threads (4 waves), tile BM x 128 columns, K staged 64 at a time.
// Weights stay int8 until they are written to LDS: each thread dequantizes
// its 16 int8 weights to T(q * s) exactly (the reference rounds the
// dequantized weight to the activation dtype before the MMA, int8.py:21),
// so the MFMA consumes bit-identical operands to the reference's tl.dot.
// Registers prefetch stage k+1 from HBM while the MFMAs consume stage k.
// In SwiGLU mode a 128-column tile is 64 gate columns + the matching 64 up
// columns, split so that every lane holds a gate value and its up partner.
#include "internal.hpp"

namespace lm {

constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLDA = kBK + 8;  // 16-bit elements per LDS row (16 B pad: no bank conflicts)

struct GemmArgs {
  const uint16_t *x;
  int64_t ldx;
  const int64_t *pos;    // gather map (routed gate_up)
  const int64_t *table;  // [tiles, 3] (expert, start, stop)
  int64_t M;             // dense rows
  const int8_t *q;
  int64_t q_es;
  const float *s;
  int64_t s_es;
  uint16_t *y;
  int64_t ldy;
  int N;
  int K;
  int tile_rows;  // rows covered by one table tile (<= BM)
};

template <typename T, int BM, int WM, bool SWIGLU, bool GATHER, bool DENSE>
__global__ __launch_bounds__(256) void w8a16_mfma_kernel(GemmArgs a) {
  constexpr int WN = 4 / WM;
  constexpr int TM = BM / WM;
  constexpr int TN = kBN / WN;
  constexpr int MI = TM / 16;
  constexpr int NI = TN / 16;
  constexpr int ACH = BM / 32;  // 16-byte A chunks per thread per stage
  __shared__ __align__(16) uint16_t As[BM * kLDA];
  __shared__ __align__(16) uint16_t Bs[kBN * kLDA];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int nt = blockIdx.x;
  const int mt = blockIdx.y;

  int64_t e = 0, start, stop;
  if constexpr (DENSE) {
    start = (int64_t)mt * BM;
    stop = a.M;
  } else {
    e = a.table[mt * 3];
    start = a.table[mt * 3 + 1];
    stop = a.table[mt * 3 + 2];
    if (start >= stop) return;
  }
  const int rows = (int)min((int64_t)(DENSE ? BM : a.tile_rows), stop - start);
  const int8_t *wq = a.q + e * a.q_es;
  const float *wsc = a.s + e * a.s_es;
  const int K = a.K;
  const int G = K >> 7;
  const int half = a.N >> 1;
  const int n0 = SWIGLU ? nt * (kBN / 2) : nt * kBN;

  // Local column c of the tile -> weight row (or -1 when past the end).
  auto wrow = [&](int c) -> int {
    if constexpr (SWIGLU) {
      const int j = n0 + (c & (kBN / 2 - 1));
      if (j >= half) return -1;
      return c < kBN / 2 ? j : half + j;
    } else {
      const int j = n0 + c;
      return j < a.N ? j : -1;
    }
  };

  // Per-thread global sources.
  const uint16_t *asrc[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + 256 * i;
    const int r = min(c >> 3, rows - 1);
    const int64_t xr = GATHER ? a.pos[start + r] : start + r;
    asrc[i] = a.x + xr * a.ldx + (c & 7) * 8;
  }
  const int8_t *bsrc[2];
  const float *ssrc[2];
  bool bok[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;
    const int wr = wrow(c >> 2);
    bok[i] = wr >= 0;
    const int wr0 = bok[i] ? wr : 0;
    bsrc[i] = wq + (int64_t)wr0 * K + (c & 3) * 16;
    ssrc[i] = wsc + (int64_t)wr0 * G;
  }

  u32x4 areg[ACH], breg[2];
  float sreg[2];
  auto prefetch = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < ACH; ++i) areg[i] = ldg16(asrc[i] + k0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      breg[i] = bok[i] ? ldg16(bsrc[i] + k0) : u32x4{0u, 0u, 0u, 0u};
      sreg[i] = bok[i] ? ssrc[i][k0 >> 7] : 0.0f;
    }
  };

  f32x4 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto col_base = [&](int ni) -> int {
    if constexpr (SWIGLU) {
      return ni < NI / 2 ? wn * (TN / 2) + ni * 16 : kBN / 2 + wn * (TN / 2) + (ni - NI / 2) * 16;
    } else {
      return wn * TN + ni * 16;
    }
  };

  const int KT = K / kBK;
  prefetch(0);
  for (int kt = 0; kt < KT; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&As[(c >> 3) * kLDA + (c & 7) * 8]) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + 256 * i;
      uint32_t wd[8];
      dequant16<T>(breg[i], sreg[i], wd);
      uint16_t *dst = &Bs[(c >> 2) * kLDA + (c & 3) * 16];
      *reinterpret_cast<u32x4 *>(dst) = u32x4{wd[0], wd[1], wd[2], wd[3]};
      *reinterpret_cast<u32x4 *>(dst + 8) = u32x4{wd[4], wd[5], wd[6], wd[7]};
    }
    __syncthreads();
    if (kt + 1 < KT) prefetch(kt + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      const int kk = ks * 32 + (lane >> 4) * 8;
      u32x4 af[MI], bfr[NI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        af[mi] = *reinterpret_cast<const u32x4 *>(
            &As[(wm * TM + mi * 16 + (lane & 15)) * kLDA + kk]);
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bfr[ni] = *reinterpret_cast<const u32x4 *>(&Bs[(col_base(ni) + (lane & 15)) * kLDA + kk]);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = T::mfma16x16x32(af[mi], bfr[ni], acc[mi][ni]);
    }
  }

  // Epilogue.  MFMA 16x16 layout: lane holds column (lane & 15) and rows
  // 4 * (lane >> 4) + it, it = 0..3, of each 16x16 tile.
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int rl = wm * TM + mi * 16 + (lane >> 4) * 4 + it;
      if (rl >= rows) continue;
      uint16_t *yrow = a.y + (start + rl) * a.ldy;
      if constexpr (SWIGLU) {
#pragma unroll
        for (int ni = 0; ni < NI / 2; ++ni) {
          const int col = n0 + wn * (TN / 2) + ni * 16 + (lane & 15);
          if (col < half) {
            const float gate = T::round(acc[mi][ni][it]);
            const float up = T::round(acc[mi][ni + NI / 2][it]);
            const float act = T::round(silu_f32(gate));
            yrow[col] = T::from_f32(act * up);
          }
        }
      } else {
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          const int col = n0 + col_base(ni) + (lane & 15);
          if (col < a.N) yrow[col] = T::from_f32(acc[mi][ni][it]);
        }
      }
    }
  }
}

template <typename T, int BM, int WM, bool SWIGLU, bool GATHER, bool DENSE>
static int launch_gemm(const GemmArgs &a, unsigned mtiles, hipStream_t st) {
  const int nt = SWIGLU ? (int)cdiv(a.N / 2, kBN / 2) : (int)cdiv(a.N, kBN);
  if (mtiles == 0) return LM_OK;
  w8a16_mfma_kernel<T, BM, WM, SWIGLU, GATHER, DENSE><<<dim3(nt, mtiles), 256, 0, st>>>(a);
  return check_launch("w8a16_mfma_kernel");
}

int w8a16_gemm_dense(const void *x, const int8_t *q, const float *s, void *y, int64_t m,
                     int64_t n, int64_t k, int dtype, int large_tile, hipStream_t st) {
  GemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = k;
  a.M = m;
  a.q = q;
  a.s = s;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = n;
  a.N = (int)n;
  a.K = (int)k;
  (void)large_tile;
  const unsigned mt = cdiv(m, 128);
  if (dtype == LM_BF16) return launch_gemm<BF16, 128, 2, false, false, true>(a, mt, st);
  return launch_gemm<FP16, 128, 2, false, false, true>(a, mt, st);
}

// Routed grouped GEMM over a (expert, start, stop) tile table of height bm.
int routed_gemm(const void *x, const int8_t *q, const float *s, const int64_t *pos,
                const int64_t *table, int64_t n_tiles, int64_t bm, void *y, int64_t n, int64_t k,
                bool gather, bool swiglu, int64_t q_es, int64_t s_es, int64_t ldx,
                hipStream_t st) {
  GemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = ldx;
  a.pos = pos;
  a.table = table;
  a.q = q;
  a.q_es = q_es;
  a.s = s;
  a.s_es = s_es;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = swiglu ? n / 2 : n;
  a.N = (int)n;
  a.K = (int)k;
  a.tile_rows = (int)bm;
  const unsigned mt = (unsigned)n_tiles;
  if (bm <= 64) {
    if (swiglu)
      return gather ? launch_gemm<BF16, 64, 1, true, true, false>(a, mt, st)
                    : launch_gemm<BF16, 64, 1, true, false, false>(a, mt, st);
    return gather ? launch_gemm<BF16, 64, 1, false, true, false>(a, mt, st)
                  : launch_gemm<BF16, 64, 1, false, false, false>(a, mt, st);
  }
  if (swiglu)
    return gather ? launch_gemm<BF16, 128, 2, true, true, false>(a, mt, st)
                  : launch_gemm<BF16, 128, 2, true, false, false>(a, mt, st);
  return gather ? launch_gemm<BF16, 128, 2, false, true, false>(a, mt, st)
                : launch_gemm<BF16, 128, 2, false, false, false>(a, mt, st);
}

int w8a16_gemv_dense(const void *x, const int8_t *q, const float *s, void *y, int64_t m,
                     int64_t n, int64_t k, int dtype, hipStream_t st);

}  // namespace lm

using namespace lm;

extern "C" int lm_w8a16_linear(const void *x, const int8_t *q, const float *s, void *y, int64_t m,
                               int64_t n, int64_t k, int dtype, int large_tile, void *stream) {
  LM_REQUIRE(dtype == LM_BF16 || dtype == LM_FP16, LM_EINVAL,
             "W8A16 requires CUDA FP16/BF16 activations");
  LM_REQUIRE(k > 0 && k % 128 == 0 && n > 0 && m >= 0 && n < (1LL << 31), LM_EINVAL,
             "Invalid INT8 group geometry");
  if (m == 0) return LM_OK;
  LM_REQUIRE(x && q && s && y, LM_EINVAL, "null pointer");
  if (m <= 8) return w8a16_gemv_dense(x, q, s, y, m, n, k, dtype, as_stream(stream));
  LM_REQUIRE(m < (1LL << 31) / 1, LM_EINVAL, "Invalid INT8 group geometry");
  return w8a16_gemm_dense(x, q, s, y, m, n, k, dtype, large_tile, as_stream(stream));
}

static int check_routed(const void *x, const int8_t *q, const float *s, const int64_t *table,
                        int64_t n_tiles, int64_t bm, void *y, int64_t n, int64_t k) {
  LM_REQUIRE(k > 0 && k % 128 == 0 && n > 0 && n < (1LL << 30), LM_EINVAL,
             "Invalid INT8 group geometry");
  LM_REQUIRE(bm >= 1 && bm <= 128, LM_EINVAL, "tile height must be in 1..128");
  LM_REQUIRE(n_tiles >= 0 && n_tiles < 65536, LM_EINVAL, "too many tiles");
  LM_REQUIRE(n_tiles == 0 || (x && q && s && table && y), LM_EINVAL, "null pointer");
  return LM_OK;
}

extern "C" int lm_routed_gemm_w8a16(const void *x, const int8_t *q, const float *s,
                                    const int64_t *pos, const int64_t *table, int64_t n_tiles,
                                    int64_t bm, void *y, int64_t n, int64_t k, int gather,
                                    int64_t q_expert_stride, int64_t s_expert_stride,
                                    void *stream) {
  if (int rc = check_routed(x, q, s, table, n_tiles, bm, y, n, k)) return rc;
  LM_REQUIRE(!gather || pos || n_tiles == 0, LM_EINVAL, "gather needs pos");
  return routed_gemm(x, q, s, pos, table, n_tiles, bm, y, n, k, gather != 0, false,
                     q_expert_stride, s_expert_stride, k, as_stream(stream));
}

extern "C" int lm_routed_gate_up_swiglu(const void *x, const int8_t *q, const float *s,
                                        const int64_t *pos, const int64_t *table,
                                        int64_t n_tiles, int64_t bm, void *h, int64_t n, int64_t k,
                                        int64_t q_expert_stride, int64_t s_expert_stride,
                                        void *stream) {
  if (int rc = check_routed(x, q, s, table, n_tiles, bm, h, n, k)) return rc;
  LM_REQUIRE(n % 2 == 0, LM_EINVAL, "gate_up needs an even number of rows");
  LM_REQUIRE(pos || n_tiles == 0, LM_EINVAL, "gather needs pos");
  return routed_gemm(x, q, s, pos, table, n_tiles, bm, h, n, k, true, true, q_expert_stride,
                     s_expert_stride, k, as_stream(stream));
}
