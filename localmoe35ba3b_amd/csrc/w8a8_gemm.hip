// W8A8 MFMA GEMM for more than 8 rows (gfx950, v_mfma_i32_16x16x64_i8).
//
//   y[m, n] = bf16(acc),  acc = sum over 128-wide K groups g, ascending, of
//             (f32(p[m, n, g]) * xs[m, g]) * s[n, g],
//   p[m, n, g] = sum_{k in g} xq[m, k] * q[n, k]            (int32, exact)
//
// on rows already quantized by lm_act_quant_g128 (w8a8.py:8-22).  This is
// w8a8._linear (w8a8.py:25-41) for every row of x rather than row 0 only: the
// int8 tl.dot of a group becomes int32 MFMAs (|p| <= 127 * 127 * 128 < 2^24,
// so the partial and its conversion to fp32 are exact), and after each group
// the epilogue runs in the reference's order without fused operations (the
// library is compiled with -ffp-contract=off), so every fp32 accumulator, and
// therefore its bf16 rounding, is bit-identical to the reference's.
//
// Tile: 128 rows x 128 columns per workgroup of four waves (2 x 2, 64 x 64
// each); one K group (128 bytes of every A row and B row) per stage, staged in
// LDS with a 16-byte row pad and prefetched into registers one group ahead.
// Within a 16x16x64 MFMA a lane holds row (lane & 15) and 16 consecutive K
// bytes at offset 16 (lane >> 4) of the 64-K step, for A and B alike; the
// order of K inside the sum does not matter because the int32 sum is exact.
// The per-group epilogue (four fp32 operations per output element) costs
// about as much issue time as the group's MFMAs, so the kernel's ceiling is
// below the int8 MFMA peak by that ratio.
//
// SwiGLU mode reads the n weight rows as [gate; up] halves: a tile's columns
// pair gate column j with its up partner half + j in the same lane, and the
// epilogue writes h = bf16(bf16(silu(bf16(gate))) * bf16(up)) (int8.py:182-184).
#include "internal.hpp"

namespace lm {
namespace {

constexpr int kQBM = 128;  // tile rows
constexpr int kQBN = 128;  // tile columns
constexpr int kQOcc = 2;   // workgroups per CU the register budget targets
constexpr int kQG = 128;         // K group
constexpr int kQPitch = kQG + 16;  // LDS bytes per staged row

typedef int i32x4 __attribute__((ext_vector_type(4)));

struct W8A8GemmArgs {
  const int8_t *xq;
  const float *xs;
  const int8_t *q;
  const float *s;
  uint16_t *y;
  int64_t M;
  int N, K, ldy;
  int nt_count, mt_count;
};

template <typename T, bool SWIGLU, int BN, int OCC>
__global__ __launch_bounds__(256, OCC) void w8a8_mfma_kernel(W8A8GemmArgs a) {
  constexpr int MI = 4, NI = BN / 32;  // 16x16 sub-tiles per wave (64 x BN/2)
  constexpr int BCH = BN / 32;         // 16-byte B chunks per thread per group
  __shared__ __align__(16) int8_t As[kQBM * kQPitch];
  __shared__ __align__(16) int8_t Bs[BN * kQPitch];
  __shared__ float xsl[kQBM];
  __shared__ float wsl[BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // All column tiles of one row tile run back to back on one XCD (linear id
  // b is dealt to XCD b % 8), so the row tile's activations stay in its L2.
  const int b = blockIdx.x;
  const int j = b >> 3;
  const int mt = (j / a.nt_count) * 8 + (b & 7);
  const int nt = j % a.nt_count;
  if (mt >= a.mt_count) return;

  const int64_t m0 = (int64_t)mt * kQBM;
  const int rows = (int)min((int64_t)kQBM, a.M - m0);
  const int K = a.K;
  const int G = K / kQG;
  const int half = a.N >> 1;
  const int n0 = SWIGLU ? nt * (BN / 2) : nt * BN;

  auto wrow = [&](int c) -> int {  // tile column -> weight row, -1 past the end
    if constexpr (SWIGLU) {
      const int jj = n0 + (c & (BN / 2 - 1));
      if (jj >= half) return -1;
      return c < BN / 2 ? jj : half + jj;
    } else {
      const int jj = n0 + c;
      return jj < a.N ? jj : -1;
    }
  };
  auto col_base = [&](int ni) -> int {
    if constexpr (SWIGLU) {
      return ni < NI / 2 ? wn * (BN / 4) + ni * 16 : BN / 2 + wn * (BN / 4) + (ni - NI / 2) * 16;
    } else {
      return wn * (BN / 2) + ni * 16;
    }
  };

  // Per-thread sources of one group: 16-byte chunk c = tid + 256 i of the
  // 128-byte rows of the A and B tiles (row c / 8, chunk c % 8).  Rows past M
  // and columns past N re-read row 0 of the tile / weight row 0 and are never
  // stored.
  const int8_t *asrc[4];
  const int8_t *bsrc[BCH];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i;
    const int r = c >> 3;
    asrc[i] = a.xq + (m0 + (r < rows ? r : 0)) * K + (c & 7) * 16;
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int c = tid + 256 * i;
    const int wr = wrow(c >> 3);
    bsrc[i] = a.q + (int64_t)(wr >= 0 ? wr : 0) * K + (c & 7) * 16;
  }
  // thread t < 128 carries the scale of tile row t, 128 <= t < 128 + BN that
  // of column t - 128
  const float *ssrc = nullptr;
  if (tid < kQBM) {
    ssrc = a.xs + (m0 + (tid < rows ? tid : 0)) * G;
  } else if (tid < kQBM + BN) {
    const int wr = wrow(tid - kQBM);
    ssrc = a.s + (int64_t)(wr >= 0 ? wr : 0) * G;
  }

  u32x4 areg[4], breg[BCH];
  float sreg = 0.0f;
  auto prefetch = [&](int g) {
    const int k0 = g * kQG;
#pragma unroll
    for (int i = 0; i < 4; ++i) areg[i] = ldg16(asrc[i] + k0);
#pragma unroll
    for (int i = 0; i < BCH; ++i) breg[i] = ldg16(bsrc[i] + k0);
    if (ssrc) sreg = ssrc[g];
  };

  f32x4 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  prefetch(0);
  for (int g = 0; g < G; ++g) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&As[(c >> 3) * kQPitch + (c & 7) * 16]) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&Bs[(c >> 3) * kQPitch + (c & 7) * 16]) = breg[i];
    }
    if (tid < kQBM)
      xsl[tid] = sreg;
    else if (tid < kQBM + BN)
      wsl[tid - kQBM] = sreg;
    __syncthreads();
    if (g + 1 < G) prefetch(g + 1);

    i32x4 p[MI][NI];
#pragma unroll
    for (int ks = 0; ks < kQG / 64; ++ks) {
      const int kk = ks * 64 + (lane >> 4) * 16;
      i32x4 af[MI], bfr[NI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        af[mi] = *reinterpret_cast<const i32x4 *>(
            &As[(wm * 64 + mi * 16 + (lane & 15)) * kQPitch + kk]);
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bfr[ni] = *reinterpret_cast<const i32x4 *>(&Bs[(col_base(ni) + (lane & 15)) * kQPitch + kk]);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          p[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
              af[mi], bfr[ni], ks == 0 ? i32x4{0, 0, 0, 0} : p[mi][ni], 0, 0, 0);
    }
    // acc = acc + (f32(p) * xs) * ws, each operation rounded (w8a8.py:40).
    // MFMA 16x16 layout: lane holds column (lane & 15), rows 4 (lane >> 4) + it.
    float wv[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) wv[ni] = wsl[col_base(ni) + (lane & 15)];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const float xv = xsl[wm * 64 + mi * 16 + (lane >> 4) * 4 + it];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni][it] = add_rn(acc[mi][ni][it], mul_rn(mul_rn((float)p[mi][ni][it], xv), wv[ni]));
      }
    }
  }

#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int rl = wm * 64 + mi * 16 + (lane >> 4) * 4 + it;
      if (rl >= rows) continue;
      uint16_t *yrow = a.y + (m0 + rl) * a.ldy;
      if constexpr (SWIGLU) {
#pragma unroll
        for (int ni = 0; ni < NI / 2; ++ni) {
          const int col = n0 + wn * (BN / 4) + ni * 16 + (lane & 15);
          if (col < half) {
            const float gate = T::round(acc[mi][ni][it]);
            const float up = T::round(acc[mi][ni + NI / 2][it]);
            yrow[col] = T::from_f32(T::round(silu_f32(gate)) * up);
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

}  // namespace
}  // namespace lm

using namespace lm;

extern "C" int lm_w8a8_gemm(const int8_t *xq, const float *xs, const int8_t *q, const float *s,
                            void *y, int64_t m, int64_t n, int64_t k, int swiglu, int y_dtype,
                            void *stream) {
  LM_REQUIRE(y_dtype == LM_BF16 || y_dtype == LM_FP16, LM_EINVAL,
             "W8A8 output must be bf16 or fp16");
  LM_REQUIRE(m >= 0 && m <= (int64_t(1) << 31) / 128, LM_EINVAL, "invalid row count");
  LM_REQUIRE(n > 0 && n <= (1 << 24) && k > 0 && k % 128 == 0 && k <= 65536, LM_EINVAL,
             "Invalid INT8 group geometry");
  LM_REQUIRE(!swiglu || n % 2 == 0, LM_EINVAL, "SwiGLU needs an even number of rows");
  if (m == 0) return LM_OK;
  LM_REQUIRE(xq && xs && q && s && y, LM_EINVAL, "null pointer");
  W8A8GemmArgs a{};
  a.xq = xq;
  a.xs = xs;
  a.q = q;
  a.s = s;
  a.y = static_cast<uint16_t *>(y);
  a.M = m;
  a.N = (int)n;
  a.K = (int)k;
  a.ldy = (int)(swiglu ? n / 2 : n);
  a.nt_count = (int)(swiglu ? cdiv(n / 2, kQBN / 2) : cdiv(n, kQBN));
  a.mt_count = (int)cdiv(m, kQBM);
  const int64_t grid = 8 * (int64_t)a.nt_count * ((a.mt_count + 7) / 8);
  LM_REQUIRE(grid < (int64_t(1) << 31), LM_EINVAL, "problem too large for one launch");
  hipStream_t st = as_stream(stream);
  const bool bf = y_dtype == LM_BF16;
  if (swiglu) {
    if (bf) w8a8_mfma_kernel<BF16, true, kQBN, kQOcc><<<(unsigned)grid, 256, 0, st>>>(a);
    else w8a8_mfma_kernel<FP16, true, kQBN, kQOcc><<<(unsigned)grid, 256, 0, st>>>(a);
  } else {
    if (bf) w8a8_mfma_kernel<BF16, false, kQBN, kQOcc><<<(unsigned)grid, 256, 0, st>>>(a);
    else w8a8_mfma_kernel<FP16, false, kQBN, kQOcc><<<(unsigned)grid, 256, 0, st>>>(a);
  }
  return check_launch("w8a8_mfma_kernel");
}
