// W8A16 MFMA GEMMs for prefill (gfx950, v_mfma_f32_16x16x32_{bf16,f16}).
//
// Used three ways:
//   dense   y = x . dequant(q)^T                 lm_w8a16_linear, m > 8 (int8.py:9-37)
//   routed  per tile (e, start, stop) of a route-plan table, rows gathered
//           through pos (gate_up) or contiguous (down)   (prefill.py:12-34)
//   swiglu  the gate_up variant with bf16(bf16(silu(gate)) * up) fused in the
//           epilogue                                     (prefill.py:75-78)
//
// Every kernel dequantizes each int8 weight to T(q * s) exactly before the
// MFMA (the reference rounds the dequantized weight to the activation dtype
// before the MMA, int8.py:21), so the MFMA consumes bit-identical operands
// to the reference's tl.dot; only the fp32 summation order differs.
//   w8a16_mfma_kernel    dense and generic (fp16 rows, other K): 256 threads,
//                        BM x 128 tile, K in 64-wide stages, weights
//                        dequantized into LDS.
//   grouped_mfma_kernel  routed, any K, up to 128-row tiles (large_tile).
//   grouped_rb_kernel    routed, and dense bf16, at the model's K (2048
//                        gate_up, 512 down) in tiles of up to 96 rows:
//                        weights streamed straight into registers and
//                        dequantized there.
// In SwiGLU mode a tile's columns pair every gate column with its up partner
// in the same lane.
#include <type_traits>

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
  // bounds of the routed mode: table experts are clamped into [0, experts),
  // starts and stops into [0, y_rows], gathered row indices into [0, x_rows)
  int64_t experts;
  int64_t y_rows;
  int64_t x_rows;
  const int8_t *q;
  int64_t q_es;
  const int8_t *q_tiles;  // q in the 16-row tile layout (weight load modes kWlTiles*)
  const int *x_exp;       // kWlTilesF16: x row r holds fp16(x_r * 2^x_exp[r])
  const int *ptile;       // gathered tile GEMMs: x row of tile row r of table row i at i * tile_rows + r
  const float *s;
  int64_t s_es;
  uint16_t *y;
  int64_t ldy;
  int N;
  int K;
  int tile_rows;  // rows covered by one table tile (<= BM)
  int nt_count;   // column tiles
  int mt_count;   // row tiles (table rows, or dense M tiles)
};

// Workgroups are dealt to the 8 XCDs round-robin by linear id.  Map linear
// id b -> (row tile, column tile) so that all column tiles of one row tile
// run on the same XCD back to back: the gathered activation rows of a tile
// are then read from HBM/MALL once and served from that XCD's L2 for the
// other column tiles.  Returns false for padding workgroups.
__device__ __forceinline__ bool xcd_tile(const GemmArgs &a, int &mt, int &nt) {
  const int b = blockIdx.x;
  const int j = b >> 3;
  mt = (j / a.nt_count) * 8 + (b & 7);
  nt = j % a.nt_count;
  return mt < a.mt_count;
}

// Workgroups of an XCD-mapped launch; callers reject counts beyond one
// launch's grid (2^31 - 1) before launching.
static int64_t xcd_grid(int64_t mtiles, int64_t ntiles) {
  return 8 * ntiles * ((mtiles + 7) / 8);
}

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
  int mt, nt;
  if (!xcd_tile(a, mt, nt)) return;

  int64_t e = 0, start;
  int rows;
  if constexpr (DENSE) {
    start = (int64_t)mt * BM;
    rows = (int)min((int64_t)BM, a.M - start);
  } else {
    const TileBounds tb = tile_bounds(a.table[mt * 3], a.table[mt * 3 + 1], a.table[mt * 3 + 2],
                                      a.experts, a.y_rows, a.tile_rows);
    if (tb.rows <= 0) return;
    e = tb.expert;
    start = tb.start;
    rows = tb.rows;
  }
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
    const int64_t xr = GATHER ? clamp_index(a.pos[start + r], a.x_rows) : start + r;
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

// Routed grouped GEMM (prefill MoE shape: ~64 routes per expert, up to 128
// rows per tile so one tile covers a whole expert and its weights are read
// and dequantized once).  Row sub-tiles of 16 beyond the tile's routes are
// skipped entirely (no loads, no MFMA), so an expert with 70 routes costs
// 80 rows of MFMA work.  The four waves split the BN columns; each wave keeps
// its own int8 B fragments in LDS and dequantizes them exactly (T(q * s)) right
// before the MFMA, once per workgroup per weight.  A and B of the next stage
// are prefetched into registers while the current stage computes.
constexpr int kGBM = 128;
constexpr int kLDB = kBK + 8;  // int8 bytes per LDS row of the weight tile

// Eight int8 weights -> eight T(q * s): the signed byte converts exactly
// (v_cvt_f32_i32 with a sign-extended byte operand), so q * s is the
// correctly rounded fp32 product, then RNE to T - bit-identical to
// dequant8 with one operation fewer per four weights.
template <typename T>
__device__ __forceinline__ u32x4 dequant8s(uint2 w, float s) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = (float)(int8_t)(w.x >> (8 * i)) * s;
    f[4 + i] = (float)(int8_t)(w.y >> (8 * i)) * s;
  }
  return u32x4{T::pack2(f[0], f[1]), T::pack2(f[2], f[3]), T::pack2(f[4], f[5]),
               T::pack2(f[6], f[7])};
}

// Eight weights of the LM_TILES_F16 format (bytes u = q + 128, each dword
// holding k = 0, 2, 1, 3 in byte order) -> eight fp16 values q, exactly, in k
// order.  A byte placed under the fp16 exponent of 1024 is the value 1024 + u
// (one v_bitop3 (S0 & S1) | S2 for k = 0, 1, one byte permute for k = 2, 3);
// subtracting 1152 leaves q.  Four VALU operations per four weights, against
// eleven for the exact bf16(q * s).
__device__ __forceinline__ u32x4 dequant8_f16(uint2 w) {
  constexpr unsigned kAndOr = (0xF0u & 0xCCu) | 0xAAu;  // bitop3 table of (S0 & S1) | S2
  const f16x2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  auto sub = [&](uint32_t m) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, m) + bias);
  };
  return u32x4{sub(__builtin_amdgcn_bitop3_b32(w.x, 0x00FF00FFu, 0x64006400u, kAndOr)),
               sub(__builtin_amdgcn_perm(0x64646464u, w.x, 0x07030701u)),
               sub(__builtin_amdgcn_bitop3_b32(w.y, 0x00FF00FFu, 0x64006400u, kAndOr)),
               sub(__builtin_amdgcn_perm(0x64646464u, w.y, 0x07030701u))};
}

// SiLU for the prefill epilogue from the hardware exp2 and reciprocal
// (about 2 ulp in fp32); the product is rounded to bf16 right after.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

template <typename T>
__device__ __forceinline__ u32x4 dequant8(uint2 w, float s) {
  const float n = -128.0f * s;
  float f[8];
  dequant4(w.x, s, n, f);
  dequant4(w.y, s, n, f + 4);
  return u32x4{T::pack2(f[0], f[1]), T::pack2(f[2], f[3]), T::pack2(f[4], f[5]),
               T::pack2(f[6], f[7])};
}

template <typename T, bool SWIGLU, bool GATHER, int BN>
__global__ __launch_bounds__(256) void grouped_mfma_kernel(GemmArgs a) {
  constexpr int TN = BN / 4;       // columns per wave
  constexpr int MI = kGBM / 16;    // row sub-tiles
  constexpr int NI = TN / 16;      // column sub-tiles per wave
  constexpr int ACH = kGBM * 8 / 256;  // 16-byte A chunks per thread per stage
  constexpr int BCH = BN * 4 / 256;    // 16-byte B chunks per thread per stage
  __shared__ __align__(16) uint16_t As[kGBM * kLDA];
  __shared__ __align__(16) int8_t Bs[BN * kLDB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wn = tid >> 6;
  int mt, nt;
  if (!xcd_tile(a, mt, nt)) return;
  const TileBounds tb = tile_bounds(a.table[mt * 3], a.table[mt * 3 + 1], a.table[mt * 3 + 2],
                                    a.experts, a.y_rows, a.tile_rows);
  if (tb.rows <= 0) return;
  const int64_t e = tb.expert;
  const int64_t start = tb.start;
  const int rows = tb.rows;
  const int msub = (rows + 15) >> 4;  // live row sub-tiles
  const int8_t *wq = a.q + e * a.q_es;
  const float *wsc = a.s + e * a.s_es;
  const int K = a.K;
  const int G = K >> 7;
  const int half = a.N >> 1;
  const int n0 = SWIGLU ? nt * (BN / 2) : nt * BN;

  auto wrow = [&](int c) -> int {
    if constexpr (SWIGLU) {
      const int j = n0 + (c & (BN / 2 - 1));
      if (j >= half) return -1;
      return c < BN / 2 ? j : half + j;
    } else {
      const int j = n0 + c;
      return j < a.N ? j : -1;
    }
  };
  auto col_base = [&](int ni) -> int {
    if constexpr (SWIGLU) {
      return ni < NI / 2 ? wn * (TN / 2) + ni * 16 : BN / 2 + wn * (TN / 2) + (ni - NI / 2) * 16;
    } else {
      return wn * TN + ni * 16;
    }
  };

  const uint16_t *asrc[ACH];
  bool aok[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + 256 * i;
    const int r = c >> 3;
    aok[i] = r < rows;
    const int64_t xr = aok[i] ? (GATHER ? clamp_index(a.pos[start + r], a.x_rows) : start + r) : 0;
    asrc[i] = a.x + xr * a.ldx + (c & 7) * 8;
  }
  const int8_t *bsrc[BCH];
  bool bok[BCH];
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int c = tid + 256 * i;
    const int wr = wrow(c >> 2);
    bok[i] = wr >= 0;
    bsrc[i] = wq + (int64_t)(bok[i] ? wr : 0) * K + (c & 3) * 16;
  }
  const float *ssrc[NI];
  bool sok[NI];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int wr = wrow(col_base(ni) + (lane & 15));
    sok[ni] = wr >= 0;
    ssrc[ni] = wsc + (int64_t)(sok[ni] ? wr : 0) * G;
  }

  u32x4 ra[ACH], rb[BCH];
  float rs[NI];
  auto prefetch = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < ACH; ++i) ra[i] = aok[i] ? ldg16(asrc[i] + k0) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < BCH; ++i) rb[i] = bok[i] ? ldg16(bsrc[i] + k0) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) rs[ni] = sok[ni] ? ssrc[ni][k0 >> 7] : 0.0f;
  };

  f32x4 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / kBK;
  prefetch(0);
  for (int kt = 0; kt < KT; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      if (aok[i]) *reinterpret_cast<u32x4 *>(&As[(c >> 3) * kLDA + (c & 7) * 8]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i;
      int8_t *bd = &Bs[(c >> 2) * kLDB + (c & 3) * 16];
      *reinterpret_cast<uint2 *>(bd) = uint2{rb[i][0], rb[i][1]};
      *reinterpret_cast<uint2 *>(bd + 8) = uint2{rb[i][2], rb[i][3]};
    }
    float sc[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) sc[ni] = rs[ni];
    __syncthreads();
    if (kt + 1 < KT) prefetch(kt + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      const int kk = ks * 32 + (lane >> 4) * 8;
      u32x4 bfr[NI];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        bfr[ni] = dequant8<T>(
            *reinterpret_cast<const uint2 *>(&Bs[(col_base(ni) + (lane & 15)) * kLDB + kk]),
            sc[ni]);
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        if (mi < msub) {
          const u32x4 af =
              *reinterpret_cast<const u32x4 *>(&As[(mi * 16 + (lane & 15)) * kLDA + kk]);
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            acc[mi][ni] = T::mfma16x16x32(af, bfr[ni], acc[mi][ni]);
        }
      }
    }
  }

#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    if (mi >= msub) continue;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int rl = mi * 16 + (lane >> 4) * 4 + it;
      if (rl >= rows) continue;
      uint16_t *yrow = a.y + (start + rl) * a.ldy;
      if constexpr (SWIGLU) {
#pragma unroll
        for (int ni = 0; ni < NI / 2; ++ni) {
          const int col = n0 + wn * (TN / 2) + ni * 16 + (lane & 15);
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

// Workgroup barrier without the release/acquire fences of __syncthreads():
// those would make every wave wait for all of its outstanding global loads.
// Callers wait for exactly what they need first (the LDS writes); the memory
// clobber keeps the compiler from moving LDS accesses across.
__device__ __forceinline__ void barrier_raw() { asm volatile("s_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------
// Register-streamed variant: the int8 weights never touch LDS.  Each wave
// owns TN columns of the tile and streams its own weight rows straight into
// registers, BD stages deep (BD - 1 stages of 64 K in flight while one is
// consumed), dequantizes them exactly in registers and feeds them to the
// MFMA as the B operand.  Only the activation rows (shared by the four
// waves) are staged in LDS, in a 3-slot ring loaded through registers one
// stage ahead of their LDS write.  All loads are ordinary compiler-tracked
// loads, so every wait the compiler inserts is exact.  Within a stage the
// next 8-K piece is dequantized while the MFMAs of the current one run (the
// two are independent, and the compiler interleaves them), so a wave keeps
// the matrix pipe and the VALU busy together.
//
// K order inside a 64-K stage: in the MFMA layout lane l (quarter q = l >> 4)
// holds 16 consecutive weights k = 16 q .. 16 q + 15 of column l & 15; MFMA
// step `sub` takes the half 8 sub .. 8 sub + 7.  The A fragment of the same
// lane and step reads the same k from LDS, so each product pairs the right x
// and w (a fixed permutation of the summation order inside the stage).
//
// Weight load modes (WL):
//   kWlDirect  dense weights, which every row tile re-reads from cache: each
//              lane loads its MFMA operand piece directly (a quarter-wave
//              touches 16 rows 2 KB apart);
//   kWlPermute streamed (routed) weights in the standard layout: quarter-wave
//              a loads 64 contiguous bytes of each of rows 4 a .. 4 a + 3
//              (lane 16 a + 4 b + p: row 4 a + b, piece p), 4 lines per
//              quarter-wave instead of 16, and one ds_bpermute per dword
//              moves piece p of row r to lane 16 p + r while the previous
//              stage's MFMAs run;
//   kWlTiles   streamed weights in the 16-row tile layout (lm_w8_tile_rows):
//              a wave's load of one 16-row x 64-K block is 1 KB contiguous
//              and lands in the MFMA layout, no permute.
//   kWlTilesF16  the tile layout in its fp16 format (LM_TILES_F16) on fp16
//              activation rows x_r = fp16(row r * 2^x_exp[r]) (exact for the
//              bf16 values of a normalized row down to 2^-31 of its norm): the
//              MFMAs multiply exact fp16 q by the exact rows in fp16 with
//              fp32 accumulation, and the group scales act on the
//              accumulators.  Before the first MFMA of group g each
//              accumulator of column n is multiplied by s[n, g-1] / s[n, g],
//              so it always holds sum_{g' <= g} s[n, g'] P_g' / s[n, g]; the
//              epilogue multiplies by s[n, G-1] and 2^-x_exp[r].  The
//              accumulator of a tile was last written 16 MFMAs earlier, so
//              the multiply waits for nothing.  Scales are clamped into
//              [2^-40, 2^40] for the ratios (a clamped group contributes at
//              most 2^-40 |P| instead of nothing).  Unlike the bf16 path this
//              does not round q * s to bf16 before the products.
constexpr int kWlDirect = 0, kWlPermute = 1, kWlTiles = 2, kWlTilesF16 = 3;
//
// A stage in LDS: BM rows x 128 B (64 bf16); 16-byte chunk p of row r is
// stored at chunk p ^ rb_swz(r).  Scales of the tile are staged once,
// transposed: [K / 128][BN cols] floats.
constexpr int rb_gcd(int a, int b) { return b == 0 ? a : rb_gcd(b, a % b); }

// LDS chunk swizzle of activation row r (16-byte chunks, XOR on the low
// three chunk bits).  Rows r and r + 8 read by one 16-lane phase share
// (r & 7); folding in bit 3 of r puts them on different chunks, so the 16
// rows of an A fragment hit 16 different bank groups.
__device__ __forceinline__ int rb_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// One tile with MS live 16-row sub-tiles (rows <= 16 MS).  Instantiated per
// MS so the inner loop carries no row branches; every load is unconditional
// (rows past the tile re-read its last row), which keeps the compiler's
// wait counts exact.  A stage is KS = 64 HL values of K: each lane loads HL
// 16-byte pieces per column sub-tile (bytes 64 h + 16 p, h < HL), so four
// consecutive lanes read 64 contiguous bytes of a weight row.  Weights are
// requested BD - 1 stages ahead, activation rows AD stages ahead (AD - 1
// stages wait in registers, one more in LDS).
template <typename T, bool SWIGLU, bool GATHER, int WL, int K, int BM, int TN, int BD, int HL, int AD,
          int NW, int MS>
__device__ __forceinline__ void rb_tile(const GemmArgs &a, int64_t e, int64_t start, int rows,
                                        int nt, unsigned char *smem, const int *gx, int gk) {
  constexpr int KS = 64 * HL;
  constexpr int KT = K / KS;
  constexpr int G = K / 128;
  constexpr int BN = NW * TN;
  constexpr int NT = NW * 64;              // threads
  constexpr int NI = TN / 16;
  constexpr int AR = 3;
  constexpr int AS = AD - 1;               // activation stages held in registers
  constexpr int ROWB = KS * 2;             // LDS bytes per activation row per stage
  constexpr int CPR = ROWB / 16;           // 16-byte chunks per row
  constexpr int RPL = 1024 / ROWB;         // rows per 1 KB wave-load
  constexpr int A_STAGE = BM * ROWB;
  constexpr int A_W = (MS * 16 / RPL + NW - 1) / NW;  // wave-loads per wave covering 16 MS rows
  constexpr int SC_P = BN * G / 4;            // 16-byte scale pieces of the tile
  constexpr int SC_W = (SC_P + NT - 1) / NT;
  constexpr int U0 = BD / rb_gcd(BD, AS) * AS;  // unroll: both ring indices static
  constexpr int GS = 128 / KS;                   // stages per scale group
  // kWlTilesF16 also needs the group boundaries static in the unrolled loop
  constexpr int U = WL == kWlTilesF16 && U0 % GS ? U0 * GS / rb_gcd(U0, GS) : U0;
  static_assert(MS * 16 <= BM && BD >= 2 && AD >= 2 && NW * A_W * RPL <= BM, "shape");
  constexpr bool F16 = WL == kWlTilesF16;
  constexpr bool TILES = WL == kWlTiles || F16;
  using MT = typename std::conditional<F16, FP16, T>::type;  // MFMA operand type
  static_assert(!F16 || G % 4 == 0, "fp16 tiles: whole 16-byte scale pieces per column");
  // [G][BN] fp32 scales, or (kWlTilesF16) the ratios s[g-1] / s[g] (1 at
  // g = 0); then (kWlTilesF16) s[G-1] per column and the x_exp of each row
  float *scl = reinterpret_cast<float *>(smem + AR * A_STAGE);
  float *slast = scl + G * BN;
  int *rowk = reinterpret_cast<int *>(slast + BN);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4;
  const int8_t *wq = a.q + e * a.q_es;
  const float *wsc = a.s + e * a.s_es;
  const int half = a.N >> 1;
  const int n0 = SWIGLU ? nt * (BN / 2) : nt * BN;

  auto wrow = [&](int c) -> int {  // tile column -> weight row, -1 past the end
    if constexpr (SWIGLU) {
      const int j = n0 + (c & (BN / 2 - 1));
      if (j >= half) return -1;
      return c < BN / 2 ? j : half + j;
    } else {
      const int j = n0 + c;
      return j < a.N ? j : -1;
    }
  };
  auto col_base = [&](int ni) -> int {
    if constexpr (SWIGLU) {
      return ni < NI / 2 ? wave * (TN / 2) + ni * 16
                         : BN / 2 + wave * (TN / 2) + (ni - NI / 2) * 16;
    } else {
      return wave * TN + ni * 16;
    }
  };

  // Scales of the tile (16-byte piece p: column p / (G/4), groups 4 (p % (G/4)) ..),
  // requested first; written to LDS transposed ([group][column], so a wave's
  // 16 column lanes read consecutive words) once the first stages are in flight.
  u32x4 sreg[SC_W];
#pragma unroll
  for (int j = 0; j < SC_W; ++j) {
    const int piece = (tid + NT * j) % SC_P;
    const int wr = wrow(piece / (G / 4));
    sreg[j] = ldg16(wsc + (int64_t)(wr >= 0 ? wr : 0) * G + (piece % (G / 4)) * 4);
  }
  // Weight sources of column sub-tile ni (16 weight rows from a multiple of
  // 16), stage 0.  kWlDirect: lane l loads column col_base(ni) + (l & 15),
  // bytes 16 q (+ 64 h).  kWlPermute: lane 16 a + 4 b + p loads column
  // col_base(ni) + 4 a + b, bytes 16 p, and rb_perm moves them into the MFMA
  // layout.  kWlTiles: the sub-tile's 1 KB tile of each 64-K block, byte 16 l.
  const int8_t *bsrc[NI];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    if constexpr (TILES) {
      const int wr = wrow(col_base(ni));
      bsrc[ni] = a.q_tiles + e * a.q_es + (int64_t)((wr >= 0 ? wr : 0) >> 4) * (K / 64) * 1024 +
                 lane * 16;
    } else {
      const int wr =
          wrow(col_base(ni) + (WL == kWlPermute ? 4 * q + ((lane & 15) >> 2) : lane & 15));
      bsrc[ni] = wq + (int64_t)(wr >= 0 ? wr : 0) * K + (WL == kWlPermute ? lane & 3 : q) * 16;
    }
  }
  // Activation sources: wave-load j fills rows RPL (4 j + wave) ..; lane ->
  // row RPL (4 j + wave) + lane / CPR, LDS chunk lane % CPR, which holds the
  // logical chunk (lane % CPR) ^ (row & 7).  Gathered rows on the tile
  // copies come from the tile-major map (gx, requested by the caller with
  // the table row), rows past the tile's end from x row 0; otherwise from
  // pos, rows past the end re-reading the tile's last row.
  constexpr bool PT = GATHER && TILES;
  const uint16_t *asrc[A_W];
#pragma unroll
  for (int j = 0; j < A_W; ++j) {
    const int r = RPL * (NW * j + wave) + lane / CPR;
    const int rr = min(r, rows - 1);
    const int64_t xr = GATHER ? clamp_index(PT ? (r < rows ? gx[j] : 0) : a.pos[start + rr], a.x_rows)
                              : start + rr;
    asrc[j] = a.x + xr * a.ldx + (((lane % CPR) ^ rb_swz(r)) * 8);
  }
  // kWlTilesF16: thread t < BM fetches the exponent of tile row t (consumed
  // in the epilogue; written to LDS before the last stage's barrier)
  int rk = 0;
  if constexpr (F16) {
    const int rr = min(tid, rows - 1);
    rk = a.x_exp[GATHER ? clamp_index(PT ? (tid < rows ? gk : 0) : a.pos[start + rr], a.x_rows)
                        : start + rr];
  }

  u32x4 breg[BD][NI][HL];
  u32x4 areg[AS][A_W];
  // Lane 16 p + r takes piece p of row r from lane 16 (r >> 2) + 4 (r & 3) + p
  // (a byte address for ds_bpermute).
  const int perm_src = 4 * (16 * ((lane & 15) >> 2) + 4 * (lane & 3) + q);
  auto rb_perm = [&](int slot) {
    if constexpr (WL == kWlPermute) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int h = 0; h < HL; ++h)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            breg[slot][ni][h][j] =
                (uint32_t)__builtin_amdgcn_ds_bpermute(perm_src, (int)breg[slot][ni][h][j]);
    }
  };
  // Tile-layout weights of a tile of at most 80 rows (MS < 6; a routed
  // expert's only tile, typically) are read by this tile alone: non-temporal
  // loads stream them past the caches, which both raises the read rate and
  // leaves the caches to the activation rows and the next kernel's inputs.
  // Fuller tiles (the shared expert's, a hot expert's) keep cached loads, as
  // other row tiles of the same expert re-read their weights.
  constexpr bool NTW = TILES && MS < 6;
  auto load_b = [&](int slot, int s) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int h = 0; h < HL; ++h) {
        const int8_t *p = bsrc[ni] + (TILES ? (s * HL + h) * 1024 : s * KS + 64 * h);
        breg[slot][ni][h] = NTW ? ldg16_nt(p) : ldg16(p);
      }
  };
  auto load_a = [&](int slot, int s) {
#pragma unroll
    for (int j = 0; j < A_W; ++j) areg[slot][j] = ldg16(asrc[j] + s * KS);
  };
  auto store_a = [&](int slot, int s) {
    unsigned char *base = smem + (s % AR) * A_STAGE;
#pragma unroll
    for (int j = 0; j < A_W; ++j)
      *reinterpret_cast<u32x4 *>(base + (NW * j + wave) * 1024 + lane * 16) = areg[slot][j];
  };

  f32x4 acc[MS][NI];
#pragma unroll
  for (int mi = 0; mi < MS; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: A(0) into LDS; A(1 .. AD-1) and B(0 .. BD-2) in flight.  All
  // of them are requested before the first wait, so the tile pays one load
  // latency before its first stage (A(0) goes through registers of its own).
  u32x4 a0[A_W];
#pragma unroll
  for (int j = 0; j < A_W; ++j) a0[j] = ldg16(asrc[j]);
#pragma unroll
  for (int s = 0; s < BD - 1; ++s) load_b(s, s);
#pragma unroll
  for (int s = 1; s < AD; ++s)
    if (s < KT) load_a(s % AS, s);
#pragma unroll
  for (int j = 0; j < SC_W; ++j) {
    const int piece = tid + NT * j;
    const int c = piece / (G / 4), g0 = 4 * (piece % (G / 4));
    if constexpr (F16) {
      // the column's pieces sit in consecutive lanes: group g0 - 1 is the
      // last of the previous lane's four
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sc[i] = fminf(fmaxf(__uint_as_float(sreg[j][i]), 0x1.0p-40f), 0x1.0p40f);
      const float prev = __shfl_up(sc[3], 1, 64);
      if (piece < SC_P) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          scl[(g0 + i) * BN + c] = g0 + i == 0 ? 1.0f : (i ? sc[i - 1] : prev) / sc[i];
        if (g0 + 4 == G) slast[c] = sc[3];
      }
    } else {
      if (piece < SC_P) {
#pragma unroll
        for (int i = 0; i < 4; ++i) scl[(g0 + i) * BN + c] = __uint_as_float(sreg[j][i]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < A_W; ++j)
    *reinterpret_cast<u32x4 *>(smem + (NW * j + wave) * 1024 + lane * 16) = a0[j];

  // Piece p of a stage (h = p / 2, sub = p % 2): 8 K per lane per column
  // sub-tile.  dq dequantizes one piece of stage s from weight slot ub.
  constexpr int P = 2 * HL;
  auto dq = [&](int ub, int s, int p, u32x4 *out) {
    const int g = (s * KS) >> 7;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const uint2 w{breg[ub][ni][p >> 1][2 * (p & 1)], breg[ub][ni][p >> 1][2 * (p & 1) + 1]};
      if constexpr (F16)
        out[ni] = dequant8_f16(w);
      else
        out[ni] = dequant8s<T>(w, scl[g * BN + col_base(ni) + (lane & 15)]);
    }
  };
  // The B operand of the piece being multiplied; the next piece (the first
  // piece of the next stage, after a stage's last) is dequantized while the
  // MFMAs of this one run.
  u32x4 bcur[NI];
  __builtin_amdgcn_s_waitcnt(0xC07F);
  barrier_raw();
  rb_perm(0);
  dq(0, 0, 0, bcur);
  // resc: stage s opens a scale group (kWlTilesF16 rescales the accumulators)
  auto step = [&](int s, int ub, int ua, bool st_a, bool ld_a, bool ld_b, bool has_next,
                  bool resc) {
    float rr[NI];
    if constexpr (F16) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        rr[ni] = resc ? scl[((s * KS) >> 7) * BN + col_base(ni) + (lane & 15)] : 1.0f;
    }
    if (st_a) store_a(ua, s + 1);
    if constexpr (F16) {
      if (!has_next && tid < BM) rowk[tid] = rk;  // read by the epilogue, after this barrier
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    barrier_raw();
    if (ld_a) load_a(ua, s + AD);
    if (ld_b) load_b((ub + BD - 1) % BD, s + BD - 1);
    __builtin_amdgcn_sched_barrier(0);
    const unsigned char *sa = smem + (s % AR) * A_STAGE;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      u32x4 af[MS];
#pragma unroll
      for (int mi = 0; mi < MS; ++mi) {
        const int r = mi * 16 + (lane & 15);
        af[mi] = *reinterpret_cast<const u32x4 *>(
            sa + r * ROWB + (((8 * (p >> 1) + 2 * q + (p & 1)) ^ rb_swz(r)) * 16));
      }
      const bool nxt = p + 1 < P || has_next;
      // The next stage's weights are moved into the MFMA layout during this
      // stage's first piece, one piece before their first dequantization.
      if (p == 0 && has_next) rb_perm((ub + 1) % BD);
      u32x4 bn[NI];
      if (p + 1 < P)
        dq(ub, s, p + 1, bn);
      else if (has_next)
        dq((ub + 1) % BD, s + 1, 0, bn);
#pragma unroll
      for (int mi = 0; mi < MS; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          if (F16 && resc && p == 0) acc[mi][ni] = acc[mi][ni] * rr[ni];
          acc[mi][ni] = MT::mfma16x16x32(af[mi], bcur[ni], acc[mi][ni]);
        }
      __builtin_amdgcn_sched_barrier(0);
      if (nxt) {
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) bcur[ni] = bn[ni];
      }
    }
  };
  // Main loop: every load in range.  The tail (TL >= max(BD - 1, AD) stages,
  // fully unrolled) issues only the loads that are still in range.
  constexpr int TLM = BD - 1 > AD ? BD - 1 : AD;
  constexpr int TL0 = KT % U;
  constexpr int TL = TL0 >= TLM ? TL0 : TL0 + U * ((TLM - TL0 + U - 1) / U);
  static_assert(TL <= KT, "stage count");
  for (int s0 = 0; s0 < KT - TL; s0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      step(s0 + u, u % BD, (u + 1) % AS, true, true, true, true, (u * KS) % 128 == 0);
  }
#pragma unroll
  for (int v = 0; v < TL; ++v) {
    const int s = KT - TL + v;
    step(s, s % BD, (s + 1) % AS, s + 1 < KT, s + AD < KT, s + BD - 1 < KT, s + 1 < KT,
         (s * KS) % 128 == 0);
  }

#pragma unroll
  for (int mi = 0; mi < MS; ++mi) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int rl = mi * 16 + q * 4 + it;
      if (rl >= rows) continue;
      uint16_t *yrow = a.y + (start + rl) * a.ldy;
      // kWlTilesF16: the last group's scale, then the row's power of two (exact)
      const int kr = F16 ? rowk[rl] : 0;
      auto val = [&](int ni) {
        return F16 ? ldexpf(acc[mi][ni][it] * slast[col_base(ni) + (lane & 15)], -kr)
                   : acc[mi][ni][it];
      };
      if constexpr (SWIGLU) {
#pragma unroll
        for (int ni = 0; ni < NI / 2; ++ni) {
          const int col = n0 + wave * (TN / 2) + ni * 16 + (lane & 15);
          if (col < half) {
            const float gate = T::round(val(ni));
            const float up = T::round(val(ni + NI / 2));
            yrow[col] = T::from_f32(T::round(silu_fast(gate)) * up);
          }
        }
      } else {
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          const int col = n0 + col_base(ni) + (lane & 15);
          if (col < a.N) yrow[col] = T::from_f32(val(ni));
        }
      }
    }
  }
}

template <typename T, bool SWIGLU, bool GATHER, int WL, int K, int BM, int TN, int BD, int HL,
          int AD, int NW, int OCC>
__global__ __launch_bounds__(NW * 64, OCC) void grouped_rb_kernel(GemmArgs a) {
  constexpr int SC_BYTES = NW * TN * (K / 128) * 4 + (WL == kWlTilesF16 ? (NW * TN + BM) * 4 : 0);
  __shared__ __align__(16) unsigned char smem[3 * BM * 128 * HL + SC_BYTES];
  int mt, nt;
  if (!xcd_tile(a, mt, nt)) return;
  // Gathered rows on the tile copies: this tile's rows of the tile-major
  // gather map, requested before the table row and independently of it
  // (the rows rb_tile assigns to this lane for the tallest tile, and to
  // thread t < BM for the row exponents), so the activation loads wait for
  // one dependent load instead of two.
  constexpr bool PT = GATHER && (WL == kWlTiles || WL == kWlTilesF16);
  constexpr int RPL = 8 / HL, CPR = 8 * HL;
  constexpr int AWM = (BM / RPL + NW - 1) / NW;
  static_assert(NW * AWM * RPL <= BM, "gather map rows inside the tile");
  int gx[AWM];
  int gk = 0;
#pragma unroll
  for (int j = 0; j < AWM; ++j) gx[j] = 0;
  if constexpr (PT) {
    const int *pt = a.ptile + (int64_t)mt * a.tile_rows;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < AWM; ++j) gx[j] = pt[RPL * (NW * j + wave) + lane / CPR];
    if constexpr (WL == kWlTilesF16) gk = pt[min((int)threadIdx.x, BM - 1)];
  }
  int64_t e = 0, start;
  int rows;
  if (a.table) {
    const TileBounds tb = tile_bounds(a.table[mt * 3], a.table[mt * 3 + 1], a.table[mt * 3 + 2],
                                      a.experts, a.y_rows, a.tile_rows);
    e = tb.expert;
    start = tb.start;
    rows = tb.rows;
  } else {  // dense: row tile mt of an [M, K] matrix
    start = (int64_t)mt * BM;
    rows = (int)min((int64_t)a.tile_rows, a.M - start);
  }
  if (rows <= 0) return;
  if constexpr (BM == 128) {  // dense rows at M >= kDenseTallM
    if (rows > 96)
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 8>(a, e, start, rows, nt, smem, gx, gk);
    else if (rows > 64)
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 6>(a, e, start, rows, nt, smem, gx, gk);
    else if (rows > 32)
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 4>(a, e, start, rows, nt, smem, gx, gk);
    else
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 2>(a, e, start, rows, nt, smem, gx, gk);
  } else {
    static_assert(BM == 96, "row-count dispatch below covers 96-row tiles");
    if (rows > 80)
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 6>(a, e, start, rows, nt, smem, gx, gk);
    else if (rows > 64)
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 5>(a, e, start, rows, nt, smem, gx, gk);
    else if (rows > 32)
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 4>(a, e, start, rows, nt, smem, gx, gk);
    else
      rb_tile<T, SWIGLU, GATHER, WL, K, BM, TN, BD, HL, AD, NW, 2>(a, e, start, rows, nt, smem, gx, gk);
  }
}

// Configuration of grouped_rb_kernel, chosen by measurement on the
// 2048-token prefill chunk: 4 waves of TN columns each, a 3-slot weight ring
// of one 64-K piece per stage, activations prefetched 2 stages ahead and a
// register budget for OCC workgroups per CU.  The routed GEMMs on the tile
// layout (kWlTiles) use 64 columns per wave at 2 workgroups per CU: a tile
// streams 512 KB of one expert's weights and its activation rows are re-read
// half as often as with 32 columns.  On the 40-layer stack, two chunks
// overlapped, that is 3 % more prefill tokens/s, though each GEMM alone is
// 1-2 % slower (and 8 % on a Zipf-skewed chunk, whose hot expert is compute
// bound at the lower occupancy).  Every other use keeps 32 columns at 3 per CU,
// except dense matrices of at least kDenseTallM rows: 128-row tiles, so each
// dequantized weight feeds 8 row sub-tiles instead of 6, with activations 3
// stages ahead (56 KB of LDS: 2 workgroups per CU).  At M = 2048 (512 tiles,
// the chip's 512 slots) that is 44.5-46.4 us against 50.5-51.5 us; below
// M = 1024 the 96-row tiles are faster (25 against 29 us at M = 256, where
// each tile's 32 stages set the time).
constexpr int kRbTN = 32;
constexpr int kRbOcc = 3;
constexpr int kRbTnTiles = 64;
constexpr int kRbOccTiles = 2;
constexpr int kRbBD = 3;
constexpr int kRbHL = 1;
constexpr int kRbAD = 2;
constexpr int kRbNW = 4;
constexpr int kGroupedBN = 128;  // grouped_mfma_kernel tile columns
constexpr int kRbBMTall = 128;
constexpr int kRbADTall = 3;
constexpr int64_t kDenseTallM = 1024;
// Wide dense tiles: 8 waves over 256 columns of a 128-row tile, one
// workgroup per CU.  Each activation stage then feeds twice the columns, a
// third fewer wave-loads per MFMA than two 4-wave workgroups; taken when the
// launch still gives each of the 256 CUs a tile.
constexpr int kRbNWWide = 8;
constexpr int64_t kRbWideTiles = 256;

template <typename T, bool SWIGLU, bool GATHER, int WL, int K, int BM = 96, int NW = kRbNW>
static int launch_rb(GemmArgs a, unsigned mtiles, hipStream_t st) {
  constexpr bool TILES = WL == kWlTiles || WL == kWlTilesF16;
  constexpr bool TALL = BM == kRbBMTall;
  static_assert(!TALL || (WL == kWlDirect && !SWIGLU && !GATHER), "tall tiles serve dense rows");
  static_assert(NW == kRbNW || (TALL && NW == kRbNWWide), "wide tiles serve dense tall rows");
  constexpr int TN = TILES ? kRbTnTiles : kRbTN;
  constexpr int OCC = NW == kRbNWWide ? 1 : TILES || TALL ? kRbOccTiles : kRbOcc;
  constexpr int AD = TALL ? kRbADTall : kRbAD;
  constexpr int RBN = NW * TN;
  a.nt_count = SWIGLU ? (int)cdiv(a.N / 2, RBN / 2) : (int)cdiv(a.N, RBN);
  a.mt_count = (int)mtiles;
  const int64_t grid = xcd_grid(a.mt_count, a.nt_count);
  LM_REQUIRE(grid < (int64_t(1) << 31), LM_EINVAL, "problem too large for one launch");
  grouped_rb_kernel<T, SWIGLU, GATHER, WL, K, BM, TN, kRbBD, kRbHL, AD, NW, OCC>
      <<<(unsigned)grid, NW * 64, 0, st>>>(a);
  return check_launch("grouped_rb_kernel");
}

// WL: weight load mode (kWlDirect for dense weights, kWlPermute or kWlTiles
// for the routed GEMMs, which stream each expert's weights once).
template <typename T, bool SWIGLU, bool GATHER, int WL>
static int launch_grouped(GemmArgs a, unsigned mtiles, hipStream_t st) {
  if (mtiles == 0) return LM_OK;
  if constexpr (WL == kWlDirect && !SWIGLU && !GATHER) {
    if (!a.table && a.tile_rows == kRbBMTall && (a.K == 2048 || a.K == 512)) {
      if ((int64_t)mtiles * cdiv(a.N, kRbNWWide * kRbTN) >= kRbWideTiles)
        return a.K == 2048
                   ? launch_rb<T, false, false, WL, 2048, kRbBMTall, kRbNWWide>(a, mtiles, st)
                   : launch_rb<T, false, false, WL, 512, kRbBMTall, kRbNWWide>(a, mtiles, st);
      return a.K == 2048 ? launch_rb<T, false, false, WL, 2048, kRbBMTall>(a, mtiles, st)
                         : launch_rb<T, false, false, WL, 512, kRbBMTall>(a, mtiles, st);
    }
  }
  if (a.tile_rows <= 96 && (a.K == 2048 || a.K == 512))
    return a.K == 2048 ? launch_rb<T, SWIGLU, GATHER, WL, 2048>(a, mtiles, st)
                       : launch_rb<T, SWIGLU, GATHER, WL, 512>(a, mtiles, st);
  constexpr int BN = kGroupedBN;
  a.nt_count = SWIGLU ? (int)cdiv(a.N / 2, BN / 2) : (int)cdiv(a.N, BN);
  a.mt_count = (int)mtiles;
  const int64_t grid = xcd_grid(a.mt_count, a.nt_count);
  LM_REQUIRE(grid < (int64_t(1) << 31), LM_EINVAL, "problem too large for one launch");
  grouped_mfma_kernel<T, SWIGLU, GATHER, BN><<<(unsigned)grid, 256, 0, st>>>(a);
  return check_launch("grouped_mfma_kernel");
}


template <typename T, int BM, int WM, bool SWIGLU, bool GATHER, bool DENSE>
static int launch_gemm(GemmArgs a, unsigned mtiles, hipStream_t st) {
  a.nt_count = SWIGLU ? (int)cdiv(a.N / 2, kBN / 2) : (int)cdiv(a.N, kBN);
  a.mt_count = (int)mtiles;
  if (mtiles == 0) return LM_OK;
  const int64_t grid = xcd_grid(a.mt_count, a.nt_count);
  LM_REQUIRE(grid < (int64_t(1) << 31), LM_EINVAL, "problem too large for one launch");
  w8a16_mfma_kernel<T, BM, WM, SWIGLU, GATHER, DENSE><<<(unsigned)grid, 256, 0, st>>>(a);
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
  // Rows at the model's K: the register-streamed kernel over 96-row tiles of
  // the dense matrix (128-row tiles from kDenseTallM rows; no tile table),
  // faster than the LDS-dequant kernel because each wave dequantizes only
  // its own columns' weights.
  if (k == 2048 || k == 512) {
    const int bm = m >= kDenseTallM ? kRbBMTall : 96;
    a.tile_rows = bm;
    return dtype == LM_BF16 ? launch_grouped<BF16, false, false, kWlDirect>(a, cdiv(m, bm), st)
                            : launch_grouped<FP16, false, false, kWlDirect>(a, cdiv(m, bm), st);
  }
  const unsigned mt = cdiv(m, 128);
  if (dtype == LM_BF16) return launch_gemm<BF16, 128, 2, false, false, true>(a, mt, st);
  return launch_gemm<FP16, 128, 2, false, false, true>(a, mt, st);
}

template <typename T>
static int routed_dispatch(const GemmArgs &a, unsigned mt, bool gather, bool swiglu,
                           hipStream_t st) {
  // The tile layout serves the fused layer's two GEMMs (gathered gate_up +
  // SwiGLU, contiguous down) in bf16; every other form reads q.
  const bool tiles = a.q_tiles != nullptr && std::is_same<T, BF16>::value;
  if (a.x_exp) {  // fp16 rows on LM_TILES_F16 weights, bf16 out (checked by routed_gemm)
    if constexpr (std::is_same<T, BF16>::value) {
      if (swiglu && gather) return launch_grouped<T, true, true, kWlTilesF16>(a, mt, st);
    }
    return set_error(LM_EINVAL, "fp16 tiles serve the gathered gate_up GEMM with SwiGLU");
  }
  if (swiglu) {
    if (gather)
      return tiles ? launch_grouped<T, true, true, kWlTiles>(a, mt, st)
                   : launch_grouped<T, true, true, kWlPermute>(a, mt, st);
    return launch_grouped<T, true, false, kWlPermute>(a, mt, st);
  }
  if (!gather)
    return tiles ? launch_grouped<T, false, false, kWlTiles>(a, mt, st)
                 : launch_grouped<T, false, false, kWlPermute>(a, mt, st);
  return launch_grouped<T, false, true, kWlPermute>(a, mt, st);
}

int routed_gemm(const RoutedGemm &r, hipStream_t st) {
  GemmArgs a{};
  a.x = static_cast<const uint16_t *>(r.x);
  a.ldx = r.ldx;
  a.pos = r.pos;
  a.table = r.table;
  a.experts = r.experts;
  a.y_rows = r.y_rows;
  a.x_rows = r.x_rows;
  a.q = r.q;
  a.q_es = r.q_es;
  a.q_tiles = r.q_tiles;
  a.x_exp = r.x_exp;
  a.ptile = r.ptile;
  a.s = r.s;
  a.s_es = r.s_es;
  a.y = static_cast<uint16_t *>(r.y);
  a.ldy = r.swiglu ? r.n / 2 : r.n;
  LM_REQUIRE(!r.q_tiles || (r.n % 32 == 0 && r.k % 64 == 0), LM_EINVAL,
             "the tile layout needs n % 32 == 0 and k % 64 == 0");
  LM_REQUIRE(!r.q_tiles || !r.gather || (r.ptile && r.bm == 96), LM_EINVAL,
             "gathered rows on the tile layout need the tile-major gather map of 96-row tiles");
  LM_REQUIRE(!r.x_exp || (r.q_tiles && r.dtype == LM_BF16 && r.bm <= 96 &&
                          (r.k == 2048 || r.k == 512)),
             LM_EINVAL, "fp16 rows need LM_TILES_F16 weights, bf16 output, tiles <= 96 rows "
                        "and k = 2048 or 512");
  a.N = (int)r.n;
  a.K = (int)r.k;
  a.tile_rows = (int)r.bm;
  const unsigned mt = (unsigned)r.n_tiles;
  return r.dtype == LM_BF16 ? routed_dispatch<BF16>(a, mt, r.gather, r.swiglu, st)
                            : routed_dispatch<FP16>(a, mt, r.gather, r.swiglu, st);
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
  LM_REQUIRE(m < (1LL << 31), LM_EINVAL, "Invalid INT8 group geometry");
  return w8a16_gemm_dense(x, q, s, y, m, n, k, dtype, large_tile, as_stream(stream));
}

static int check_routed(const RoutedGemm &r) {
  LM_REQUIRE(r.dtype == LM_BF16 || r.dtype == LM_FP16, LM_EINVAL,
             "W8A16 requires CUDA FP16/BF16 activations");
  LM_REQUIRE(r.k > 0 && r.k % 128 == 0 && r.n > 0 && r.n < (1LL << 30), LM_EINVAL,
             "Invalid INT8 group geometry");
  LM_REQUIRE(r.bm >= 1 && r.bm <= 128, LM_EINVAL, "tile height must be in 1..128");
  LM_REQUIRE(r.n_tiles >= 0 && r.n_tiles < 65536, LM_EINVAL, "too many tiles");
  LM_REQUIRE(r.experts >= 1 && r.y_rows >= 0 && r.x_rows >= 0, LM_EINVAL,
             "invalid bank or row count");
  if (r.n_tiles == 0 || r.y_rows == 0) return LM_OK;
  LM_REQUIRE(r.x && r.q && r.s && r.table && r.y, LM_EINVAL, "null pointer");
  LM_REQUIRE(r.x_rows >= 1, LM_EINVAL, "no activation rows");
  LM_REQUIRE(!r.gather || r.pos, LM_EINVAL, "gather needs pos");
  // contiguous rows: output row p reads activation row p
  LM_REQUIRE(r.gather || r.y_rows <= r.x_rows, LM_EINVAL, "more output rows than activation rows");
  return LM_OK;
}

extern "C" int lm_routed_gemm_w8a16(const void *x, int64_t x_rows, const int8_t *q, const float *s,
                                    int64_t experts, int64_t q_expert_stride,
                                    int64_t s_expert_stride, const int64_t *pos,
                                    const int64_t *table, int64_t n_tiles, int64_t bm, void *y,
                                    int64_t y_rows, int64_t n, int64_t k, int gather, int dtype,
                                    void *stream) {
  RoutedGemm r{x, k, x_rows, q, s, q_expert_stride, s_expert_stride, experts, pos, table,
               n_tiles, bm, y, y_rows, n, k, gather != 0, false, dtype};
  if (int rc = check_routed(r)) return rc;
  if (n_tiles == 0 || y_rows == 0) return LM_OK;
  return routed_gemm(r, as_stream(stream));
}

extern "C" int lm_routed_gate_up_swiglu(const void *x, int64_t x_rows, const int8_t *q,
                                        const float *s, int64_t experts, int64_t q_expert_stride,
                                        int64_t s_expert_stride, const int64_t *pos,
                                        const int64_t *table, int64_t n_tiles, int64_t bm,
                                        void *h, int64_t h_rows, int64_t n, int64_t k, int dtype,
                                        void *stream) {
  RoutedGemm r{x, k, x_rows, q, s, q_expert_stride, s_expert_stride, experts, pos, table,
               n_tiles, bm, h, h_rows, n, k, true, true, dtype};
  if (int rc = check_routed(r)) return rc;
  LM_REQUIRE(n % 2 == 0, LM_EINVAL, "gate_up needs an even number of rows");
  if (n_tiles == 0 || h_rows == 0) return LM_OK;
  return routed_gemm(r, as_stream(stream));
}
