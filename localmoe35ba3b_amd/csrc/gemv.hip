// Decode GEMV kernels behind the generic operator entry points:
//   lm_w8a8_grouped_gemv / lm_w8a8_grouped_linear   (w8a8.py:25-48)
//   lm_w8a8_linear (dense, optional SwiGLU)          (config: W8A8 gate_up)
//   lm_w8a8_group_partials                           (exact int32 partials)
//   lm_w8a16_grouped_gemv                            (int8.py:213-237)
//   lm_w8a16_linear for m <= 8                       (int8.py:9-37)
// All of them stream the weights with gemv_core.hpp; blockIdx.y selects the
// expert of a descriptor table (grouped mode) or is 0 (dense mode).
#include "gemv_core.hpp"

namespace lm {

constexpr int kGemvThreads = 256;  // workgroup size of the any-K kernels
constexpr int kGemvLoads = 8;      // weight loads per lane at kGemvThreads
// Large workgroups for launches that leave CUs idle or carry several
// activation rows: four times more threads share a block's rows, so the
// activation quantization, the weight loads of a lane (2 instead of 8) and
// the dot products of each wave shrink by four, and four waves per SIMD hide
// each other's dependency chains.  Launches of many blocks keep 256-thread
// workgroups, several per CU, which keep more bytes in flight per CU.
constexpr int kGemvThreadsK = 1024;
static bool gemv_large_blocks(int64_t blocks, int mt) { return blocks < 256 || mt >= 4; }

struct GemvArgs {
  const int64_t *table;  // grouped mode: [experts, 5] descriptor rows
  int field;
  int shared;
  const int8_t *q;  // dense mode weights [N, K] and scales [N, G]
  const float *s;
  const uint16_t *x;  // 16-bit activations [M, ldx]
  int64_t ldx;
  const int8_t *xq;  // pre-quantized activations [M, K] / [M, G]
  const float *xs;
  int M;
  uint16_t *y;  // output [M or experts, ldy]
  int64_t ldy;
  int32_t *partials;  // [M, N, G] (partials mode)
  int N;
  int K;
  int RB;  // weight rows per block (before SwiGLU pairing)
  int swiglu;
};

struct Resolved {
  const int8_t *q;
  const float *s;
  int xrow;   // first activation row used by this block
  int yrow;   // first output row written by this block
  int n0;     // first output column
  int rvalid; // rows streamed by this block
  RowMap map;
};

__device__ __forceinline__ Resolved resolve(const GemvArgs &a) {
  Resolved r;
  const int e = blockIdx.y;
  if (a.table) {
    r.q = reinterpret_cast<const int8_t *>(a.table[e * 5 + a.field]);
    r.s = reinterpret_cast<const float *>(a.table[e * 5 + a.field + 1]);
    r.xrow = a.shared ? 0 : e;
    r.yrow = e;
  } else {
    r.q = a.q;
    r.s = a.s;
    r.xrow = 0;
    r.yrow = 0;
  }
  if (a.swiglu) {
    const int half = a.N >> 1;
    const int hb = a.RB >> 1;
    r.n0 = blockIdx.x * hb;
    const int rh = min(hb, half - r.n0);
    r.rvalid = 2 * rh;
    r.map = RowMap{r.n0, half + r.n0, rh};
  } else {
    r.n0 = blockIdx.x * a.RB;
    r.rvalid = min(a.RB, a.N - r.n0);
    r.map = RowMap{r.n0, 0, 0};
  }
  return r;
}

// LDS carve-up: [xq or x16 | xs | ws | partials]
// T: dtype of the activations (QUANT) and of the output.
// KC: the reduction length as a compile-time constant (the model's 2048 and
// 512), or 0 for any K; with a constant K the load issue has no loops and
// no branches, so every wait count stays exact.
template <typename T, int MT, bool QUANT, bool PARTIALS, int KC, int TH>
__global__ __launch_bounds__(TH) void w8a8_gemv_kernel(GemvArgs a) {
  constexpr int LD = kGemvLoads * kGemvThreads / TH;  // weight loads per lane
  static_assert(LD >= 1, "workgroup size");
  extern __shared__ __align__(16) unsigned char smem[];
  const Resolved rv = resolve(a);
  const int K = KC ? KC : a.K, G = K >> 7, M = a.M;
  int8_t *xq = reinterpret_cast<int8_t *>(smem);
  float *xs = reinterpret_cast<float *>(smem + MT * K);
  float *ws = xs + MT * G;
  int *part = reinterpret_cast<int *>(ws + a.RB * G);
  const int RG = a.RB * G;
  const int8_t *q = rv.q;
  auto row_ptr = [&](int r) { return q + (int64_t)rv.map(r) * K; };
  const int sub = threadIdx.x & 7;
  // All MT rows are computed branch-free (rows past M read LDS rows that are
  // never stored back; only the stores are guarded), so the dot-product
  // chains of the rows interleave instead of running one basic block at a time.
  auto body = [&](u32x4 w, int r, int g, int f, bool ok) {
    u32x4 xv[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
      xv[m] = *reinterpret_cast<const u32x4 *>(xq + m * K + g * 128 + sub * 16);
    int p[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) p[m] = octet_sum_i32(dot16_i8(w, xv[m]));
    if (ok && sub == 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m < M) part[m * RG + f] = p[m];
    }
  };

  // One batch: when the block's weights fit one RowLoads batch and its
  // activations one register stage, the activations and scales are requested
  // first, the weights next, and the activations are staged in LDS only then,
  // so their wait does not include the weights: the two load latencies overlap.
  constexpr int QJ = 2 * MT * kGemvThreads / TH > 0 ? 2 * MT * kGemvThreads / TH : 1;
  constexpr int XN = MT * kGemvThreads / TH > 0 ? MT * kGemvThreads / TH : 1;
  // Four or more rows at the model's K: the int8 products on the matrix
  // cores (v_mfma_i32_16x16x64_i8).  The block's RB * G (row, group) pairs
  // are 16 tasks of 16 rows x one 128-group, one per wave: two MFMAs give the
  // group's exact int32 partials for 16 rows x 16 activation rows (rows past
  // M are computed from a repeated row and dropped), where the VALU path
  // would read every activation row from LDS once per weight piece.
  constexpr bool MF = MT >= 4 && KC != 0 && TH == 1024;
  static_assert(!MF || (32768 / KC) * (KC / 128) == 16 * (TH / 64), "one MFMA task per wave");
  // With K fixed, QuantRows stages the rows: one 128-group per slot of LPG
  // lanes (8 lanes from 8 rows, 16 from 4, a half-wave below), each slot a
  // fixed group of every QSTEP-th row, QJ2 rows per slot.
  constexpr int QG = KC ? KC / 128 : 1;
  constexpr int LPG = MT >= 8 ? 8 : MT >= 4 ? 16 : 32;
  constexpr bool QFIX = KC != 0 && (TH / LPG) % QG == 0;
  constexpr int QSTEP = TH / LPG / QG > 0 ? TH / LPG / QG : 1;
  constexpr int QJ2 = (MT + QSTEP - 1) / QSTEP;
  using QS = typename std::conditional<QFIX, QuantRows<T, QJ2, QG, TH, LPG>, QuantStage<T, QJ>>::type;
  const int th = threadIdx.x;
  if (rv.rvalid * G <= LD * 8 * (TH / 64) && M * G <= TH &&
      (QUANT ? (QFIX || M * G <= QJ * (TH / 32)) : M * K <= XN * 16 * TH)) {
    QS qst;
    RowStage<XN> cst;
    if constexpr (QUANT)
      qst.load(a.x + (int64_t)rv.xrow * a.ldx, a.ldx, M, K);
    else
      cst.load(reinterpret_cast<const unsigned char *>(a.xq + (int64_t)rv.xrow * K), K, M, K);
    const int ti = min(th, M * G - 1);
    const float xsv = (!QUANT && a.xs) ? ldg_f32(a.xs + (int64_t)(rv.xrow + ti / G) * G + ti % G) : 0.0f;
    const int tw = min(th, rv.rvalid * G - 1);
    const float wsv = PARTIALS ? 0.0f : ldg_f32(rv.s + (int64_t)rv.map(tw / G) * G + tw % G);
    RowLoads<MF ? 1 : LD, TH> L;
    // MFMA task of this wave: rows 16 rb .. 16 rb + 15 of the block, group mg;
    // lane l holds weight row 16 rb + (l & 15), bytes 16 (l >> 4) of each
    // 64-K half of the group (the MFMA B layout).
    const int lane = th & 63, rb = (th >> 6) / G, mg = (th >> 6) - rb * G;
    const int mrow = 16 * rb + (lane & 15);
    i32x4 mb[2];
    if constexpr (MF) {
      const int8_t *bp = row_ptr(min(mrow, rv.rvalid - 1)) + mg * 128 + (lane >> 4) * 16;
      mb[0] = ldg<i32x4>(bp);
      mb[1] = ldg<i32x4>(bp + 64);
    } else {
      L.issue(rv.rvalid, G, row_ptr);
    }
    if constexpr (QUANT)
      qst.store(K, xq, xs);
    else
      cst.store(reinterpret_cast<unsigned char *>(xq));
    // branch-free: surplus threads rewrite the last entry with its own value
    if (!QUANT && a.xs) xs[ti] = xsv;
    if (!PARTIALS) ws[tw] = wsv;
    __syncthreads();
    if constexpr (MF) {
      // A: activation row (lane & 15) (repeated past MT), same bytes as B.
      const int8_t *ap = xq + (lane & 15 & (MT - 1)) * K + mg * 128 + (lane >> 4) * 16;
      i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4 *>(ap), mb[0],
                                                     i32x4{0, 0, 0, 0}, 0, 0, 0);
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4 *>(ap + 64), mb[1], c,
                                               0, 0, 0);
      // C layout: lane l holds weight row 16 rb + (l & 15), activation rows
      // 4 (l >> 4) .. 4 (l >> 4) + 3.
      if (mrow < rv.rvalid) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 4 * (lane >> 4) + i;
          if (m < M) part[m * RG + mrow * G + mg] = c[i];
        }
      }
    } else {
      L.consume(body);
    }
    __syncthreads();
  } else {
    // Activations: quantize bf16 rows, or copy pre-quantized rows.
    if constexpr (QUANT) {
      quantize_rows_to_lds<T>(a.x + (int64_t)rv.xrow * a.ldx, a.ldx, M, K, xq, xs);
    } else {
      for (int i = threadIdx.x; i < M * K / 16; i += blockDim.x) {
        const int m = (i * 16) / K, c = (i * 16) - m * K;
        *reinterpret_cast<u32x4 *>(xq + m * K + c) =
            ldg16(a.xq + (int64_t)(rv.xrow + m) * K + c);
      }
      if (a.xs)
        for (int i = threadIdx.x; i < M * G; i += blockDim.x)
          xs[i] = a.xs[(int64_t)(rv.xrow + i / G) * G + i % G];
    }
    if constexpr (!PARTIALS) {
      for (int i = threadIdx.x; i < rv.rvalid * G; i += blockDim.x) {
        const int r = i / G, g = i - r * G;
        ws[i] = ldg_f32(rv.s + (int64_t)rv.map(r) * G + g);
      }
    }
    __syncthreads();
    stream_rows<kGemvLoads>(rv.rvalid, G, row_ptr, body);
    __syncthreads();
  }

  if constexpr (PARTIALS) {
    for (int i = threadIdx.x; i < M * rv.rvalid * G; i += blockDim.x) {
      const int m = i / (rv.rvalid * G);
      const int f = i - m * rv.rvalid * G;
      const int r = f / G, g = f - r * G;
      a.partials[((int64_t)m * a.N + rv.map(r)) * G + g] = part[m * RG + f];
    }
    return;
  } else {
    if (a.swiglu) {
      const int rh = rv.rvalid >> 1;
      for (int i = threadIdx.x; i < M * rh; i += blockDim.x) {
        const int m = i / rh, t = i - m * rh;
        const float gate = T::round(w8a8_epilogue(part + m * RG + t * G, xs + m * G, ws + t * G, G));
        const float up =
            T::round(w8a8_epilogue(part + m * RG + (rh + t) * G, xs + m * G, ws + (rh + t) * G, G));
        const float act = T::round(silu_f32(gate));
        a.y[(int64_t)(rv.yrow + m) * a.ldy + rv.n0 + t] = T::from_f32(act * up);
      }
    } else {
      for (int i = threadIdx.x; i < M * rv.rvalid; i += blockDim.x) {
        const int m = i / rv.rvalid, t = i - m * rv.rvalid;
        const float acc = w8a8_epilogue(part + m * RG + t * G, xs + m * G, ws + t * G, G);
        a.y[(int64_t)(rv.yrow + m) * a.ldy + rv.n0 + t] = T::from_f32(acc);
      }
    }
  }
}

// W8A16: dequantize to T exactly (T(q * s)), fp32 dot products.
// LDS carve-up: [x16 rows | ws | partials]
template <typename T, int MT, int KC, int TH>
__global__ __launch_bounds__(TH) void w8a16_gemv_kernel(GemvArgs a) {
  constexpr int LD = kGemvLoads * kGemvThreads / TH;  // weight loads per lane
  static_assert(LD >= 1, "workgroup size");
  extern __shared__ __align__(16) unsigned char smem[];
  const Resolved rv = resolve(a);
  const int K = KC ? KC : a.K, G = K >> 7, M = a.M;
  uint16_t *xl = reinterpret_cast<uint16_t *>(smem);
  float *ws = reinterpret_cast<float *>(smem + MT * K * 2);
  float *part = ws + a.RB * G;
  const int RG = a.RB * G;
  const int8_t *q = rv.q;
  auto row_ptr = [&](int r) { return q + (int64_t)rv.map(r) * K; };
  const int sub = threadIdx.x & 7;
  // All MT rows computed branch-free, stores guarded (as in w8a8_gemv_kernel).
  auto body = [&](u32x4 w, int r, int g, int f, bool ok) {
    const float sc = ok ? ws[f] : 0.0f;
    u32x4 x0[MT], x1[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint16_t *xp = xl + m * K + g * 128 + sub * 16;
      x0[m] = *reinterpret_cast<const u32x4 *>(xp);
      x1[m] = *reinterpret_cast<const u32x4 *>(xp + 8);
    }
    uint32_t wd[8];
    dequant16<T>(w, sc, wd);
    float p[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) p[m] = octet_sum_f32(dot16_w16<T>(wd, x0[m], x1[m]));
    if (ok && sub == 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m < M) part[m * RG + f] = p[m];
    }
  };
  const unsigned char *xsrc = reinterpret_cast<const unsigned char *>(a.x + (int64_t)rv.xrow * a.ldx);
  // One batch, as in w8a8_gemv_kernel: activations and scales requested
  // before the weights, staged in LDS after them.
  constexpr int XN = 2 * MT * kGemvThreads / TH > 0 ? 2 * MT * kGemvThreads / TH : 1;
  if (rv.rvalid * G <= LD * 8 * (TH / 64) && M * K * 2 <= XN * 16 * TH) {
    RowStage<XN> cst;
    cst.load(xsrc, a.ldx * 2, M, K * 2);
    const int tw = min((int)threadIdx.x, rv.rvalid * G - 1);
    const float wsv = ldg_f32(rv.s + (int64_t)rv.map(tw / G) * G + tw % G);
    RowLoads<LD, TH> L;
    L.issue(rv.rvalid, G, row_ptr);
    cst.store(reinterpret_cast<unsigned char *>(xl));
    ws[tw] = wsv;  // branch-free: surplus threads rewrite the last entry with its own value
    __syncthreads();
    L.consume(body);
  } else {
    for (int i = threadIdx.x; i < M * K / 8; i += blockDim.x) {
      const int m = (i * 8) / K, c = (i * 8) - m * K;
      *reinterpret_cast<u32x4 *>(xl + m * K + c) = ldg16(a.x + (int64_t)(rv.xrow + m) * a.ldx + c);
    }
    for (int i = threadIdx.x; i < rv.rvalid * G; i += blockDim.x) {
      const int r = i / G, g = i - r * G;
      ws[i] = ldg_f32(rv.s + (int64_t)rv.map(r) * G + g);
    }
    __syncthreads();
    stream_rows<kGemvLoads>(rv.rvalid, G, row_ptr, body);
  }
  __syncthreads();

  for (int i = threadIdx.x; i < M * rv.rvalid; i += blockDim.x) {
    const int m = i / rv.rvalid, t = i - m * rv.rvalid;
    const float acc = ordered_sum8(part + m * RG + t * G, G);
    a.y[(int64_t)(rv.yrow + m) * a.ldy + rv.n0 + t] = T::from_f32(acc);
  }
}

// Rows per block: about 32 KB of weights (8 loads in flight per lane).
static int gemv_rows_per_block(int64_t k) {
  int rb = (int)(32768 / k);
  if (rb < 2) rb = 2;
  if (rb > 256) rb = 256;
  rb &= ~1;
  return rb;
}

static int mt_for(int64_t m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8; }

template <typename T, int MT, bool QUANT, bool PARTIALS>
static int launch_w8a8(const GemvArgs &a, unsigned gy, hipStream_t st) {
  const int G = a.K / 128;
  const size_t lds = (size_t)MT * a.K + (size_t)MT * G * 4 + (size_t)a.RB * G * 4 +
                     (size_t)MT * a.RB * G * 4;
  LM_REQUIRE(lds <= 160 * 1024, LM_EINVAL, "Invalid INT8 group geometry");
  const unsigned gx = a.swiglu ? cdiv(a.N / 2, a.RB / 2) : cdiv(a.N, a.RB);
  const dim3 grid(gx, gy);
  const bool large = gemv_large_blocks((int64_t)gx * gy, MT);
  if (a.K == 2048 && large)
    w8a8_gemv_kernel<T, MT, QUANT, PARTIALS, 2048, kGemvThreadsK>
        <<<grid, kGemvThreadsK, lds, st>>>(a);
  else if (a.K == 2048)
    w8a8_gemv_kernel<T, MT, QUANT, PARTIALS, 2048, kGemvThreads>
        <<<grid, kGemvThreads, lds, st>>>(a);
  else if (a.K == 512 && large)
    w8a8_gemv_kernel<T, MT, QUANT, PARTIALS, 512, kGemvThreadsK>
        <<<grid, kGemvThreadsK, lds, st>>>(a);
  else if (a.K == 512)
    w8a8_gemv_kernel<T, MT, QUANT, PARTIALS, 512, kGemvThreads>
        <<<grid, kGemvThreads, lds, st>>>(a);
  else
    w8a8_gemv_kernel<T, MT, QUANT, PARTIALS, 0, kGemvThreads><<<grid, kGemvThreads, lds, st>>>(a);
  return check_launch("w8a8_gemv_kernel");
}

template <typename T, bool QUANT, bool PARTIALS>
static int dispatch_w8a8_t(const GemvArgs &a, unsigned gy, hipStream_t st) {
  switch (mt_for(a.M)) {
    case 1: return launch_w8a8<T, 1, QUANT, PARTIALS>(a, gy, st);
    case 2: return launch_w8a8<T, 2, QUANT, PARTIALS>(a, gy, st);
    case 4: return launch_w8a8<T, 4, QUANT, PARTIALS>(a, gy, st);
    default: return launch_w8a8<T, 8, QUANT, PARTIALS>(a, gy, st);
  }
}
template <bool QUANT, bool PARTIALS>
static int dispatch_w8a8(const GemvArgs &a, int dtype, unsigned gy, hipStream_t st) {
  return dtype == LM_FP16 ? dispatch_w8a8_t<FP16, QUANT, PARTIALS>(a, gy, st)
                          : dispatch_w8a8_t<BF16, QUANT, PARTIALS>(a, gy, st);
}

template <typename T, int MT>
static int launch_w8a16(const GemvArgs &a, unsigned gy, hipStream_t st) {
  const int G = a.K / 128;
  const size_t lds = (size_t)MT * a.K * 2 + (size_t)a.RB * G * 4 + (size_t)MT * a.RB * G * 4;
  LM_REQUIRE(lds <= 160 * 1024, LM_EINVAL, "Invalid INT8 group geometry");
  const dim3 grid(cdiv(a.N, a.RB), gy);
  const bool large = gemv_large_blocks((int64_t)grid.x * gy, MT);
  if (a.K == 2048 && large)
    w8a16_gemv_kernel<T, MT, 2048, kGemvThreadsK><<<grid, kGemvThreadsK, lds, st>>>(a);
  else if (a.K == 2048)
    w8a16_gemv_kernel<T, MT, 2048, kGemvThreads><<<grid, kGemvThreads, lds, st>>>(a);
  else if (a.K == 512 && large)
    w8a16_gemv_kernel<T, MT, 512, kGemvThreadsK><<<grid, kGemvThreadsK, lds, st>>>(a);
  else if (a.K == 512)
    w8a16_gemv_kernel<T, MT, 512, kGemvThreads><<<grid, kGemvThreads, lds, st>>>(a);
  else
    w8a16_gemv_kernel<T, MT, 0, kGemvThreads><<<grid, kGemvThreads, lds, st>>>(a);
  return check_launch("w8a16_gemv_kernel");
}

template <typename T>
static int dispatch_w8a16(const GemvArgs &a, unsigned gy, hipStream_t st) {
  switch (mt_for(a.M)) {
    case 1: return launch_w8a16<T, 1>(a, gy, st);
    case 2: return launch_w8a16<T, 2>(a, gy, st);
    case 4: return launch_w8a16<T, 4>(a, gy, st);
    default: return launch_w8a16<T, 8>(a, gy, st);
  }
}

int w8a16_gemv_dense(const void *x, const int8_t *q, const float *s, void *y, int64_t m,
                     int64_t n, int64_t k, int dtype, hipStream_t st) {
  GemvArgs a{};
  a.q = q;
  a.s = s;
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = k;
  a.M = (int)m;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = n;
  a.N = (int)n;
  a.K = (int)k;
  a.RB = gemv_rows_per_block(k);
  return dtype == LM_BF16 ? dispatch_w8a16<BF16>(a, 1, st) : dispatch_w8a16<FP16>(a, 1, st);
}

}  // namespace lm

using namespace lm;

static int check_grouped(int64_t experts, int64_t n, int64_t k, int field) {
  LM_REQUIRE(experts >= 0 && n > 0 && k > 0 && k % 128 == 0 && k <= 65536, LM_EINVAL,
             "Invalid INT8 group geometry");
  LM_REQUIRE(field == 0 || field == 2, LM_EINVAL, "descriptor field must be 0 or 2");
  LM_REQUIRE(n <= (1 << 24), LM_EINVAL, "Invalid INT8 group geometry");
  return LM_OK;
}

static int check_dtype(int dtype, const char *msg) {
  LM_REQUIRE(dtype == LM_BF16 || dtype == LM_FP16, LM_EINVAL, msg);
  return LM_OK;
}

extern "C" int lm_w8a8_grouped_gemv(const int8_t *xq, const float *xs, const int64_t *table,
                                    void *y, int64_t experts, int64_t n, int64_t k, int field,
                                    int shared, int y_dtype, void *stream) {
  if (int rc = check_grouped(experts, n, k, field)) return rc;
  if (int rc = check_dtype(y_dtype, "W8A8 output must be bf16 or fp16")) return rc;
  if (experts == 0) return LM_OK;
  LM_REQUIRE(xq && xs && table && y, LM_EINVAL, "null pointer");
  GemvArgs a{};
  a.table = table;
  a.field = field;
  a.shared = shared;
  a.xq = xq;
  a.xs = xs;
  a.M = 1;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = n;
  a.N = (int)n;
  a.K = (int)k;
  a.RB = gemv_rows_per_block(k);
  return dispatch_w8a8<false, false>(a, y_dtype, (unsigned)experts, as_stream(stream));
}

extern "C" int lm_w8a8_grouped_linear(const void *x, const int64_t *table, void *y,
                                      int64_t experts, int64_t n, int64_t k, int field,
                                      int shared, int dtype, void *stream) {
  if (int rc = check_grouped(experts, n, k, field)) return rc;
  if (int rc = check_dtype(dtype, "Expected CUDA rows with K divisible by 128")) return rc;
  if (experts == 0) return LM_OK;
  LM_REQUIRE(x && table && y, LM_EINVAL, "null pointer");
  GemvArgs a{};
  a.table = table;
  a.field = field;
  a.shared = shared;
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = k;
  a.M = 1;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = n;
  a.N = (int)n;
  a.K = (int)k;
  a.RB = gemv_rows_per_block(k);
  return dispatch_w8a8<true, false>(a, dtype, (unsigned)experts, as_stream(stream));
}

extern "C" int lm_w8a8_linear(const void *x, const int8_t *q, const float *s, void *y, int64_t m,
                              int64_t n, int64_t k, int swiglu, int dtype, void *stream) {
  LM_REQUIRE(m >= 0 && m <= 8, LM_EINVAL, "W8A8 decode linear supports 1..8 rows");
  LM_REQUIRE(n > 0 && k > 0 && k % 128 == 0 && k <= 65536, LM_EINVAL,
             "Invalid INT8 group geometry");
  LM_REQUIRE(!swiglu || n % 2 == 0, LM_EINVAL, "SwiGLU needs an even number of rows");
  if (int rc = check_dtype(dtype, "Expected CUDA rows with K divisible by 128")) return rc;
  if (m == 0) return LM_OK;
  LM_REQUIRE(x && q && s && y, LM_EINVAL, "null pointer");
  GemvArgs a{};
  a.q = q;
  a.s = s;
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = k;
  a.M = (int)m;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = swiglu ? n / 2 : n;
  a.N = (int)n;
  a.K = (int)k;
  a.RB = gemv_rows_per_block(k);
  a.swiglu = swiglu ? 1 : 0;
  return dispatch_w8a8<true, false>(a, dtype, 1, as_stream(stream));
}

extern "C" int lm_w8a8_group_partials(const int8_t *xq, const int8_t *wq, int32_t *p, int64_t m,
                                      int64_t n, int64_t k, void *stream) {
  LM_REQUIRE(m >= 0 && m <= 8, LM_EINVAL, "W8A8 partials support 1..8 rows");
  LM_REQUIRE(n > 0 && k > 0 && k % 128 == 0 && k <= 65536, LM_EINVAL,
             "Invalid INT8 group geometry");
  if (m == 0) return LM_OK;
  LM_REQUIRE(xq && wq && p, LM_EINVAL, "null pointer");
  GemvArgs a{};
  a.q = wq;
  a.xq = xq;
  a.xs = nullptr;
  a.M = (int)m;
  a.partials = p;
  a.N = (int)n;
  a.K = (int)k;
  a.RB = gemv_rows_per_block(k);
  return dispatch_w8a8<false, true>(a, LM_BF16, 1, as_stream(stream));
}

extern "C" int lm_w8a16_grouped_gemv(const void *x, const int64_t *table, void *y,
                                     int64_t experts, int64_t n, int64_t k, int field, int shared,
                                     int dtype, void *stream) {
  if (int rc = check_grouped(experts, n, k, field)) return rc;
  if (int rc = check_dtype(dtype, "W8A16 requires CUDA FP16/BF16 activations")) return rc;
  if (experts == 0) return LM_OK;
  LM_REQUIRE(x && table && y, LM_EINVAL, "null pointer");
  GemvArgs a{};
  a.table = table;
  a.field = field;
  a.shared = shared;
  a.x = static_cast<const uint16_t *>(x);
  a.ldx = k;
  a.M = 1;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = n;
  a.N = (int)n;
  a.K = (int)k;
  a.RB = gemv_rows_per_block(k);
  return dtype == LM_FP16 ? dispatch_w8a16<FP16>(a, (unsigned)experts, as_stream(stream))
                          : dispatch_w8a16<BF16>(a, (unsigned)experts, as_stream(stream));
}
