// Fused MoE-FFN layer of the synthetic stack: RMSNorm -> router top-8 ->
// 8 routed experts + the always-on shared expert -> weighted combine ->
// sigmoid-gated shared add -> residual (HF:779-798, 801-815, 866-875).
//
// Decode (one token) runs three kernels and never leaves the device:
//   decode_router_kernel   RMSNorm, fp64 router logits (one wave per expert),
//                          activation quantization of the normalized row, the
//                          shared-expert gate.
//   decode_gate_up_kernel  top-8 + softmax renormalisation (every workgroup,
//                          redundantly), then gate_up rows of the 8 routed
//                          experts (W8A8, w8a8.py) and of the shared expert
//                          (W8A16), SwiGLU.
//   decode_down_kernel     down rows of all 9 experts for 8 output columns,
//                          W8A8 (row-quantized SwiGLU output) / W8A16, then the
//                          ascending-expert bf16 combine (int8.py:240-250), the
//                          gated shared add and the residual add, in place.
// Prefill runs: RMSNorm + shared gate, router (fp64 MFMA), top-k with
// per-workgroup expert counts, the route plan scan (with the shared expert
// appended as extra tiles), grouped W8A16 gate_up GEMM with fused SwiGLU,
// grouped W8A16 down GEMM, and a per-token combine.
#include <algorithm>
#include <mutex>
#include <unordered_map>

#include "gemv_core.hpp"
#include "internal.hpp"

namespace lm {

constexpr int kH = 2048;
constexpr int kI = 512;
constexpr int kE = 256;
constexpr int kTopK = 8;
constexpr int kBM = 96;  // prefill MFMA tile height (one tile covers a typical expert)
constexpr int kTopkTokens = 8;  // prefill top-k: tokens (waves) per workgroup
static_assert(kE == 256, "the prefill kernels map one thread of a 256-thread workgroup to each expert");

struct WsLayout {
  int64_t bcounts, xn, xh, xk, gl, logits, nx, nw, ids, wts, sel, selw, xq, xs, dacc_gu, dacc_dn,
      pos, table, ptile, rslot, rpos, hbuf, vbuf, total;
  int64_t max_tiles, n_tiles;
};

constexpr int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

constexpr WsLayout layout(int64_t T) {
  WsLayout w{};
  const int64_t R = T * kTopK;
  w.max_tiles = (R + kBM - 1) / kBM + kE;
  w.n_tiles = w.max_tiles + (T + kBM - 1) / kBM;
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o = align256(o + bytes);
    return at;
  };
  w.xn = take(T * kH * 2);
  w.xh = take(T * kH * 2);  // prefill: fp16(xn * 2^xk) for the fp16 gate_up GEMM
  w.xk = take(T * 4);       // prefill: the per-row power of two of xh
  w.gl = take(T * 4);
  w.logits = take(T * kE * 4);
  w.nx = take(T * 4);
  w.nw = take(kE * 4);
  w.ids = take(T * kTopK * 8);
  w.wts = take(T * kTopK * 2);
  w.sel = take(kTopK * 4);
  w.selw = take(kTopK * 4);
  w.xq = take(kH);
  w.xs = take(kH / 128 * 4);
  w.dacc_gu = take(kTopK * 2 * kI * 4);  // decode: fp32 W8A8 sums of the routed gate_up rows
  w.dacc_dn = take(kTopK * kH * 4);      // decode: fp32 W8A8 sums of the routed down rows
  w.pos = take((R + T) * 8);
  w.table = take(w.n_tiles * 3 * 8);
  w.ptile = take(w.n_tiles * kBM * 4);  // token of row r of table tile i at i * kBM + r
  w.bcounts = take((T + kTopkTokens - 1) / kTopkTokens * kE);  // per top-k workgroup expert counts (bytes)
  w.rslot = take(R * 4);  // rank of each route inside its top-k workgroup and expert
  w.rpos = take(R * 4);   // sorted row of each route
  w.hbuf = take((R + T) * kI * 2);
  w.vbuf = take((R + T) * kH * 2);
  w.total = o;
  return w;
}

struct LayerArgs {
  const uint16_t *router_w;
  const float *router_bias;
  const uint16_t *gate_w;
  const float *norm_w;
  const int8_t *gu_q;
  const float *gu_s;
  const int8_t *dn_q;
  const float *dn_s;
  int64_t gu_qes, gu_ses, dn_qes, dn_ses;
  uint16_t *h;
  float eps;
  // workspace views
  uint16_t *xn;
  uint16_t *xh;  // prefill: fp16(xn * 2^xk), exact
  int *xk;
  float *gl;
  float *logits;
  float *nx;  // prefill: |xn| of each token row
  float *nw;  // prefill: |w_e| of each router row
  int64_t *ids;
  uint16_t *wts;
  int *sel;
  float *selw;
  int8_t *xq;
  float *xs;
  uint16_t *hbuf;
  uint16_t *vbuf;   // decode: the 8 routed down rows (bf16) and the shared one
  float *dacc_gu;   // decode: fp32 epilogue sums of the routed gate_up rows [8, 2I]
  float *dacc_dn;   // decode: fp32 epilogue sums of the routed down rows [8, H]
  int32_t *ids_out;
  uint16_t *wts_out;
};

// ------------------------------------------------------------------ decode
// The norm weight of a layer that has none: zeros, so that the factor
// (1 + w) is exactly 1 and both cases share one branch-free path.
__device__ float g_zero_norm_w[kH];

// Thread t's norm weights w[8 t .. 8 t + 7] as two 16-byte pieces, requested
// unconditionally: a load under a branch would make the compiler wait for
// every load in flight where the branch joins.
struct NormW {
  u32x4 lo, hi;
};
__device__ __forceinline__ NormW load_norm_w(const float *nw) {
  const float *p = (nw ? nw : g_zero_norm_w) + threadIdx.x * (kH / 256);
  return NormW{ldg16(p), ldg16(p + 4)};
}

// RMSNorm of one row of kH bf16 values (HF:807-815).  Thread t passes in
// its chunk, values 8 t .. 8 t + 7, and its norm weights, and receives the
// chunk normalized and rounded to bf16.  Fixed reduction order (per-thread
// sum, 64-lane xor butterfly, the 4 wave sums left to right, IEEE 1/sqrtf),
// which the oracle restates.
__device__ __forceinline__ void norm_row(u32x4 raw, const NormW &nw, float eps, float *red,
                                         float y[kH / 256]) {
  constexpr int PER = kH / 256;
  const int t = threadIdx.x;
  float v[PER];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = bf16_bits_to_f32(raw[j] & 0xFFFFu);
    v[2 * j + 1] = bf16_bits_to_f32(raw[j] >> 16);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) ss += v[j] * v[j];
  ss = wave_sum_f32(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float r = 1.0f / sqrtf(tot / (float)kH + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float w = __uint_as_float(j < 4 ? nw.lo[j] : nw.hi[j - 4]);
    y[j] = round_bf16((v[j] * r) * (1.0f + w));
  }
}

// The normalized row as LDS floats (bf16-rounded values); `raw` is thread
// t's chunk of the row (values 8 t .. 8 t + 7).
__device__ __forceinline__ void norm_row_to_lds(u32x4 raw, const NormW &nw, float eps, float *xf,
                                                float *red) {
  constexpr int PER = kH / 256;
  float y[PER];
  norm_row(raw, nw, eps, red, y);
#pragma unroll
  for (int j = 0; j < PER; ++j) xf[threadIdx.x * PER + j] = y[j];
  __syncthreads();
}

constexpr int kGuPairs = 8;  // routed SwiGLU columns per gate_up workgroup
constexpr int kRouterBlocks = kE / 4;  // one router expert per wave, + 1 workgroup for the gate logit

// Decode layer, first kernel: router logits of the token (workgroups
// 0 .. E/4 - 1, one expert per wave) and the shared-expert gate logit
// (workgroup E/4).  The hidden row is requested first and the router rows
// right after it, so the RMSNorm waits for the row alone and the router
// rows' HBM latency overlaps it.  Every workgroup normalizes the row itself,
// so workgroups 0 .. H/128 - 1 also write one 128-wide group of the
// normalized row and its W8A8 quantization.  No inter-workgroup sync.
// The three decode kernels take the pointers their first loads need as
// leading scalar arguments (the rest stay in LayerArgs): moe.hip is built
// with kernel-argument preloading, so the hardware places those pointers in
// SGPRs at launch and the first loads are issued without waiting for a
// kernel-argument fetch (one memory round trip, about 0.3-0.5 us, on each of
// the three dependent launches of a decode layer).
__global__ __launch_bounds__(256) void decode_router_kernel(uint16_t *p_h, const float *p_norm_w,
                                                            const uint16_t *p_router_w,
                                                            const uint16_t *p_gate_w, LayerArgs a) {
  a.h = p_h;
  a.norm_w = p_norm_w;
  a.router_w = p_router_w;
  a.gate_w = p_gate_w;
  __shared__ float xf[kH];
  __shared__ float red[4];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const bool routed = blockIdx.x < kRouterBlocks;
  // Workgroup b runs on XCD b % 8.  Expert groups are dealt out so that the
  // 8 workgroups writing one 128-byte line of logits share an XCD.
  const int b = blockIdx.x;
  const int e = ((b & 7) * (kRouterBlocks / 8) + (b >> 3)) * 4 + wave;
  const uint16_t *wrow = routed ? a.router_w + (int64_t)e * kH : a.gate_w;
  const u32x4 hrow = ldg16(a.h + t * (kH / 256));
  const NormW nwv = load_norm_w(a.norm_w);
  u32x4 wv[kH / 512];
#pragma unroll
  for (int j = 0; j < kH / 512; ++j) wv[j] = ldg16(wrow + lane * 8 + j * 512);
  norm_row_to_lds(hrow, nwv, a.eps, xf, red);

  if (blockIdx.x < kH / 128) {
    const int g = blockIdx.x;
    if (t < 64) {
      a.xn[g * 128 + 2 * t] = f32_to_bf16_bits(xf[g * 128 + 2 * t]);
      a.xn[g * 128 + 2 * t + 1] = f32_to_bf16_bits(xf[g * 128 + 2 * t + 1]);
    } else if (t < 96) {  // w8a8.quantize of group g: 32 lanes x 4 values
      const int l = t - 64;
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = xf[g * 128 + l * 4 + j];
      const float am =
          halfwave_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
      const float sc = fmaxf(am, 1e-10f) * (float)(1.0 / 127.0);
      const float rs = 1.0f / sc;
      uint32_t packed = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        packed |= ((uint32_t)(uint8_t)(int8_t)(int)rintf(quant_div(v[j], sc, rs))) << (8 * j);
      *reinterpret_cast<uint32_t *>(a.xq + g * 128 + l * 4) = packed;
      if (l == 0) a.xs[g] = sc;
    }
  }

  if (routed || wave == 0) {
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < kH / 512; ++j) {
      const int k0 = lane * 8 + j * 512;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc = __builtin_fma((double)xf[k0 + 2 * i], (double)bf16_bits_to_f32(wv[j][i] & 0xFFFFu),
                            acc);
        acc = __builtin_fma((double)xf[k0 + 2 * i + 1], (double)bf16_bits_to_f32(wv[j][i] >> 16),
                            acc);
      }
    }
    acc = wave_sum_f64_dpp(acc);
    if (lane == 0) {
      float l = round_bf16((float)acc);
      if (routed) {
        if (a.router_bias) l = l + a.router_bias[e];
        a.logits[e] = l;
      } else {
        a.gl[0] = l;
      }
    }
  }
}

// Top-8 of the decode token over the 256 router logits (HF:770-774), with
// all four waves of the workgroup: thread t holds expert t's logit v, every
// wave selects the 8 largest keys (logit desc, id asc) of its 64 experts,
// and after one barrier every wave merges the four lists itself, so no wave
// waits on another again.  Lanes 0 .. 7 of the result hold the top 8 in
// descending key order.  Every gate_up workgroup runs it on the same inputs,
// so all of them agree.
template <class KT>
__device__ __forceinline__ typename KT::T decode_top8(float v) {
  using T = typename KT::T;
  __shared__ T lists[4 * kTopK];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  T k = wave_top8(KT::make(v, t), lane);
  if (lane < kTopK) lists[wave * kTopK + lane] = k;
  __syncthreads();
  k = lists[lane & 31];
  k = merge_top8<15>(k, lane);
  return merge_top8<23>(k, lane);
}

// Expert id of combine slot `slot` (the slot-th smallest of the 8 selected
// ids), from the merged keys k of decode_top8.
template <class KT>
__device__ __forceinline__ int decode_slot_expert(typename KT::T k, int slot) {
  const int lane = threadIdx.x & 63;
  const int id = clamp_index32(KT::index(k), kE);
  int rank = 0;
#pragma unroll
  for (int i = 0; i < kTopK; ++i)
    rank += clamp_index32(KT::index(KT::readlane(k, i)), kE) < id ? 1 : 0;
  const unsigned long long m = __ballot(lane < kTopK && rank == slot);
  return __builtin_amdgcn_readlane(id, m ? (int)__builtin_ctzll(m) : 0);
}

// Routing weights of the selection and its publication for the down kernel
// and the caller (one wave of workgroup 0): the softmax denominator from v4,
// lane l's logits of experts 4 l .. 4 l + 3, fp32 softmax, renormalisation
// in rank order, bf16 weights - topk_wave's arithmetic, so ids and weights
// equal the single-wave selection bit for bit.  a.sel / a.selw are in combine
// order (ascending expert id).
template <class KT>
__device__ __forceinline__ void decode_publish(const LayerArgs &a, typename KT::T k,
                                               const float v4[4]) {
  const int lane = threadIdx.x & 63;
  const float mx = KT::value(KT::readlane(k, 0));
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) part += expf(v4[j] - mx);
  part = row_sum_f32(part);
  const float d = (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 0)) +
                   __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 16))) +
                  (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 32)) +
                   __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 48)));
  const float pe = expf(KT::value(k) - mx) / d;
  float psum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), 0));
#pragma unroll
  for (int i = 1; i < kTopK; ++i)
    psum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), i));
  const uint16_t wb = f32_to_bf16_bits(pe / psum);
  const int id = clamp_index32(KT::index(k), kE);
  int rank = 0;  // combine slot: rank of the id in ascending order (the ids are distinct)
#pragma unroll
  for (int i = 0; i < kTopK; ++i)
    rank += clamp_index32(KT::index(KT::readlane(k, i)), kE) < id ? 1 : 0;
  if (lane < kTopK) {
    a.ids[lane] = id;
    a.wts[lane] = wb;
    if (a.ids_out) a.ids_out[lane] = id;
    if (a.wts_out) a.wts_out[lane] = wb;
    a.sel[rank] = id;
    a.selw[rank] = bf16_bits_to_f32(wb);
  }
}

// Decode layer, second kernel: gate_up of one routed slot (W8A8),
// 8 output columns per workgroup: rows n0..n0+7 (gate) and kI+n0.. (up),
// K = kH, after the top-8.  The W8A8 per-group terms (f32(p) * xs_g) * ws_g
// are formed by the lane that owns the partial and summed in ascending group
// order by the epilogue (w8a8.py:40).  The grid is 512 workgroups, two per
// CU; each also computes one column of the shared expert's gate_up + SwiGLU
// (W8A16 on the normalized row), whose inputs do not depend on the routing:
// they are requested behind the logits and consumed while the routed
// weights are in flight.  Workgroup 0 also publishes the routing (ids,
// weights, combine order) after its own work.
__global__ __launch_bounds__(256) void decode_gate_up_kernel(float *p_logits, int8_t *p_xq,
                                                             float *p_xs, uint16_t *p_xn,
                                                             const int8_t *p_gu_q,
                                                             const float *p_gu_s, LayerArgs a) {
  a.logits = p_logits;
  a.xq = p_xq;
  a.xs = p_xs;
  a.xn = p_xn;
  a.gu_q = p_gu_q;
  a.gu_s = p_gu_s;
  constexpr int G = kH / 128;
  constexpr int R = 2 * kGuPairs;
  static_assert(R * G == 256, "one group scale per thread");
  static_assert(kI / kGuPairs * kTopK == kI, "one shared column per workgroup");
  static_assert(kI / kGuPairs == 64 && kTopK == 8, "the XCD deal below");
  __shared__ __align__(16) int8_t xbuf[kH];
  __shared__ __align__(16) uint16_t xb[kH];
  __shared__ float xs[G];
  __shared__ float wsc[R * G];
  __shared__ float term[R * G];
  __shared__ float wsh[2 * G];
  __shared__ float tsh[2 * G];
  const int t = threadIdx.x;
  // Workgroup b runs on XCD x = b % 8.  (slot, column) tiles are dealt out
  // so that the 8 workgroups writing one 128-byte line of a SwiGLU row (64
  // columns), and the 64 writing one line of the shared row, share an XCD.
  const int b = blockIdx.x, x = b & 7, k = b >> 3;
  const int pair = x + 8 * (k >> 3);  // (slot, line) pair: 8 slots x 8 lines
  const int slot = pair >> 3;
  const int n0 = ((pair & 7) * 8 + (k & 7)) * kGuPairs;
  const int nsh = x * 64 + k;  // shared column of this workgroup
  const RowMap map{n0, kI + n0, kGuPairs};
  const RowMap map_sh{nsh, kI + nsh, 1};
  // The logits first, then the quantized activation row, then the shared
  // column's inputs; the routed weights follow as soon as the selection is
  // known.  (Loads complete in issue order, so the selection waits for the
  // logits and the activation row alone.)
  // Every load is issued by every thread from a valid address (only the
  // stores are guarded): a load inside a branch makes the compiler wait for
  // all loads in flight where the branch joins.
  const float v = a.logits[t];
  const float4 f4 = *reinterpret_cast<const float4 *>(a.logits + (t & 63) * 4);
  const float v4[4] = {f4.x, f4.y, f4.z, f4.w};  // for workgroup 0's routing weights
  const u32x4 xv = ldg16(a.xq + (t & (kH / 16 - 1)) * 16);
  const float xsv = a.xs[t & (G - 1)];
  const u32x4 xnv = ldg16(a.xn + t * (kH / 256));
  const int8_t *wq_sh = a.gu_q + (int64_t)kE * a.gu_qes;
  RowLoads<1> Ls;
  Ls.issue(2, G, [&](int r) { return wq_sh + (int64_t)map_sh(r) * kH; });
  const int fs = t & (2 * G - 1);
  const float ssv = a.gu_s[(int64_t)kE * a.gu_ses + (int64_t)map_sh(fs / G) * G + fs % G];
  unsigned long long k64 = 0;
  uint32_t k32 = 0;
  int e;
  if (a.router_bias) {  // biased logits are fp32 values: 64-bit keys
    k64 = decode_top8<Key64>(v);
    e = decode_slot_expert<Key64>(k64, slot);
  } else {  // bf16 logits: 32-bit keys order them identically
    k32 = decode_top8<Key32>(v);
    e = decode_slot_expert<Key32>(k32, slot);
  }
  const int8_t *wq = a.gu_q + (int64_t)e * a.gu_qes;
  const float my_scale = a.gu_s[(int64_t)e * a.gu_ses + (int64_t)map(t / G) * G + t % G];
  RowLoads<8> L;
  L.issue(R, G, [&](int r) { return wq + (int64_t)map(r) * kH; });

  // shared column (its inputs arrived during the selection)
  reinterpret_cast<u32x4 *>(xb)[t] = xnv;
  if (t < 2 * G) wsh[t] = ssv;
  if (t < kH / 16) reinterpret_cast<u32x4 *>(xbuf)[t] = xv;
  if (t < G) xs[t] = xsv;
  __syncthreads();
  const int sub = t & 7;
  Ls.consume([&](u32x4 w, int r, int g, int f, bool ok) {
    uint32_t wd[8];
    dequant16<BF16>(w, wsh[f], wd);
    const uint16_t *xp = xb + g * 128 + sub * 16;
    const float p = octet_sum_f32(dot16_w16<BF16>(wd, *reinterpret_cast<const u32x4 *>(xp),
                                                  *reinterpret_cast<const u32x4 *>(xp + 8)));
    if (ok && sub == 0) tsh[f] = p;
  });
  // The scales of the pairs a wave consumes are the ones its own threads
  // loaded (pair f = thread f), so they are handed over within the wave and
  // no workgroup barrier waits for them.
  wsc[t] = my_scale;
  wave_lds_sync();

  L.consume([&](u32x4 w, int r, int g, int f, bool ok) {
    const int p =
        octet_sum_i32(dot16_i8(w, *reinterpret_cast<const u32x4 *>(xbuf + g * 128 + sub * 16)));
    if (ok && sub == 0) term[f] = mul_rn(mul_rn((float)p, xs[g]), wsc[f]);
  });
  __syncthreads();
  if (t < kGuPairs) {
    float sg = 0.0f, su = 0.0f;
    for (int g = 0; g < G; ++g) {
      sg = add_rn(sg, term[t * G + g]);
      su = add_rn(su, term[(kGuPairs + t) * G + g]);
    }
    const float gate = round_bf16(sg), up = round_bf16(su);
    a.hbuf[slot * kI + n0 + t] = f32_to_bf16_bits(round_bf16(silu_f32(gate)) * up);
    // the fp32 epilogue sums, before the bf16 rounding of w8a8.py:41
    a.dacc_gu[slot * 2 * kI + n0 + t] = sg;
    a.dacc_gu[slot * 2 * kI + kI + n0 + t] = su;
  } else if (t == 64) {  // the shared column, from the terms of all four waves
    float sg = 0.0f, su = 0.0f;
    for (int g = 0; g < G; ++g) {
      sg = add_rn(sg, tsh[g]);
      su = add_rn(su, tsh[G + g]);
    }
    const float gate = round_bf16(sg), up = round_bf16(su);
    a.hbuf[kTopK * kI + nsh] = f32_to_bf16_bits(round_bf16(silu_f32(gate)) * up);
  }
  // Workgroup 0 publishes the routing last: only the down kernel and the
  // caller read it, so no workgroup's weight stream waits for the softmax.
  if (b == 0 && t < 64) {
    if (a.router_bias)
      decode_publish<Key64>(a, k64, v4);
    else
      decode_publish<Key32>(a, k32, v4);
  }
}

// Decode layer, third kernel: down rows of the 8 routed experts and of the
// shared expert for 8 output columns c0 .. c0 + 7 (W8A8 on the row-quantized
// SwiGLU rows / W8A16), then the ascending-expert bf16 combine
// (int8.py:240-250), the gated shared add and the residual add, in place.
// The expert ids are requested first (scalar loads); the small inputs that
// do not depend on them - the routed and shared SwiGLU rows, the shared
// expert's scales, the residual columns, the gate logit - follow at once,
// then the routed scales and weights as soon as the ids land, and last the
// shared expert's weight rows.  The 8 routed SwiGLU rows are quantized per
// row (w8a8.quantize on [8, kI]) in one parallel pass: thread t owns 16
// values of row t / 32.
constexpr int kDnCols = 8;
__global__ __launch_bounds__(256) void decode_down_kernel(int *p_sel, uint16_t *p_hbuf, float *p_selw,
                                                          const int8_t *p_dn_q, const float *p_dn_s,
                                                          uint16_t *p_h, LayerArgs a) {
  a.sel = p_sel;
  a.hbuf = p_hbuf;
  a.selw = p_selw;
  a.dn_q = p_dn_q;
  a.dn_s = p_dn_s;
  a.h = p_h;
  constexpr int G = kI / 128;
  constexpr int RR = kTopK * kDnCols;  // routed rows
  constexpr int R = RR + kDnCols;      // + the shared expert's
  static_assert(RR * G == 256, "one routed group scale per thread");
  static_assert(RR == 64, "the epilogue's per-slot terms fill wave 0");
  __shared__ __align__(16) int8_t xq[kTopK * kI];
  __shared__ float xs[kTopK * G];
  __shared__ __align__(16) uint16_t xsh[kI];
  __shared__ float term[R * G];
  __shared__ float wsc[R * G];
  __shared__ float selw[kTopK];
  __shared__ float prod[RR];
  const int t = threadIdx.x;
  // Workgroup b runs on XCD b % 8; column tiles are dealt out so that the 8
  // workgroups writing one 128-byte line of h (64 columns) share an XCD.
  const int b = blockIdx.x;
  const int c0 = (((b & 7) * 4 + ((b >> 3) >> 3)) * 8 + ((b >> 3) & 7)) * kDnCols;
  int ex[kTopK];
#pragma unroll
  for (int s = 0; s < kTopK; ++s) ex[s] = a.sel[s];
  __builtin_amdgcn_sched_barrier(0);  // the ids are requested before anything else
  // Every load is issued by every thread from a valid address (only the
  // stores are guarded): a load inside a branch makes the compiler wait for
  // all loads in flight where the branch joins.  Loads complete in issue
  // order, so the SwiGLU rows (quantized while the weights stream) and the
  // other small inputs that do not depend on the ids come first, then the
  // routed scales and weights, and last the shared expert's weights.
  const int row = t >> 5, col = (t & 31) * 16;
  const u32x4 h0 = ldg16(a.hbuf + row * kI + col);
  const u32x4 h1 = ldg16(a.hbuf + row * kI + col + 8);
  const float wsel = a.selw[t & (kTopK - 1)];
  const u32x4 hsh = ldg16(a.hbuf + kTopK * kI + (t & (kI / 8 - 1)) * 8);
  const int fs = t & (kDnCols * G - 1);
  const float ssv = a.dn_s[(int64_t)kE * a.dn_ses + (int64_t)(c0 + fs / G) * G + fs % G];
  const uint16_t hres = a.h[c0 + (t & (kDnCols - 1))];
  const float glv = a.gl[0];
  __builtin_amdgcn_sched_barrier(0);  // the inputs above are requested before the weights
  // Routed pairs f = row * G + group: wave w owns pairs 64 w .. 64 w + 63,
  // i.e. the rows of slots 2 w and 2 w + 1, and thread f loads the scale of
  // pair f.
  const int w2 = 2 * __builtin_amdgcn_readfirstlane(t >> 6);
  const int8_t *q_lo = a.dn_q + (int64_t)clamp_index32(ex[w2], kE) * a.dn_qes + (int64_t)c0 * kI;
  const int8_t *q_hi =
      a.dn_q + (int64_t)clamp_index32(ex[w2 + 1], kE) * a.dn_qes + (int64_t)c0 * kI;
  const float *s_own = a.dn_s + (int64_t)clamp_index32(ex[t >> 5], kE) * a.dn_ses +
                       (int64_t)c0 * G;
  const float sv = s_own[t & (kDnCols * G - 1)];
  RowLoads<8> L;
  L.issue(RR, G, [&](int r) {
    return ((r / kDnCols) & 1 ? q_hi : q_lo) + (int64_t)(r % kDnCols) * kI;
  });
  RowLoads<1> Ls;  // the shared expert's 8 rows
  Ls.issue(kDnCols, G, [&](int r) {
    return a.dn_q + (int64_t)kE * a.dn_qes + (int64_t)(c0 + r) * kI;
  });
  __builtin_amdgcn_sched_barrier(0);  // keep the quantization below the weight loads

  // Row quantization of hbuf[0..7]: 16 values per thread, a 128-group is
  // spread over 8 consecutive lanes.
  float v[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = bf16_bits_to_f32(h0[j] & 0xFFFFu);
    v[2 * j + 1] = bf16_bits_to_f32(h0[j] >> 16);
    v[8 + 2 * j] = bf16_bits_to_f32(h1[j] & 0xFFFFu);
    v[8 + 2 * j + 1] = bf16_bits_to_f32(h1[j] >> 16);
  }
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) am = fmaxf(am, fabsf(v[j]));
  am = fmaxf(am, __uint_as_float(lane_xor<1>(__float_as_uint(am))));
  am = fmaxf(am, __uint_as_float(lane_xor<2>(__float_as_uint(am))));
  am = fmaxf(am, __uint_as_float(lane_xor<4>(__float_as_uint(am))));
  const float sc = fmaxf(am, 1e-10f) * (float)(1.0 / 127.0);
  const float rs = 1.0f / sc;
  u32x4 packed;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t pk = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pk |= ((uint32_t)(uint8_t)(int8_t)(int)rintf(quant_div(v[4 * j + i], sc, rs))) << (8 * i);
    packed[j] = pk;
  }
  *reinterpret_cast<u32x4 *>(xq + row * kI + col) = packed;
  if ((t & 7) == 0) xs[row * G + col / 128] = sc;
  if (t < kTopK) selw[t] = wsel;
  if (t < kDnCols * G) wsc[RR * G + t] = ssv;
  if (t < kI / 8) reinterpret_cast<u32x4 *>(xsh)[t] = hsh;
  __syncthreads();

  // The routed scales of the pairs a wave consumes are the ones its own
  // threads loaded (pair f = thread f): a wave-local hand-off, so the
  // workgroup barrier above did not wait for them.
  wsc[t] = sv;
  wave_lds_sync();
  const int sub = t & 7;
  L.consume([&](u32x4 w, int r, int g, int f, bool ok) {
    const int s = r / kDnCols;  // uniform across the wave instruction
    const int p = octet_sum_i32(
        dot16_i8(w, *reinterpret_cast<const u32x4 *>(xq + s * kI + g * 128 + sub * 16)));
    if (ok && sub == 0) term[f] = mul_rn(mul_rn((float)p, xs[s * G + g]), wsc[f]);
  });
  Ls.consume([&](u32x4 w, int r, int g, int f, bool ok) {
    uint32_t wd[8];
    dequant16<BF16>(w, wsc[RR * G + f], wd);
    const uint16_t *xp = xsh + g * 128 + sub * 16;
    const float p = octet_sum_f32(dot16_w16<BF16>(wd, *reinterpret_cast<const u32x4 *>(xp),
                                                  *reinterpret_cast<const u32x4 *>(xp + 8)));
    if (ok && sub == 0) term[RR * G + f] = p;
  });
  __syncthreads();
  // Epilogue in wave 0.  Lane r = s * kDnCols + c forms slot s's weighted
  // term bf16(bf16(row sum) * w_s) of column c, which does not depend on the
  // running sum; lanes 0 .. kDnCols - 1 then add the 8 terms in ascending
  // slot order with a bf16 rounding after each add (int8.py:240-250), and the
  // gated shared term.
  if (t < RR) {
    const int c = t & (kDnCols - 1);
    float v8 = 0.0f;
    for (int g = 0; g < G; ++g) v8 = add_rn(v8, term[t * G + g]);
    const float vr = round_bf16(v8);
    prod[t] = round_bf16(vr * selw[t / kDnCols]);
    float vs = 0.0f;
    for (int g = 0; g < G; ++g) vs += term[(RR + c) * G + g];
    const float shared = round_bf16(round_bf16(sigmoid_f32(glv)) * round_bf16(vs));
    // The layer's intermediates stay in the workspace: slot s's down row
    // (bf16 and its fp32 epilogue sum) and, from lanes 0 .. 7, the shared one.
    const int s = t / kDnCols;
    a.vbuf[s * kH + c0 + c] = f32_to_bf16_bits(vr);
    a.dacc_dn[s * kH + c0 + c] = v8;
    if (t < kDnCols) a.vbuf[kTopK * kH + c0 + c] = f32_to_bf16_bits(vs);
    wave_lds_sync();
    if (t < kDnCols) {
      float acc = 0.0f;
#pragma unroll
      for (int s = 0; s < kTopK; ++s) acc = round_bf16(acc + prod[s * kDnCols + t]);
      const float out = round_bf16(acc + shared);
      a.h[c0 + t] = f32_to_bf16_bits(bf16_bits_to_f32(hres) + out);
    }
  }
}

// ------------------------------------------------------------------ prefill
// RMSNorm of each token row + the shared-expert gate logit (fp64 dot) + the
// Euclidean norms that bound the approximate router logits: |xn| of each
// token (workgroups < T) and |w_e| of each router row (workgroups < kE).
// Leading pointer arguments: preloaded into SGPRs at launch, as in the decode
// kernels.
//
// The norm |w_e| of router row e (thread t holds its values 8 t .. 8 t + 7 in
// wv), for the prefill router's error bound; red2 is reused.
__device__ __forceinline__ void router_row_norm(u32x4 wv, float *nw_out, float *red2) {
  const int t = threadIdx.x;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = bf16_bits_to_f32(wv[j] & 0xFFFFu), hi = bf16_bits_to_f32(wv[j] >> 16);
    ss += lo * lo + hi * hi;
  }
  ss = wave_sum_f32(ss);
  __syncthreads();  // red2 is free again
  if ((t & 63) == 0) red2[t >> 6] = ss;
  __syncthreads();
  if (t == 0) *nw_out = sqrtf((red2[0] + red2[1]) + (red2[2] + red2[3]));
}

// The prefill norm work of token `tok` for the layer whose norm and gate
// weights `a` holds (nwv, gv: thread t's norm weights and gate values
// 8 t .. 8 t + 7): RMSNorm of the row (thread t holds its bf16 values
// 8 t .. 8 t + 7 in raw) into xn, the row's Euclidean norm nx, the
// shared-gate logit gl (fp64 dot) and, when a.xh is set, the fp16 copy of the
// row for the gate_up GEMM on fp16 tiles with its power of two xk.
__device__ __forceinline__ void prefill_norm_token(u32x4 raw, const NormW &nwv, u32x4 gv,
                                                   const LayerArgs &a, int tok, float *red,
                                                   float *red2, double *dred) {
  const int t = threadIdx.x;
  constexpr int PER = kH / 256;
  // the normalized values stay in the thread's registers: every use below
  // reads the thread's own values (no LDS copy, no barrier for it)
  float y[PER];
  norm_row(raw, nwv, a.eps, red, y);
  {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss += y[j] * y[j];
    ss = wave_sum_f32(ss);
    if ((t & 63) == 0) red2[t >> 6] = ss;
  }
  u32x4 packed;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    packed[j] = BF16::pack2(y[2 * j], y[2 * j + 1]);
  *reinterpret_cast<u32x4 *>(a.xn + (int64_t)tok * kH + t * PER) = packed;
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc = __builtin_fma((double)y[2 * j], (double)bf16_bits_to_f32(gv[j] & 0xFFFFu), acc);
    acc = __builtin_fma((double)y[2 * j + 1], (double)bf16_bits_to_f32(gv[j] >> 16), acc);
  }
  acc = wave_sum_f64_dpp(acc);
  if ((t & 63) == 0) dred[t >> 6] = acc;
  __syncthreads();
  const float nxt = sqrtf((red2[0] + red2[1]) + (red2[2] + red2[3]));
  if (t == 0) {
    a.gl[tok] = round_bf16((float)(dred[0] + dred[1] + dred[2] + dred[3]));
    a.nx[tok] = nxt;
  }
  // The fp16 copy of the row for the gate_up GEMM on fp16 tiles (xh is null
  // otherwise): xn * 2^k with the row's Euclidean norm (which bounds every
  // |value|) in [2^14, 2^15).  A bf16 value with |v| 2^k >= 2^-17 is exact in
  // fp16; smaller ones (below 2^-31 of the norm) round to the fp16 subnormal
  // grid.
  if (a.xh) {
    int ex = 0;
    (void)frexpf(nxt, &ex);
    const int k = nxt > 0.0f ? min(max(15 - ex, -126), 126) : 0;
    u32x4 hp;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f16x2 v;
      v.x = (_Float16)ldexpf(y[2 * j], k);
      v.y = (_Float16)ldexpf(y[2 * j + 1], k);
      hp[j] = __builtin_bit_cast(uint32_t, v);
    }
    *reinterpret_cast<u32x4 *>(a.xh + (int64_t)tok * kH + t * PER) = hp;
    if (t == 0) a.xk[tok] = k;
  }
}

__global__ __launch_bounds__(256) void prefill_norm_gate_kernel(uint16_t *p_h, const uint16_t *p_router_w,
                                                                const uint16_t *p_gate_w,
                                                                const float *p_norm_w, int T,
                                                                LayerArgs a) {
  a.h = p_h;
  a.router_w = p_router_w;
  a.gate_w = p_gate_w;
  a.norm_w = p_norm_w;
  __shared__ float red[4];
  __shared__ float red2[4];
  __shared__ double dred[4];
  const int tok = blockIdx.x;
  const int t = threadIdx.x;
  constexpr int PER = kH / 256;
  // Both weight rows are requested at entry, ahead of the token's row, so
  // their latency overlaps the RMSNorm; the router-row norm (blocks < E) is
  // finished after the token's work, which it must not delay.
  const u32x4 wv = tok < kE ? ldg16(a.router_w + (int64_t)tok * kH + t * PER)
                            : u32x4{0u, 0u, 0u, 0u};
  const u32x4 gv = ldg16(a.gate_w + t * PER);
  const NormW nwv = load_norm_w(a.norm_w);
  if (tok >= T) {
    if (tok < kE) router_row_norm(wv, a.nw + tok, red2);
    return;
  }
  prefill_norm_token(ldg16(a.h + (int64_t)tok * kH + t * PER), nwv, gv, a, tok, red, red2, dred);
  if (tok < kE) router_row_norm(wv, a.nw + tok, red2);
}

// Approximate router logits of the prefill tokens: bf16 MFMA with fp32
// sums (neither rounded to bf16 nor biased).  A workgroup owns 32 tokens x
// 64 experts; its four waves each take one quarter of K for the whole tile
// (2 x 4 MFMA tiles, so every fragment read feeds two or four MFMAs) and the
// quarters are summed through LDS at the end.  K is streamed
// in 128-wide segments with coalesced loads: a wave load covers 4 whole
// 256-byte row segments, one row per quarter-wave (a load in the MFMA
// operand layout would touch 16 rows 4 KB apart per quarter-wave and keep
// the address path stalled).  The segments go through the wave's own LDS
// region (pitch 272 B, so the 16 rows of a fragment read fall in distinct
// banks) and are read back in the MFMA layout; the next segment's loads are
// in flight meanwhile.  Every MFMA sums its 32 products from zero and its
// result is added to the wave's fp32 sum; prefill_topk_count_kernel's error
// bound counts the roundings of exactly this scheme (31 + 15 + 3).
constexpr int kRaTok = 32, kRaExp = 64;
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void
router_approx_kernel(uint16_t *p_xn, const uint16_t *p_router_w, float *p_logits, int T, LayerArgs a) {
  a.xn = p_xn;
  a.router_w = p_router_w;
  a.logits = p_logits;
  constexpr int KQ = kH / 4;
  constexpr int SS = 128, NSS = KQ / SS, PITCH = 272;
  constexpr int NLD = (kRaTok + kRaExp) / 4;  // wave loads per segment: 8 token + 16 expert
  static_assert(KQ % SS == 0 && kE % kRaExp == 0 && kRaTok == 32 && kRaExp == 64, "router tiling");
  __shared__ f32x4 part[3][8][64];
  __shared__ __align__(16) unsigned char stg[4][(kRaTok + kRaExp) * PITCH];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int t0 = blockIdx.x * kRaTok;
  const int e0 = blockIdx.y * kRaExp;
  unsigned char *my = stg[wave];
  // wave load j: staging rows 4 j .. 4 j + 3 (0..31 tokens, 32..95 experts),
  // row 4 j + lane / 16, values 8 (lane % 16) .. + 7 of the segment
  const int lr = lane >> 4, lc = lane & 15;
  const uint16_t *src[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    src[j] = j < kRaTok / 4 ? a.xn + (int64_t)min(t0 + 4 * j + lr, T - 1) * kH
                            : a.router_w + (int64_t)(e0 + 4 * (j - kRaTok / 4) + lr) * kH;
    src[j] += wave * KQ + lc * 8;
  }
  f32x4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 rg[NLD];
  auto gload = [&](int ss) {
#pragma unroll
    for (int j = 0; j < NLD; ++j) rg[j] = ldg16(src[j] + ss * SS);
  };
  gload(0);
  for (int ss = 0; ss < NSS; ++ss) {
#pragma unroll
    for (int j = 0; j < NLD; ++j)
      *reinterpret_cast<u32x4 *>(my + (4 * j + lr) * PITCH + lc * 16) = rg[j];
    // the segment is read across lanes: every lane's stores come first
    wave_lds_sync();
    if (ss + 1 < NSS) gload(ss + 1);
#pragma unroll
    for (int st = 0; st < SS / 32; ++st) {  // 32-wide MFMA steps: values 32 st + 8 q .. + 7
      u32x4 av[2], bv[4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        av[i] = *reinterpret_cast<const u32x4 *>(my + (16 * i + r) * PITCH + st * 64 + q * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bv[j] = *reinterpret_cast<const u32x4 *>(my + (kRaTok + 16 * j + r) * PITCH + st * 64 +
                                                 q * 16);
      // each MFMA sums its 32 products from zero; its result is added to
      // the running fp32 sum, which bounds the roundings a product passes
      // through by 31 + 15 + 3 (see topk_exact_wave)
      // (all eight MFMAs issue before the first add reads a result)
      f32x4 pr[2][4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pr[i][j] = BF16::mfma16x16x32(av[i], bv[j], f32x4{0.f, 0.f, 0.f, 0.f});
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] + pr[i][j];
    }
    wave_lds_sync();  // every lane's reads before the next segment is stored
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) part[wave - 1][4 * i + j][lane] = acc[i][j];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 v = acc[i][j] + part[0][4 * i + j][lane] + part[1][4 * i + j][lane] +
                      part[2][4 * i + j][lane];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int t = t0 + 16 * i + 4 * q + m;
        if (t < T) a.logits[(int64_t)t * kE + e0 + 16 * j + r] = v[m];
      }
    }
}

// Exact top-8 of one prefill token (one wave) from the approximate logits.
// An approximate logit A is the fp32 sum of the exactly representable
// bf16 x bf16 products: each MFMA of router_approx_kernel sums 32 of them
// from zero (at most 31 roundings in any order), its result joins the
// wave's running sum of 16 MFMAs (15 roundings) and the four waves' sums
// are added (3), so a product passes through at most 49 roundings and
// |A - S| <= 49 2^-23 sum_k |x_k w_ek| <= 49 2^-23 |x| |w_e| <= 2^-17 |x| |w_e| / 1.3
// for the exact dot product S (Cauchy-Schwarz; the 30% absorbs the second-
// order terms, the fp64 error of the exact dot products and the rounding
// of the norms and of eps).  Rounding to bf16 and adding the bias are
// monotone, so the exact logit round_bf16(S) (+ bias) lies in
// [lo, hi] = [round_bf16(A - eps), round_bf16(A + eps)] (+ bias).  With T8
// the 8th largest lower-bound key, an expert whose upper-bound key is below
// T8 is beaten by 8 experts whatever its exact logit is; every other expert
// is a candidate.  A candidate with lo == hi has that exact logit already,
// and so has round_bf16(A) (+ bias), which lies between them; only the
// others (lo < hi: A within eps of a bf16 rounding boundary, a few percent
// of the candidates) get their exact logit from an fp64 dot product, the
// same value router_logits computes.  The selection and softmax then run on
// exact logits for the candidates and rounded approximate ones elsewhere,
// which can only enter the softmax denominator.
template <class KT>
__device__ void topk_exact_wave(const LayerArgs &a, int tok, int lane, unsigned long long *scratch,
                                float *lv, int *cand, int *amb, int64_t *ids_out,
                                uint16_t *w_out) {
  using T = typename KT::T;
  u32x4 xv[4];  // the token's row, loaded only when a candidate is open
  const float4 av = *reinterpret_cast<const float4 *>(a.logits + (int64_t)tok * kE + lane * 4);
  const float4 nv = *reinterpret_cast<const float4 *>(a.nw + lane * 4);
  const float nx = a.nx[tok];
  const float A[4] = {av.x, av.y, av.z, av.w};
  const float NW[4] = {nv.x, nv.y, nv.z, nv.w};
  float lo[4], hi[4];
  T klo[4], khi[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane * 4 + j;
    const float eps = 0x1.0p-17f * (nx * NW[j]) + 1e-30f;
    lo[j] = round_bf16(A[j] - eps);
    hi[j] = round_bf16(A[j] + eps);
    float ap = round_bf16(A[j]);
    if (a.router_bias) {
      const float b = a.router_bias[e];
      lo[j] = lo[j] + b;
      hi[j] = hi[j] + b;
      ap = ap + b;
    }
    lv[e] = ap;
    klo[j] = KT::make(lo[j], e);
    khi[j] = KT::make(hi[j], e);
  }
  static_assert(kTopK == 8, "T8 is the 8th largest lower-bound key");
  const T t8 = kth8_key_wave<KT>(klo, lane);
  // candidates, compacted into cand[0 .. n); the ones whose exact logit
  // the bounds leave open (lo != hi, also when either is NaN) into
  // amb[0 .. na)
  int n = 0, na = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool c = khi[j] >= t8;
    const unsigned long long m = __ballot(c);
    const int before = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (c) cand[n + before] = lane * 4 + j;
    n += __popcll(m);
    const bool o = c && !(lo[j] == hi[j]);
    const unsigned long long mo = __ballot(o);
    const int bo = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mo >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)mo, 0u));
    if (o) amb[na + bo] = lane * 4 + j;
    na += __popcll(mo);
  }
  wave_lds_sync();
  // exact logits of the open candidates, CB per batch, the next batch's
  // rows requested before the current batch is reduced: lane holds x[k]
  // and w[k] for k = 8 lane + 512 i + (0..7)
  constexpr int CB = 3;
  u32x4 wv[2][CB][4];
  int ec[2][CB];
  auto fetch = [&](int buf, int c0) {
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      ec[buf][b] = amb[min(c0 + b, na - 1)];
      const uint16_t *wr = a.router_w + (int64_t)ec[buf][b] * kH + lane * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[buf][b][i] = ldg16(wr + 512 * i);
    }
  };
  auto reduce = [&](int buf, int c0) {
    double acc[CB];
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      acc[b] = 0.0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[b] = __builtin_fma((double)bf16_bits_to_f32(xv[i][j] & 0xFFFFu),
                                 (double)bf16_bits_to_f32(wv[buf][b][i][j] & 0xFFFFu), acc[b]);
          acc[b] = __builtin_fma((double)bf16_bits_to_f32(xv[i][j] >> 16),
                                 (double)bf16_bits_to_f32(wv[buf][b][i][j] >> 16), acc[b]);
        }
    }
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      const double sum = wave_sum_f64_dpp(acc[b]);
      if (lane == 0 && c0 + b < na) {
        float l = round_bf16((float)sum);
        if (a.router_bias) l = l + a.router_bias[ec[buf][b]];
        lv[ec[buf][b]] = l;
      }
    }
  };
  if (na > 0) {
    const uint16_t *xr = a.xn + (int64_t)tok * kH + lane * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[i] = ldg16(xr + 512 * i);
    fetch(0, 0);
  }
  for (int c0 = 0; c0 < na; c0 += 2 * CB) {
    if (c0 + CB < na) fetch(1, c0 + CB);
    reduce(0, c0);
    if (c0 + 2 * CB < na) fetch(0, c0 + 2 * CB);
    if (c0 + CB < na) reduce(1, c0 + CB);
  }
  wave_lds_sync();
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = lv[lane * 4 + j];
  if (n > 64) {  // more candidates than lanes: the full top-k over lv
    topk_wave_v(v, kE, kTopK, lane, scratch, ids_out, w_out);
    return;
  }
  // Selection among the candidates (lane c holds candidate c); every
  // non-candidate ranks below 8 candidates.  The softmax follows
  // topk_wave_keys operation for operation, so the result is the one the
  // full top-k over lv gives.
  T *keys = reinterpret_cast<T *>(scratch);
  const bool has = lane < n;
  const int ce = has ? cand[lane] : 0;
  const float cv = has ? lv[ce] : 0.0f;
  const T ck = has ? KT::make(cv, ce) : (T)0;
  keys[lane] = ck;
  wave_lds_sync();
  int rank = 0;
  for (int c = 0; c < n; ++c) rank += keys[c] > ck ? 1 : 0;
  const unsigned long long first = __ballot(has && rank == 0);
  const float mx = __int_as_float(__builtin_amdgcn_readlane(
      __float_as_int(KT::value(ck)), (int)__builtin_ctzll(first)));
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) part += expf(v[j] - mx);
  part = row_sum_f32(part);
  const float denom = (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 0)) +
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 16))) +
                      (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 32)) +
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 48)));
  float *prob = reinterpret_cast<float *>(scratch + 64);
  const bool chosen = has && rank < kTopK;
  const float pe = expf(KT::value(ck) - mx) / denom;
  if (chosen) prob[rank] = pe;
  wave_lds_sync();
  float psum = 0.0f;
#pragma unroll
  for (int i = 0; i < kTopK; ++i) psum += prob[i];
  if (chosen) {
    ids_out[rank] = ce;
    w_out[rank] = f32_to_bf16_bits(pe / psum);
  }
}

// Top-k of every prefill token (one wave per token, kTopkTokens tokens per
// workgroup) that also ranks each route among the workgroup's routes to the
// same expert (LDS atomics) and writes the workgroup's per-expert counts as
// one row of bcounts [workgroups, kE].  No global atomics: the row of a
// route in the expert-sorted order is fixed later from column prefixes of
// bcounts.  Rows of one expert are in no particular order - the grouped
// GEMMs compute every row independently and the combine walks a token's
// routes in ascending expert id, so the layer output does not depend on it.
constexpr int kScanRoutes = 1024;  // routes per prefill_scan_kernel workgroup
constexpr int kScanGroups = kScanRoutes / (kTopkTokens * kTopK);  // top-k workgroups per scan one
static_assert(kScanGroups * kTopkTokens * kTopK == kScanRoutes, "scan slices whole top-k groups");

__global__ __launch_bounds__(kTopkTokens * 64) void prefill_topk_count_kernel(
    int T, const float *p_router_bias, uint16_t *p_xn, float *p_logits, float *p_nw, float *p_nx,
    LayerArgs a, uint8_t *bcounts, int *rslot) {
  a.router_bias = p_router_bias;
  a.xn = p_xn;
  a.logits = p_logits;
  a.nw = p_nw;
  a.nx = p_nx;
  __shared__ int lcnt[kE];
  __shared__ int64_t sid[kTopkTokens][kTopK];
  __shared__ uint16_t swt[kTopkTokens][kTopK];
  __shared__ unsigned long long scratch[kTopkTokens][kTopkScratch];
  __shared__ float lv[kTopkTokens][kE];
  __shared__ int cand[kTopkTokens][kE];
  __shared__ int amb[kTopkTokens][kE];
  static_assert(kTopkTokens * 64 >= kE, "one thread per expert count");
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;
  if (t < kE) lcnt[t] = 0;
  __syncthreads();
  const int tok = blockIdx.x * kTopkTokens + w;
  int e = -1, rank = 0;
  if (tok < T) {  // wave-uniform
    if (a.router_bias)
      topk_exact_wave<Key64>(a, tok, lane, scratch[w], lv[w], cand[w], amb[w], sid[w], swt[w]);
    else
      topk_exact_wave<Key32>(a, tok, lane, scratch[w], lv[w], cand[w], amb[w], sid[w], swt[w]);
    wave_lds_sync();
    if (lane < kTopK) {
      e = (int)clamp_index(sid[w][lane], kE);
      a.ids[(int64_t)tok * kTopK + lane] = e;
      a.wts[(int64_t)tok * kTopK + lane] = swt[w][lane];
      rank = atomicAdd(&lcnt[e], 1);
    }
  }
  __syncthreads();
  // a count is at most kTopkTokens * kTopK = 64 routes: one byte
  if (t < kE) bcounts[(int64_t)blockIdx.x * kE + t] = (uint8_t)lcnt[t];
  if (e >= 0) rslot[(int64_t)tok * kTopK + lane] = rank;
}

// Expert offsets and, for each route, its row in the expert-sorted order:
// offs[e] + (routes to e of earlier top-k workgroups) + rank inside its own
// workgroup.  Each workgroup handles kScanRoutes routes and sums the bcounts
// columns itself (nb rows of kE byte counts, 64 KB for 2048 tokens), so no
// grid-wide step is needed.  Workgroup 0 also writes the tile table (the
// shared expert's tiles over rows [R, R + T), then kBM-row tiles per routed
// expert, then surplus rows (0, 0, 0)) and the shared rows' tokens.  Every
// route's token also goes to the tile-major gather map ptile (row r of
// table tile i at i * kBM + r; every workgroup scans the tile counts), which
// the gate_up GEMM reads together with its table row rather than after it.
//
// Every load of a phase is issued unconditionally (clamped rows), so the
// phase pays one load latency, not one per row.
__global__ __launch_bounds__(1024) void prefill_scan_kernel(const int64_t *__restrict__ ids,
                                                            const int *__restrict__ rslot,
                                                            const uint8_t *__restrict__ bcounts,
                                                            int nb, int T, int max_tiles,
                                                            int64_t *__restrict__ pos,
                                                            int64_t *__restrict__ table,
                                                            int *__restrict__ ptile,
                                                            int *__restrict__ rpos) {
  constexpr int Q = 16;  // row phases: wave q sums rows q, q + Q, ...
  static_assert(kE == 4 * 64, "a lane sums 4 experts' byte counts");
  __shared__ int ptot[Q][kE], ppre[Q][kE], bpre[kScanGroups][kE];
  __shared__ int offs[kE + 1], toffs[kE], scratch[4], tscratch[4];
  const int t = threadIdx.x;
  const int R = T * kTopK;
  const int r = blockIdx.x * kScanRoutes + t;
  const int e_r = r < R ? (int)clamp_index(ids[r], kE) : 0;
  const int s_r = r < R ? rslot[r] : 0;
  const int j0 = blockIdx.x * kScanGroups;
  {
    const int l = t & 63, q = t >> 6;
    int tot[4] = {0, 0, 0, 0}, pre[4] = {0, 0, 0, 0};
#pragma unroll 16
    for (int j = q; j < nb; j += Q) {
      const uint32_t v = *reinterpret_cast<const uint32_t *>(bcounts + (int64_t)j * kE + 4 * l);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = (int)((v >> (8 * i)) & 0xFFu);
        tot[i] += c;
        pre[i] += j < j0 ? c : 0;
      }
    }
    *reinterpret_cast<int4 *>(&ptot[q][4 * l]) = int4{tot[0], tot[1], tot[2], tot[3]};
    *reinterpret_cast<int4 *>(&ppre[q][4 * l]) = int4{pre[0], pre[1], pre[2], pre[3]};
  }
  // this workgroup's own kScanGroups rows, requested before the barrier
  int cj[kScanGroups];
#pragma unroll
  for (int j = 0; j < kScanGroups; ++j)
    cj[j] = bcounts[(int64_t)min(j0 + j, nb - 1) * kE + (t & (kE - 1))];
  __syncthreads();
  int c = 0;
  if (t < kE) {
    int p = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      c += ptot[q][t];
      p += ppre[q][t];
    }
#pragma unroll
    for (int j = 0; j < kScanGroups; ++j) {
      bpre[j][t] = p;
      p += (j0 + j < nb) ? cj[j] : 0;
    }
  }
  // Exclusive prefix sums over the kE experts (threads 0 .. kE - 1, the
  // first four waves) of the route counts c and the tile counts nt, in one
  // pass: wave-level shuffle scans, then the four wave totals through LDS.
  // tiles: the shared expert's nst first, then expert e's nt at nst + tex
  const int nst = (T + kBM - 1) / kBM;
  const int nt = t < kE ? (c + kBM - 1) / kBM : 0;
  int ex, tex, all, ntot;
  {
    const int ln = t & 63, wave = t >> 6;
    int incl = c, tincl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o, 64), tu = __shfl_up(tincl, o, 64);
      if (ln >= o) {
        incl += u;
        tincl += tu;
      }
    }
    if (ln == 63 && wave < 4) {
      scratch[wave] = incl;
      tscratch[wave] = tincl;
    }
    __syncthreads();
    int base = 0, tbase = 0;
    for (int i = 0; i < wave && i < 4; ++i) {
      base += scratch[i];
      tbase += tscratch[i];
    }
    all = scratch[0] + scratch[1] + scratch[2] + scratch[3];
    ntot = tscratch[0] + tscratch[1] + tscratch[2] + tscratch[3];
    ex = base + incl - c;
    tex = tbase + tincl - nt;
  }
  if (t < kE) {
    offs[t] = ex;
    toffs[t] = tex;
  }
  if (t == 0) offs[kE] = all;
  __syncthreads();
  if (r < R) {
    const int jb = r / (kTopkTokens * kTopK) - j0;
    const int p = clamp_index32(offs[e_r] + bpre[jb][e_r] + s_r, R);
    pos[p] = r / kTopK;
    rpos[r] = p;
    const int q = max(p - offs[e_r], 0);  // rank among the expert's routes
    const int tile = clamp_index32(nst + toffs[e_r] + q / kBM, nst + max_tiles);
    ptile[(int64_t)tile * kBM + q % kBM] = r / kTopK;
  }
  if (blockIdx.x != 0) return;
  // Tile table: the shared expert's nst full tiles over rows [R, R + T)
  // first (the longest tiles start first), then thread e writes the tiles of
  // routed expert e at nst + its exclusive tile prefix, and rows past the
  // last tile up to nst + max_tiles are (0, 0, 0).
  for (int k = 0; k < nt; ++k) {
    const int64_t i = nst + tex + k;
    table[i * 3] = t;
    table[i * 3 + 1] = offs[t] + (int64_t)k * kBM;
    table[i * 3 + 2] = offs[t + 1];
  }
  for (int i = nst + ntot + t; i < nst + max_tiles; i += 1024) {
    table[(int64_t)i * 3] = 0;
    table[(int64_t)i * 3 + 1] = 0;
    table[(int64_t)i * 3 + 2] = 0;
  }
  for (int j = t; j < nst; j += 1024) {
    table[(int64_t)j * 3] = kE;
    table[(int64_t)j * 3 + 1] = R + (int64_t)j * kBM;
    table[(int64_t)j * 3 + 2] = R + T;
  }
  for (int tok = t; tok < T; tok += 1024) {
    pos[R + tok] = tok;
    ptile[tok] = tok;  // shared tile j, row r: token j * kBM + r
  }
}

// The next layer of a chained prefill call: its weights for the norm work
// that the combine does on the rows it has just written.
struct NextLayer {
  const uint16_t *router_w;
  const uint16_t *gate_w;
  const float *norm_w;
  uint16_t *xh;  // the fp16 row copy, when the next gate_up runs on fp16 tiles
};

// Per token: routed combine in ascending expert order, gated shared add,
// residual add (in place on h).  256 threads x 8 columns.  With NEXT the
// same workgroup then does the next layer's norm work on the new row
// (prefill_norm_token, the norm kernel's code and order, so the next layer
// sees the same normalized rows, gate logits and fp16 copies as from its own
// norm kernel) and workgroups < E the norms of the next router's rows; the
// grid is then max(T, E) workgroups.
template <bool NEXT>
__global__ __launch_bounds__(256) void prefill_combine_kernel(int64_t *p_ids, const int *rpos,
                                                              uint16_t *p_wts, const uint16_t *vbuf,
                                                              int64_t R, int T, LayerArgs a,
                                                              NextLayer nx) {
  a.ids = p_ids;
  a.wts = p_wts;
  const int tok = blockIdx.x;
  const int c = threadIdx.x * 8;
  __shared__ float red[4], red2[4];
  __shared__ double dred[4];
  // the next layer's weights, requested first (their latency overlaps the combine)
  u32x4 wv{0u, 0u, 0u, 0u}, gv{0u, 0u, 0u, 0u};
  NormW nwv{};
  if constexpr (NEXT) {
    if (tok < kE) wv = ldg16(nx.router_w + (int64_t)tok * kH + c);
    gv = ldg16(nx.gate_w + c);
    nwv = load_norm_w(nx.norm_w);
    if (tok >= T) {
      router_row_norm(wv, a.nw + tok, red2);
      return;
    }
  }
  int e[kTopK], p[kTopK];
  float w[kTopK];
#pragma unroll
  for (int i = 0; i < kTopK; ++i) {
    e[i] = (int)clamp_index(a.ids[(int64_t)tok * kTopK + i], kE);
    p[i] = clamp_index32(rpos[(int64_t)tok * kTopK + i], (int)R);
    w[i] = bf16_bits_to_f32(a.wts[(int64_t)tok * kTopK + i]);
  }
#pragma unroll
  for (int pass = 0; pass < kTopK; ++pass) {  // ascending expert id (ids are distinct)
#pragma unroll
    for (int i = pass & 1; i + 1 < kTopK; i += 2) {
      if (e[i] > e[i + 1]) {
        const int te = e[i], tp = p[i];
        const float tw = w[i];
        e[i] = e[i + 1];
        p[i] = p[i + 1];
        w[i] = w[i + 1];
        e[i + 1] = te;
        p[i + 1] = tp;
        w[i + 1] = tw;
      }
    }
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kTopK; ++i) {
    const u32x4 v = ldg16(vbuf + (int64_t)p[i] * kH + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = round_bf16(acc[2 * j] + round_bf16(bf16_bits_to_f32(v[j] & 0xFFFFu) * w[i]));
      acc[2 * j + 1] =
          round_bf16(acc[2 * j + 1] + round_bf16(bf16_bits_to_f32(v[j] >> 16) * w[i]));
    }
  }
  const float sig = round_bf16(sigmoid_f32(a.gl[tok]));
  const u32x4 sv = ldg16(vbuf + (R + tok) * kH + c);
  uint16_t *hp = a.h + (int64_t)tok * kH + c;
  const u32x4 hv = ldg16(hp);
  u32x4 outv;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float o0 = round_bf16(acc[2 * j] + round_bf16(sig * bf16_bits_to_f32(sv[j] & 0xFFFFu)));
    float o1 = round_bf16(acc[2 * j + 1] + round_bf16(sig * bf16_bits_to_f32(sv[j] >> 16)));
    o0 = bf16_bits_to_f32(hv[j] & 0xFFFFu) + o0;
    o1 = bf16_bits_to_f32(hv[j] >> 16) + o1;
    outv[j] = BF16::pack2(o0, o1);
  }
  *reinterpret_cast<u32x4 *>(hp) = outv;
  if constexpr (NEXT) {
    // every thread has read this layer's gate logit (sig) before the
    // barriers inside, after which thread 0 overwrites it with the next one
    LayerArgs b = a;
    b.norm_w = nx.norm_w;
    b.gate_w = nx.gate_w;
    b.xh = nx.xh;
    prefill_norm_token(outv, nwv, gv, b, tok, red, red2, dred);
    if (tok < kE) router_row_norm(wv, a.nw + tok, red2);
  }
}

__global__ void export_routing_kernel(const int64_t *ids, const uint16_t *wts, int32_t *ids_out,
                                      uint16_t *wts_out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (ids_out) ids_out[i] = (int32_t)ids[i];
  if (wts_out) wts_out[i] = wts[i];
}

// Zeroes n bytes (n a multiple of 4) with a grid-stride loop of dword stores.
__global__ void fill_zero_kernel(uint32_t *p, int64_t n) {
  const int64_t words = n >> 2;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * 256)
    p[i] = 0u;
}

}  // namespace lm

using namespace lm;

extern "C" int64_t lm_moe_workspace_bytes(int64_t max_tokens, int64_t hidden, int64_t inter,
                                          int64_t experts, int64_t top_k) {
  if (hidden != kH || inter != kI || experts != kE || top_k != kTopK || max_tokens < 1) return -1;
  return layout(max_tokens).total;
}

extern "C" int lm_moe_workspace_region(int64_t tokens, int region, int64_t *offset,
                                       int64_t *bytes) {
  LM_REQUIRE(tokens >= 1 && tokens <= 65536, LM_EINVAL, "invalid token count");
  LM_REQUIRE(offset && bytes, LM_EINVAL, "null pointer");
  const WsLayout w = layout(tokens);
  const int64_t T = tokens, R = T * kTopK;
  const bool decode = T == 1;
  switch (region) {
    case LM_WS_NORMED: *offset = w.xn; *bytes = T * kH * 2; break;
    case LM_WS_GATE: *offset = w.gl; *bytes = T * 4; break;
    case LM_WS_IDS: *offset = w.ids; *bytes = R * 8; break;
    case LM_WS_WEIGHTS: *offset = w.wts; *bytes = R * 2; break;
    case LM_WS_ROUTE_ROWS:
      LM_REQUIRE(!decode, LM_EINVAL, "a decode call has no route rows");
      *offset = w.rpos; *bytes = R * 4; break;
    case LM_WS_ROUTER_APPROX:
    case LM_WS_ROW_NORMS:
    case LM_WS_ROUTER_NORMS:
      LM_REQUIRE(!decode, LM_EINVAL, "region written by prefill calls (tokens > 1) only");
      if (region == LM_WS_ROUTER_APPROX) {
        *offset = w.logits; *bytes = T * kE * 4;
      } else if (region == LM_WS_ROW_NORMS) {
        *offset = w.nx; *bytes = T * 4;
      } else {
        *offset = w.nw; *bytes = kE * 4;
      }
      break;
    case LM_WS_HIDDEN: *offset = w.hbuf; *bytes = (R + T) * kI * 2; break;
    case LM_WS_DOWN: *offset = w.vbuf; *bytes = (R + T) * kH * 2; break;
    case LM_WS_ACT_Q:
    case LM_WS_ACT_SCALES:
    case LM_WS_SLOT_IDS:
    case LM_WS_SLOT_WEIGHTS:
    case LM_WS_GATE_UP_ACC:
    case LM_WS_DOWN_ACC:
      LM_REQUIRE(decode, LM_EINVAL, "region written by decode calls (one token) only");
      switch (region) {
        case LM_WS_ACT_Q: *offset = w.xq; *bytes = kH; break;
        case LM_WS_ACT_SCALES: *offset = w.xs; *bytes = kH / 128 * 4; break;
        case LM_WS_SLOT_IDS: *offset = w.sel; *bytes = kTopK * 4; break;
        case LM_WS_SLOT_WEIGHTS: *offset = w.selw; *bytes = kTopK * 4; break;
        case LM_WS_GATE_UP_ACC: *offset = w.dacc_gu; *bytes = kTopK * 2 * kI * 4; break;
        default: *offset = w.dacc_dn; *bytes = kTopK * kH * 4; break;
      }
      break;
    default: return set_error(LM_EINVAL, "unknown workspace region");
  }
  return LM_OK;
}

namespace {
// What the last prefill call on each workspace left there for a chained
// successor: the layer whose normalized inputs it wrote, for how many rows
// and with which eps (none after an unchained call).  Host-side calls are in
// stream order per workspace, also while a HIP graph is captured.
struct ChainState {
  const lm_moe_layer *next;
  int64_t tokens;
  float eps;
};
std::mutex g_chain_mutex;
std::unordered_map<const void *, ChainState> g_chain;

}  // namespace

extern "C" int lm_moe_workspace_init(void *workspace, int64_t bytes, void *stream) {
  LM_REQUIRE(workspace && bytes >= 256 && bytes % 4 == 0, LM_EINVAL,
             "workspace must be at least 256 bytes and a multiple of 4");
  {  // a (re)initialized workspace holds no chained layer's inputs
    std::lock_guard<std::mutex> lock(g_chain_mutex);
    g_chain.erase(workspace);
  }
  const int64_t blocks = std::min<int64_t>(cdiv(bytes >> 2, 256), 4096);
  fill_zero_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(
      static_cast<uint32_t *>(workspace), bytes);
  return check_launch("fill_zero_kernel");
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the workspace of calls up to kScratchMaxTokens
// tokens lives in a file-scope device array.  Each device that runs the
// library holds its own copy until the process ends; its address on a
// device comes from hipGetSymbolAddress, taken once per device (with that
// device current) by lm_moe_static_init or, outside graph capture, by the
// first static call there, and kept.  Every call on a device shares that
// device's array, so calls that overlap on one device (other streams, other
// host threads) race.  No region needs a starting value: every call writes
// each region before reading it.
constexpr int64_t kScratchMaxTokens = 128;
constexpr int64_t kScratchBytes = layout(kScratchMaxTokens).total;  // 7,323,392 B
__device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

int current_device(int *dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess)
    return set_error(LM_ELAUNCH, std::string("hipGetDevice failed: ") + hipGetErrorString(e));
  LM_REQUIRE(*dev >= 0 && *dev < kMaxDevices, LM_EINVAL, "device index beyond 63");
  return LM_OK;
}

// The scratch address on device `dev` (the current device), resolved on
// first use unless `capturing`: the lookup is not a stream operation, but it
// is kept out of graph capture, where only stream work belongs.
int device_scratch(int dev, bool capturing, void **ptr) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    LM_REQUIRE(!capturing, LM_EINVAL,
               "the static scratch of this device is not resolved: call lm_moe_static_init() "
               "before capturing lm_moe_layer_forward_static");
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(LM_ELAUNCH, std::string("hipGetSymbolAddress(scratch) failed: ") +
                                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return LM_OK;
}
}  // namespace

namespace {
int check_layer(const lm_moe_layer *layer) {
  LM_REQUIRE(layer->struct_size == (int64_t)sizeof(lm_moe_layer), LM_EINVAL,
             "lm_moe_layer.struct_size differs from this library's sizeof(lm_moe_layer): "
             "set it, or rebuild the caller against this header");
  LM_REQUIRE(layer->router_w && layer->shared_gate_w && layer->gu_q && layer->gu_s &&
                 layer->dn_q && layer->dn_s,
             LM_EINVAL, "null layer weight");
  LM_REQUIRE(layer->gu_q_tiles_format == LM_TILES_PLAIN ||
                 layer->gu_q_tiles_format == LM_TILES_F16,
             LM_EINVAL, "unknown gu_q_tiles_format");
  return LM_OK;
}

// The fused layer.  For prefill calls (tokens > 1): with `next`, the combine
// also leaves next's normalized inputs for the same rows in the workspace;
// with input_normed, the workspace already holds this layer's (a chained
// call before it) and the norm kernel is not launched.  Decode calls ignore
// both: their router kernel normalizes the row itself.
int layer_forward(const lm_moe_layer *layer, const lm_moe_layer *next, bool input_normed,
                  void *h, int64_t tokens, int64_t hidden, int64_t inter, int64_t experts,
                  int64_t top_k, float eps, void *workspace, int64_t workspace_bytes,
                  int32_t *ids_out, void *weights_out, void *const *phase_events, void *stream) {
  LM_REQUIRE(hidden == kH && inter == kI && experts == kE && top_k == kTopK, LM_EINVAL,
             "fused MoE layer supports hidden 2048, intermediate 512, 256 experts, top-8");
  LM_REQUIRE(tokens >= 1 && tokens <= 65536, LM_EINVAL, "invalid token count");
  LM_REQUIRE(layer && h && workspace, LM_EINVAL, "null pointer");
  if (int rc = check_layer(layer)) return rc;
  if (next) {
    if (int rc = check_layer(next)) return rc;
  }
  const WsLayout w = layout(tokens);
  LM_REQUIRE(workspace_bytes >= w.total, LM_ENOMEM, "workspace too small for this token count");
  if (tokens > 1) {  // decode calls neither use nor leave normalized inputs
    std::lock_guard<std::mutex> lock(g_chain_mutex);
    if (input_normed) {
      const auto it = g_chain.find(workspace);
      LM_REQUIRE(it != g_chain.end() && it->second.next == layer && it->second.tokens == tokens &&
                     it->second.eps == eps,
                 LM_EINVAL,
                 "input_normed: the previous call on this workspace did not chain into this "
                 "layer with the same token count and eps");
    }
    if (next)
      g_chain[workspace] = ChainState{next, tokens, eps};
    else
      g_chain.erase(workspace);
  }
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  LayerArgs a{};
  a.router_w = static_cast<const uint16_t *>(layer->router_w);
  a.router_bias = layer->router_bias;
  a.gate_w = static_cast<const uint16_t *>(layer->shared_gate_w);
  a.norm_w = layer->norm_w;
  a.gu_q = layer->gu_q;
  a.gu_s = layer->gu_s;
  a.dn_q = layer->dn_q;
  a.dn_s = layer->dn_s;
  a.gu_qes = layer->gu_q_expert_stride;
  a.gu_ses = layer->gu_s_expert_stride;
  a.dn_qes = layer->dn_q_expert_stride;
  a.dn_ses = layer->dn_s_expert_stride;
  a.h = static_cast<uint16_t *>(h);
  a.eps = eps;
  a.xn = reinterpret_cast<uint16_t *>(ws + w.xn);
  // With an LM_TILES_F16 copy of gu_q the prefill gate_up GEMM runs in fp16
  // on xh (exact copies of the normalized rows, written by the norm kernel);
  // otherwise in bf16 on xn.
  const bool f16 = layer->gu_q_tiles != nullptr && layer->gu_q_tiles_format == LM_TILES_F16;
  a.xh = f16 ? reinterpret_cast<uint16_t *>(ws + w.xh) : nullptr;
  a.xk = reinterpret_cast<int *>(ws + w.xk);
  a.gl = reinterpret_cast<float *>(ws + w.gl);
  a.logits = reinterpret_cast<float *>(ws + w.logits);
  a.nx = reinterpret_cast<float *>(ws + w.nx);
  a.nw = reinterpret_cast<float *>(ws + w.nw);
  a.ids = reinterpret_cast<int64_t *>(ws + w.ids);
  a.wts = reinterpret_cast<uint16_t *>(ws + w.wts);
  a.sel = reinterpret_cast<int *>(ws + w.sel);
  a.selw = reinterpret_cast<float *>(ws + w.selw);
  a.xq = reinterpret_cast<int8_t *>(ws + w.xq);
  a.xs = reinterpret_cast<float *>(ws + w.xs);
  a.hbuf = reinterpret_cast<uint16_t *>(ws + w.hbuf);
  a.vbuf = reinterpret_cast<uint16_t *>(ws + w.vbuf);
  a.dacc_gu = reinterpret_cast<float *>(ws + w.dacc_gu);
  a.dacc_dn = reinterpret_cast<float *>(ws + w.dacc_dn);
  a.ids_out = ids_out;
  a.wts_out = static_cast<uint16_t *>(weights_out);
  hipStream_t st = as_stream(stream);
  auto mark = [&](int i) -> int {
    if (!phase_events) return LM_OK;
    hipError_t e = hipEventRecord(static_cast<hipEvent_t>(phase_events[i]), st);
    return e == hipSuccess ? LM_OK
                           : set_error(LM_ELAUNCH, std::string("hipEventRecord failed: ") +
                                                       hipGetErrorString(e));
  };

  if (tokens == 1) {
    if (int rc = mark(0)) return rc;
    decode_router_kernel<<<kRouterBlocks + 1, 256, 0, st>>>(a.h, a.norm_w, a.router_w, a.gate_w, a);
    if (int rc = check_launch("decode_router_kernel")) return rc;
    if (int rc = mark(1)) return rc;
    decode_gate_up_kernel<<<kI / kGuPairs * kTopK, 256, 0, st>>>(a.logits, a.xq, a.xs, a.xn,
                                                                 a.gu_q, a.gu_s, a);
    if (int rc = check_launch("decode_gate_up_kernel")) return rc;
    if (int rc = mark(2)) return rc;
    static_assert(kH / kDnCols == 256, "the XCD deal of decode_down_kernel");
    decode_down_kernel<<<kH / kDnCols, 256, 0, st>>>(a.sel, a.hbuf, a.selw, a.dn_q, a.dn_s, a.h, a);
    if (int rc = check_launch("decode_down_kernel")) return rc;
    return mark(3);
  }

  const int64_t T = tokens, R = T * kTopK;
  int64_t *pos = reinterpret_cast<int64_t *>(ws + w.pos);
  int64_t *table = reinterpret_cast<int64_t *>(ws + w.table);
  int *ptile = reinterpret_cast<int *>(ws + w.ptile);
  uint8_t *bcounts = ws + w.bcounts;
  int *rslot = reinterpret_cast<int *>(ws + w.rslot);
  int *rpos = reinterpret_cast<int *>(ws + w.rpos);
  uint16_t *vbuf = a.vbuf;
  if (int rc = mark(0)) return rc;
  if (!input_normed) {
    prefill_norm_gate_kernel<<<(unsigned)(T > kE ? T : kE), 256, 0, st>>>(
        a.h, a.router_w, a.gate_w, a.norm_w, (int)T, a);
    if (int rc = check_launch("prefill_norm_gate_kernel")) return rc;
  }
  if (int rc = mark(1)) return rc;
  router_approx_kernel<<<dim3(cdiv(T, kRaTok), kE / kRaExp), 256, 0, st>>>(a.xn, a.router_w,
                                                                          a.logits, (int)T, a);
  if (int rc = check_launch("router_approx_kernel")) return rc;
  if (int rc = mark(2)) return rc;
  const int nb = (int)cdiv(T, kTopkTokens);
  prefill_topk_count_kernel<<<nb, kTopkTokens * 64, 0, st>>>((int)T, a.router_bias, a.xn, a.logits,
                                                              a.nw, a.nx, a, bcounts, rslot);
  if (int rc = check_launch("prefill_topk_count_kernel")) return rc;
  if (int rc = mark(3)) return rc;
  prefill_scan_kernel<<<cdiv(R, kScanRoutes), 1024, 0, st>>>(a.ids, rslot, bcounts, nb, (int)T,
                                                              (int)w.max_tiles, pos, table, ptile,
                                                              rpos);
  if (int rc = check_launch("prefill_scan_kernel")) return rc;
  if (int rc = mark(4)) return rc;
  // gate_up over the T token rows gathered through pos, down over the R + T
  // rows of hbuf; the banks hold E + 1 experts (index E = shared expert)
  // (the weights' tile-layout copies, when the caller provides them)
  const RoutedGemm gu{f16 ? a.xh : a.xn, kH,  T,  a.gu_q, a.gu_s,  a.gu_qes, a.gu_ses,
                      kE + 1,  pos,     table, w.n_tiles, kBM, a.hbuf, R + T,
                      2 * kI,  kH,      true,  true,   LM_BF16, layer->gu_q_tiles,
                      f16 ? a.xk : nullptr, ptile};
  if (int rc = routed_gemm(gu, st)) return rc;
  if (int rc = mark(5)) return rc;
  const RoutedGemm dn{a.hbuf,  kI,      R + T, a.dn_q, a.dn_s, a.dn_qes, a.dn_ses,
                      kE + 1,  pos,     table, w.n_tiles, kBM, vbuf, R + T,
                      kH,      kI,      false, false,  LM_BF16, layer->dn_q_tiles};
  if (int rc = routed_gemm(dn, st)) return rc;
  if (int rc = mark(6)) return rc;
  if (next) {
    const bool next_f16 = next->gu_q_tiles != nullptr && next->gu_q_tiles_format == LM_TILES_F16;
    const NextLayer nl{static_cast<const uint16_t *>(next->router_w),
                       static_cast<const uint16_t *>(next->shared_gate_w), next->norm_w,
                       next_f16 ? reinterpret_cast<uint16_t *>(ws + w.xh) : nullptr};
    prefill_combine_kernel<true><<<(unsigned)(T > kE ? T : kE), 256, 0, st>>>(
        a.ids, rpos, a.wts, vbuf, R, (int)T, a, nl);
  } else {
    prefill_combine_kernel<false><<<(unsigned)T, 256, 0, st>>>(a.ids, rpos, a.wts, vbuf, R, (int)T,
                                                              a, NextLayer{});
  }
  if (int rc = check_launch("prefill_combine_kernel")) return rc;
  if (int rc = mark(7)) return rc;
  if (ids_out || weights_out) {
    export_routing_kernel<<<cdiv(R, 256), 256, 0, st>>>(a.ids, a.wts, ids_out, a.wts_out, R);
    return check_launch("export_routing_kernel");
  }
  return LM_OK;
}
}  // namespace

extern "C" int lm_moe_layer_forward(const lm_moe_layer *layer, void *h, int64_t tokens,
                                    int64_t hidden, int64_t inter, int64_t experts, int64_t top_k,
                                    float eps, void *workspace, int64_t workspace_bytes,
                                    int32_t *ids_out, void *weights_out,
                                    void *const *phase_events, void *stream) {
  return layer_forward(layer, nullptr, false, h, tokens, hidden, inter, experts, top_k, eps,
                       workspace, workspace_bytes, ids_out, weights_out, phase_events, stream);
}

extern "C" int lm_moe_layer_forward_chain(const lm_moe_layer *layer, const lm_moe_layer *next,
                                          int input_normed, void *h, int64_t tokens,
                                          int64_t hidden, int64_t inter, int64_t experts,
                                          int64_t top_k, float eps, void *workspace,
                                          int64_t workspace_bytes, int32_t *ids_out,
                                          void *weights_out, void *const *phase_events,
                                          void *stream) {
  return layer_forward(layer, next, input_normed != 0, h, tokens, hidden, inter, experts, top_k,
                       eps, workspace, workspace_bytes, ids_out, weights_out, phase_events,
                       stream);
}

extern "C" int64_t lm_moe_static_max_tokens(void) { return kScratchMaxTokens; }

extern "C" int lm_moe_static_init(void) {
  int dev = -1;
  if (int rc = current_device(&dev)) return rc;
  void *ws = nullptr;
  return device_scratch(dev, false, &ws);
}

extern "C" int lm_moe_layer_forward_static(const lm_moe_layer *layer, void *h, int64_t tokens,
                                           int64_t hidden, int64_t inter, int64_t experts,
                                           int64_t top_k, float eps, int32_t *ids_out,
                                           void *weights_out, void *const *phase_events,
                                           void *stream) {
  LM_REQUIRE(tokens >= 1, LM_EINVAL, "invalid token count");
  LM_REQUIRE(tokens <= kScratchMaxTokens, LM_ENOMEM,
             "token count exceeds the static scratch (128 tokens); use lm_moe_layer_forward "
             "with a caller workspace");
  // The array is looked up for the current device, so the kernels must run
  // there: a stream of another device would hand them a foreign address.
  int dev = -1, sdev = -1;
  if (int rc = current_device(&dev)) return rc;
  hipStream_t st = as_stream(stream);
  hipError_t e = hipStreamGetDevice(st, &sdev);
  if (e != hipSuccess)
    return set_error(LM_EINVAL, std::string("hipStreamGetDevice failed: ") + hipGetErrorString(e));
  LM_REQUIRE(sdev == dev, LM_EINVAL,
             "the stream belongs to another device than the current one; make the stream's "
             "device current for lm_moe_layer_forward_static");
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess)
    return set_error(LM_EINVAL, std::string("hipStreamIsCapturing failed: ") + hipGetErrorString(e));
  void *ws = nullptr;
  if (int rc = device_scratch(dev, cs != hipStreamCaptureStatusNone, &ws)) return rc;
  return lm_moe_layer_forward(layer, h, tokens, hidden, inter, experts, top_k, eps, ws,
                              kScratchBytes, ids_out, weights_out, phase_events, stream);
}
