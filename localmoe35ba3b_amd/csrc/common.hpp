// Shared device helpers for the gfx950 (CDNA4) kernels: 16-bit float
// conversions, exact int8 dequantization, DPP lane reductions, and the
// host-side status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "bounds.hpp"
#include "localmoe35ba3b.h"

namespace lm {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- 16-bit floats
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Activation type tags: storage is always 16-bit words.
struct BF16 {
  static __device__ __forceinline__ float to_f32(uint32_t b) { return bf16_bits_to_f32(b); }
  static __device__ __forceinline__ uint16_t from_f32(float f) { return f32_to_bf16_bits(f); }
  static __device__ __forceinline__ float round(float f) { return round_bf16(f); }
  // Pack two fp32 into two RNE 16-bit values (low = a).
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    bf16x2 v;
    v.x = (__bf16)a;
    v.y = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
  }
  // acc + a.lo*b.lo + a.hi*b.hi
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), acc, false);
  }
  static __device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

struct FP16 {
  static __device__ __forceinline__ float to_f32(uint32_t b) { return f16_bits_to_f32(b); }
  static __device__ __forceinline__ uint16_t from_f32(float f) { return f32_to_f16_bits(f); }
  static __device__ __forceinline__ float round(float f) { return (float)(_Float16)f; }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    f16x2 v;
    v.x = (_Float16)a;
    v.y = (_Float16)b;
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b),
                                  acc, false);
  }
  static __device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// ------------------------------------------------------------ exact dequant
// Four int8 weights (one dword) -> four fp32 values equal to fl32(q * s).
// The bytes are biased to unsigned (q + 128) so v_cvt_f32_ubyte* converts
// them exactly; fma(u, s, -128 s) evaluates u*s - 128*s = q*s exactly before
// its single rounding, so the result is the correctly rounded product q*s.
// (-128*s is exact: a power-of-two multiple of s.)
__device__ __forceinline__ void dequant4(uint32_t w, float s, float neg128s, float out[4]) {
  const uint32_t u = w ^ 0x80808080u;
  out[0] = __builtin_fmaf((float)(u & 255u), s, neg128s);
  out[1] = __builtin_fmaf((float)((u >> 8) & 255u), s, neg128s);
  out[2] = __builtin_fmaf((float)((u >> 16) & 255u), s, neg128s);
  out[3] = __builtin_fmaf((float)(u >> 24), s, neg128s);
}

// Sixteen int8 weights -> eight packed 16-bit words of T(q * s).
template <typename T>
__device__ __forceinline__ void dequant16(u32x4 w, float s, uint32_t out[8]) {
  const float n = -128.0f * s;
  float f[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dequant4(w[i], s, n, f);
    out[2 * i] = T::pack2(f[0], f[1]);
    out[2 * i + 1] = T::pack2(f[2], f[3]);
  }
}

// ------------------------------------------------------------ lane reductions
// Sums over the 8 lanes of each lane octet (lanes 8j..8j+7); every lane of the
// octet receives the total.  DPP: xor-1 and xor-2 quad permutations, then the
// half-row mirror pairs the two quads of the octet.
__device__ __forceinline__ int octet_sum_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  return v;
}
__device__ __forceinline__ float octet_sum_f32(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  return v;
}

// Full 64-lane fp32 sum through an xor butterfly (32, 16, ..., 1): the fixed
// order of the RMSNorm reductions, which the oracle restates.
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Full 64-lane fp64 sum without LDS round trips: DPP sums inside each
// 16-lane row, then the four row sums through readlane.  The summands here
// are exact products whose sum fp64 holds exactly, so the order is free.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = __double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const unsigned long long b = __double_as_longlong(v);
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
  v += dpp_f64<0xB1>(v);
  v += dpp_f64<0x4E>(v);
  v += dpp_f64<0x141>(v);
  v += dpp_f64<0x140>(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    unsigned long long w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

// ------------------------------------------------------------ wave LDS hand-off
// Lanes of one wave handing data to each other through LDS: every LDS access
// of the wave before this point is ordered before every LDS access after it.
// The wave barrier alone is a scheduling barrier without memory semantics
// (the compiler may move LDS accesses across it when it can prove them
// disjoint); the wavefront-scope fences make the ordering a memory-model
// guarantee.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------------ loads
// Loads from global memory through global address-space pointers, so that
// they compile to global (not flat) loads even where the pointer itself was
// loaded from memory (descriptor tables): a flat load counts on the LDS
// counter as well, and every later LDS or scalar wait would wait for it.
template <typename V>
__device__ __forceinline__ V ldg(const void *p) {
  return *(const __attribute__((address_space(1))) V *)p;
}
__device__ __forceinline__ u32x4 ldg16(const void *p) { return ldg<u32x4>(p); }
// Non-temporal 16-byte load, for data read once: it streams past the caches
// instead of evicting data that is read again.
__device__ __forceinline__ u32x4 ldg16_nt(const void *p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4 *)p);
}
__device__ __forceinline__ float ldg_f32(const float *p) { return ldg<float>(p); }
__device__ __forceinline__ uint2 ldg_u2(const void *p) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = ldg<u32x2>(p);
  return uint2{v.x, v.y};
}
// Load bypassing the non-coherent per-CU cache (data written by other
// workgroups of the same kernel).
__device__ __forceinline__ float ld_coherent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_coherent(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// fp32 ops that must not be contracted into an FMA (reference epilogues run
// with enable_fp_fusion=False).  The library is compiled with
// -ffp-contract=off, so plain operators round after every operation; fused
// multiply-adds appear only where code calls __builtin_fmaf explicitly.
__device__ __forceinline__ float mul_rn(float a, float b) { return a * b; }
__device__ __forceinline__ float add_rn(float a, float b) { return a + b; }

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// Order-preserving keys packing a logit with an index so that larger key =
// (larger value, then smaller index); -0 is folded onto +0 and comes back as
// +0, which leaves every later use unchanged.  Key64 holds any fp32 value;
// Key32 holds a value whose low 16 bits are zero (a bf16 value, which is what
// a router without bias produces) in half the bits, so each step of the
// selection moves and compares one register instead of two.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t k) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, CTRL, 0xF, 0xF, false);
}
// 64-bit value moved between lanes by one DPP pattern (both halves).
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long k) {
  const uint32_t lo = dpp_u32<CTRL>((uint32_t)k);
  const uint32_t hi = dpp_u32<CTRL>((uint32_t)(k >> 32));
  return ((unsigned long long)hi << 32) | lo;
}
// Maximum over each 16-lane row, in every lane of the row: neighbours in a
// quad, then quads of a half-row (half mirror), then half-rows (mirror).
template <typename T, T (*MOVE0)(T), T (*MOVE1)(T), T (*MOVE2)(T), T (*MOVE3)(T)>
__device__ __forceinline__ T row_max_keys(T k) {
  T o = MOVE0(k);
  k = o > k ? o : k;
  o = MOVE1(k);
  k = o > k ? o : k;
  o = MOVE2(k);
  k = o > k ? o : k;
  o = MOVE3(k);
  return o > k ? o : k;
}

struct Key64 {
  using T = unsigned long long;
  static __device__ __forceinline__ T make(float v, int idx) { return key64_make(v, idx); }
  static __device__ __forceinline__ int index(T k) { return key64_index(k); }
  static __device__ __forceinline__ float value(T k) { return key64_value(k); }
  static __device__ __forceinline__ T row_max(T k) {
    return row_max_keys<T, dpp_u64<0xB1>, dpp_u64<0x4E>, dpp_u64<0x141>, dpp_u64<0x140>>(k);
  }
  static __device__ __forceinline__ T readlane(T k, int lane) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)k, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), lane);
    return ((T)hi << 32) | lo;
  }
};

struct Key32 {
  using T = uint32_t;
  static __device__ __forceinline__ T make(float v, int idx) { return key32_make(v, idx); }
  static __device__ __forceinline__ int index(T k) { return key32_index(k); }
  static __device__ __forceinline__ float value(T k) { return key32_value(k); }
  static __device__ __forceinline__ T row_max(T k) {
    return row_max_keys<T, dpp_u32<0xB1>, dpp_u32<0x4E>, dpp_u32<0x141>, dpp_u32<0x140>>(k);
  }
  static __device__ __forceinline__ T readlane(T k, int lane) {
    return (T)__builtin_amdgcn_readlane((int)k, lane);
  }
};

__device__ __forceinline__ float row_sum_f32(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return v;
}

// x / s for the W8A8 activation quantization (w8a8.py:8-14), given
// r = 1 / s correctly rounded (one division per 128-group): one multiply and
// Markstein's fused correction step.  For every bf16 and fp16 value x with
// |x| <= the group absmax that s is formed from, rint of the result equals
// rint of the correctly rounded quotient (tests/native/test_quant_division.c
// checks all 2.07e9 such pairs), so the int8 values are the reference's.
__device__ __forceinline__ float quant_div(float x, float s, float r) {
  const float y = x * r;
  const float e = __builtin_fmaf(-y, s, x);
  return __builtin_fmaf(e, r, y);
}

// ------------------------------------------------------------ wave selection
// Lane l's copy of lane l ^ D's value (D = 1, 2, 4, 8, 16, 32): quad
// permutations for 1 and 2, the two row shifts by 4 written into alternate
// 4-lane banks for 4, the row rotation by 8, a swizzle within 32 lanes for 16
// and a permute across the wave for 32.
template <int D>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t v) {
  if constexpr (D == 1) {
    return dpp_u32<0xB1>(v);
  } else if constexpr (D == 2) {
    return dpp_u32<0x4E>(v);
  } else if constexpr (D == 4) {
    int t = __builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0x5, false);  // row_shl:4
    t = __builtin_amdgcn_update_dpp(t, (int)v, 0x114, 0xF, 0xA, false);      // row_shr:4
    return (uint32_t)t;
  } else if constexpr (D == 8) {
    return dpp_u32<0x128>(v);  // row_ror:8
  } else if constexpr (D == 16) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (16 << 10) | 0x1F);
  } else {
    static_assert(D == 32, "lane_xor_u32: D in {1, 2, 4, 8, 16, 32}");
    return (uint32_t)__shfl_xor((int)v, 32, 64);
  }
}
// Lane l's copy of lane l ^ M for the mirror partners of the top-8 merges:
// 7 (half-row mirror), 15 (row mirror), 23 (swizzle within 32 lanes), 39
// (permute across the wave).
template <int M>
__device__ __forceinline__ uint32_t lane_mirror_u32(uint32_t v) {
  if constexpr (M == 7) {
    return dpp_u32<0x141>(v);
  } else if constexpr (M == 15) {
    return dpp_u32<0x140>(v);
  } else if constexpr (M == 23) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (23 << 10) | 0x1F);
  } else {
    static_assert(M == 39, "lane_mirror_u32: M in {7, 15, 23, 39}");
    return (uint32_t)__shfl_xor((int)v, 39, 64);
  }
}
template <int D>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) { return lane_xor_u32<D>(v); }
template <int D>
__device__ __forceinline__ unsigned long long lane_xor(unsigned long long v) {
  return ((unsigned long long)lane_xor_u32<D>((uint32_t)(v >> 32)) << 32) |
         lane_xor_u32<D>((uint32_t)v);
}
template <int M>
__device__ __forceinline__ uint32_t lane_mirror(uint32_t v) { return lane_mirror_u32<M>(v); }
template <int M>
__device__ __forceinline__ unsigned long long lane_mirror(unsigned long long v) {
  return ((unsigned long long)lane_mirror_u32<M>((uint32_t)(v >> 32)) << 32) |
         lane_mirror_u32<M>((uint32_t)v);
}

// Compare-exchange with lane l ^ J: the lower lane of the pair keeps the
// larger key when `desc`, the smaller otherwise.
template <int J, typename T>
__device__ __forceinline__ T lane_cx(T k, int lane, bool desc) {
  const T p = lane_xor<J>(k);
  const T hi = k > p ? k : p, lo = k > p ? p : k;
  return (((lane & J) == 0) == desc) ? hi : lo;
}
// Bitonic sort of every 8-lane block, descending.
template <typename T>
__device__ __forceinline__ T sort8_desc(T k, int lane) {
  k = lane_cx<1>(k, lane, (lane & 2) == 0);
  k = lane_cx<2>(k, lane, (lane & 4) == 0);
  k = lane_cx<1>(k, lane, (lane & 4) == 0);
  k = lane_cx<4>(k, lane, true);
  k = lane_cx<2>(k, lane, true);
  return lane_cx<1>(k, lane, true);
}
// Every 8-lane block of a group holds the same list sorted descending; the
// partner group's list is read mirrored (lane ^ M, M = group size * 2 - 1
// folded into the block), so position i meets partner position 7 - i.  The
// larger of each pair are the 8 largest of both lists in bitonic order; a
// half-cleaner sorts them descending in every block of the merged group.
template <int M, typename T>
__device__ __forceinline__ T merge_top8(T k, int lane) {
  const T p = lane_mirror<M>(k);
  k = k > p ? k : p;
  k = lane_cx<4>(k, lane, true);
  k = lane_cx<2>(k, lane, true);
  return lane_cx<1>(k, lane, true);
}
// The 8 largest of the wave's 64 keys (one per lane, distinct), sorted
// descending in every 8-lane block: lane l holds the one of rank l & 7.
template <typename T>
__device__ __forceinline__ T wave_top8(T k, int lane) {
  k = sort8_desc(k, lane);
  k = merge_top8<15>(k, lane);
  k = merge_top8<23>(k, lane);
  return merge_top8<39>(k, lane);
}
// Two lists per 8-lane block, each sorted descending -> the 8 largest of
// both, sorted descending (b is read mirrored within the block, as in
// merge_top8).
template <typename T>
__device__ __forceinline__ T merge2_top8(T a, T b, int lane) {
  const T p = lane_mirror<7>(b);
  T k = a > p ? a : p;
  k = lane_cx<4>(k, lane, true);
  k = lane_cx<2>(k, lane, true);
  return lane_cx<1>(k, lane, true);
}
// The 8th largest of the wave's 256 keys (4 per lane, distinct), in every
// lane, by DPP exchanges alone: each key slot is sorted within its 8-lane
// blocks, the four sorted slots are merged within each block (its top 8 of
// 32), then the blocks are merged across the wave as in wave_top8.
template <class KT>
__device__ __forceinline__ typename KT::T kth8_key_wave(const typename KT::T key[4], int lane) {
  using T = typename KT::T;
  T s[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) s[j] = sort8_desc(key[j], lane);
  T k = merge2_top8(merge2_top8(s[0], s[1], lane), merge2_top8(s[2], s[3], lane), lane);
  k = merge_top8<15>(k, lane);
  k = merge_top8<23>(k, lane);
  k = merge_top8<39>(k, lane);
  return KT::readlane(k, 7);
}

// LDS scratch of one top-k wave, in 64-bit words: 4 rows x 16 candidates
// plus 16 selected probabilities.
constexpr int kTopkScratch = 80;

// One wave per token.  Selection key: (logit desc, expert id asc).  Softmax
// over all experts in fp32, renormalised over the selected ones, bf16 out.
// Lane l holds experts 4 l .. 4 l + 3, so 16-lane row r holds 64 r ..
// 64 r + 63.  Each row first finds its own top K with DPP maxima (no LDS
// round trips), then every one of the 4 K row winners takes its rank among
// all of them from LDS; the K best ranks are the selection.  K <= 16,
// E <= 256.  The probability sum runs in selection order.
// Sorts a lane's 4 keys, then finds each 16-lane row's top K by DPP maxima
// (the lane holding a row's maximum pops it) and writes the 4 K row winners
// to scratch[row * K + i].  Returns the lane's row maximum.
template <class KT>
__device__ __forceinline__ typename KT::T topk_row_winners(typename KT::T key[4], int K, int lane,
                                                          typename KT::T *scratch) {
  using T = typename KT::T;
  auto cswap = [&](int a, int b) {
    if (key[a] < key[b]) {
      const T tmp = key[a];
      key[a] = key[b];
      key[b] = tmp;
    }
  };
  cswap(0, 1);
  cswap(2, 3);
  cswap(0, 2);
  cswap(1, 3);
  cswap(1, 2);
  T top[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    top[i] = 0;
    if (i < K) {
      const T m = KT::row_max(key[0]);
      top[i] = m;
      if (key[0] == m) {
        key[0] = key[1];
        key[1] = key[2];
        key[2] = key[3];
        key[3] = 0;
      }
    }
  }
  const int row = lane >> 4;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < K && (lane & 15) == i) scratch[row * K + i] = top[i];
  return top[0];
}

// Rank of row winner `lane` among all 4 K of them (keys are distinct; 0
// keys rank last); lanes >= 4 K get 0 keys.
template <class KT>
__device__ __forceinline__ int topk_winner_rank(const typename KT::T *scratch, int K, int lane,
                                                typename KT::T &mine) {
  using T = typename KT::T;
  const int nc = 4 * K;
  mine = lane < nc ? scratch[lane] : (T)0;
  int rank = 0;
#pragma unroll 8
  for (int j = 0; j < nc; ++j) rank += scratch[j] > mine ? 1 : 0;
  return rank;
}

template <class KT>
__device__ __forceinline__ void topk_wave_keys(const float v[4], int E, int K, int lane,
                                               unsigned long long *scratch_words, int64_t *ids_out,
                                               uint16_t *w_out) {
  using T = typename KT::T;
  T *scratch = reinterpret_cast<T *>(scratch_words);
  T key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) key[j] = lane * 4 + j < E ? KT::make(v[j], lane * 4 + j) : (T)0;
  const T rowmax = topk_row_winners<KT>(key, K, lane, scratch);
  T top[1] = {rowmax};
  // Softmax statistics: the global maximum is the best of the row maxima.
  T mk = KT::readlane(top[0], 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) {
    const T o = KT::readlane(top[0], 16 * r);
    mk = o > mk ? o : mk;
  }
  const float mx = KT::value(mk);
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (lane * 4 + j < E) part += expf(v[j] - mx);
  part = row_sum_f32(part);
  const float denom = (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 0)) +
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 16))) +
                      (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 32)) +
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), 48)));
  wave_lds_sync();
  // Rank of each row winner among all 4 K of them.
  const int nc = 4 * K;
  T mine;
  const int rank = topk_winner_rank<KT>(scratch, K, lane, mine);
  float *prob = reinterpret_cast<float *>(scratch_words + 64);
  const bool chosen = lane < nc && rank < K;
  const float pe = expf(KT::value(mine) - mx) / denom;
  if (chosen) prob[rank] = pe;
  wave_lds_sync();
  float psum = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < K) psum += prob[i];
  if (chosen) {
    ids_out[rank] = KT::index(mine);
    w_out[rank] = f32_to_bf16_bits(pe / psum);
  }
}

// topk_wave_v takes lane l's logits of experts 4 l .. 4 l + 3 already loaded
// (-INFINITY past E); topk_wave loads them from lg.  The whole wave must be
// active.  When every logit of the token is a bf16 value the selection runs
// on 32-bit keys; both key widths order the keys identically.
__device__ __forceinline__ void topk_wave_v(const float v[4], int E, int K, int lane,
                                            unsigned long long *scratch, int64_t *ids_out,
                                            uint16_t *w_out) {
  const uint32_t low = (__float_as_uint(v[0]) | __float_as_uint(v[1]) | __float_as_uint(v[2]) |
                        __float_as_uint(v[3])) & 0xFFFFu;
  if (__all(low == 0u))
    topk_wave_keys<Key32>(v, E, K, lane, scratch, ids_out, w_out);
  else
    topk_wave_keys<Key64>(v, E, K, lane, scratch, ids_out, w_out);
}

__device__ __forceinline__ void topk_wave(const float *lg, int E, int K, int lane,
                                          unsigned long long *scratch, int64_t *ids_out,
                                          uint16_t *w_out) {
  float v[4];
  if (E == 256) {
    const float4 f = *reinterpret_cast<const float4 *>(lg + lane * 4);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = lane * 4 + j < E ? lg[lane * 4 + j] : -INFINITY;
  }
  topk_wave_v(v, E, K, lane, scratch, ids_out, w_out);
}

}  // namespace lm

// ---------------------------------------------------------------- host side
namespace lm {
int set_error(int code, const std::string &msg);
int check_launch(const char *what);
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }
inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }
}  // namespace lm

#define LM_REQUIRE(cond, code, msg)        \
  do {                                     \
    if (!(cond)) return lm::set_error((code), (msg)); \
  } while (0)
