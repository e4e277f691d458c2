// Shared device helpers for the gfx950 (CDNA4) kernels: 16-bit float
// conversions, exact int8 dequantization, DPP lane reductions, and the
// host-side status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

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

// Full 64-lane reductions through shuffles (used off the hot loops).
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    unsigned long long w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

// ------------------------------------------------------------ loads
__device__ __forceinline__ u32x4 ldg16(const void *p) {
  return *reinterpret_cast<const u32x4 *>(p);
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

// Order-preserving key of an fp32 value (-0 folded onto +0) packed with an
// index so that larger key = (larger value, then smaller index).
__device__ __forceinline__ unsigned long long topk_key(float v, int idx) {
  v = v + 0.0f;  // -0 -> +0
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (uint32_t)(0xFFFFu - (uint32_t)idx);
}
__device__ __forceinline__ int topk_key_index(unsigned long long k) {
  return (int)(0xFFFFu - (uint32_t)(k & 0xFFFFu));
}

// One wave per token.  Selection key: (logit desc, expert id asc).  Softmax
// over all experts in fp32, renormalised over the selected ones, bf16 out.
__device__ __forceinline__ void topk_wave(const float *lg, int E, int K, int lane,
                                          int64_t *ids_out, uint16_t *w_out) {
  unsigned long long key[4];
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? lg[e] : -INFINITY;
    key[j] = e < E ? topk_key(v[j], e) : 0ull;
  }
  float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
  mx = wave_max_f32(mx);
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (lane + 64 * j < E) part += expf(v[j] - mx);
  const float denom = wave_sum_f32(part);
  // Selection: K rounds of a wave-wide max over (value, -id) keys.
  float p[16];
  int id[16];
  float psum = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i < K) {
      unsigned long long best = key[0];
#pragma unroll
      for (int j = 1; j < 4; ++j) best = key[j] > best ? key[j] : best;
      best = wave_max_u64(best);
      const int e = topk_key_index(best);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (key[j] == best) key[j] = 0ull;
      const float pe = expf(lg[e] - mx) / denom;
      p[i] = pe;
      id[i] = e;
      psum += pe;
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i < K) {
        ids_out[i] = id[i];
        w_out[i] = f32_to_bf16_bits(p[i] / psum);
      }
    }
  }
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
