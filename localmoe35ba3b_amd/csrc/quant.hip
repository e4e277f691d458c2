// Group-128 int8 quantizers.
//
//  * lm_quantize_weight_g128: the offline weight format producer
//    (convert.py:31-37): s = max(amax / 127, 1e-30), q = clamp(rne(w / s), +-127).
//  * lm_act_quant_g128: dynamic per-row activation quantization of the W8A8
//    decode path (w8a8.py:8-22): s = max(amax, 1e-10) * fl32(1/127),
//    q = rint(x / s) with IEEE division (|x / s| <= 127 by construction).
//
// One 128-element group is handled by 32 lanes holding 4 elements each, so a
// wave quantizes two groups per iteration with fully coalesced 16-byte loads.
#include "gemv_core.hpp"

namespace lm {

__global__ __launch_bounds__(256) void quantize_weight_kernel(const float *__restrict__ w,
                                                              int8_t *__restrict__ q,
                                                              float *__restrict__ s,
                                                              int64_t ngroups) {
  const int lane = threadIdx.x & 63;
  const int l = lane & 31;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t g2 = wave; g2 * 2 < ngroups; g2 += nwaves) {
    const int64_t grp = g2 * 2 + (lane >> 5);
    const bool valid = grp < ngroups;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (valid) v = *reinterpret_cast<const f32x4 *>(w + grp * 128 + l * 4);
    float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
    const float sc = fmaxf(a / 127.0f, 1e-30f);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float r = rintf(v[i] / sc);
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      packed |= ((uint32_t)(uint8_t)(int8_t)(int)r) << (8 * i);
    }
    if (valid) {
      *reinterpret_cast<uint32_t *>(q + grp * 128 + l * 4) = packed;
      if (l == 0) s[grp] = sc;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t *__restrict__ x,
                                                        int8_t *__restrict__ q,
                                                        float *__restrict__ s,
                                                        int64_t ngroups) {
  // A half-wave quantizes B groups per pass: all B loads are issued before
  // the first is used and the groups are computed branch-free (slots past
  // the end redo the last group and store the same bytes to it again), so a
  // pass costs one load latency.
  constexpr int B = 4;
  const int l = threadIdx.x & 31;
  const int64_t half = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
  const int64_t nhalf = ((int64_t)gridDim.x * blockDim.x) >> 5;
  for (int64_t base = half; base < ngroups; base += nhalf * B) {
    uint2 raw[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int64_t grp = min(base + u * nhalf, ngroups - 1);
      raw[u] = *reinterpret_cast<const uint2 *>(x + grp * 128 + l * 4);
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int64_t grp = min(base + u * nhalf, ngroups - 1);
      quantize_group<T>(raw[u], l, q + grp * 128, s + grp);
    }
  }
}


static unsigned quant_grid(int64_t ngroups) {
  int64_t waves = (ngroups + 1) / 2;
  int64_t blocks = (waves + 3) / 4;
  if (blocks > 4096) blocks = 4096;
  return (unsigned)(blocks < 1 ? 1 : blocks);
}

// act_quant_kernel: one half-wave per 4 groups (8 half-waves per block).
static unsigned act_quant_grid(int64_t ngroups) {
  int64_t blocks = (ngroups + 31) / 32;
  if (blocks > 4096) blocks = 4096;
  return (unsigned)(blocks < 1 ? 1 : blocks);
}

}  // namespace lm

using namespace lm;

extern "C" int lm_quantize_weight_g128(const float *w, int8_t *q, float *s, int64_t rows,
                                       int64_t k, void *stream) {
  LM_REQUIRE(rows >= 0 && k > 0 && k % 128 == 0, LM_EINVAL, "Invalid INT8 group geometry");
  LM_REQUIRE(rows == 0 || (w && q && s), LM_EINVAL, "null pointer");
  const int64_t ngroups = rows * (k / 128);
  if (ngroups == 0) return LM_OK;
  quantize_weight_kernel<<<quant_grid(ngroups), 256, 0, as_stream(stream)>>>(w, q, s, ngroups);
  return check_launch("quantize_weight_kernel");
}

// The 16-row tile layout of an int8 bank (lm_w8_tile_rows): one wave per
// 1 KB block (16 rows x 64 K of one expert); lane 16 p + r copies piece p
// (16 bytes) of row r to byte 16 (16 p + r) of the block.  The fp16 format
// (LM_TILES_F16) also biases each byte to u = q + 128 and stores the bytes of
// every dword in the order k = 0, 2, 1, 3, which the GEMM's fp16 conversion
// takes apart with one mask and one byte permute.
__global__ __launch_bounds__(256) void tile_rows_kernel(const int8_t *__restrict__ q,
                                                        int8_t *__restrict__ tiles, int64_t blocks,
                                                        int64_t nb, int64_t kb, int64_t k,
                                                        int64_t es, int fmt) {
  const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= blocks) return;
  const int lane = threadIdx.x & 63, p = lane >> 4, r = lane & 15;
  const int64_t e = blk / (nb * kb), rem = blk - e * nb * kb;
  const int64_t b = rem / kb, s = rem - b * kb;
  u32x4 v = ldg16(q + e * es + (16 * b + r) * k + 64 * s + 16 * p);
  if (fmt == LM_TILES_F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = v[i] ^ 0x80808080u;
      v[i] = (u & 0xFF0000FFu) | ((u >> 8) & 0x0000FF00u) | ((u << 8) & 0x00FF0000u);
    }
  }
  *reinterpret_cast<u32x4 *>(tiles + e * es + (b * kb + s) * 1024 + lane * 16) = v;
}

extern "C" int lm_w8_tile_rows(const int8_t *q, int64_t experts, int64_t n, int64_t k,
                               int64_t expert_stride, int8_t *tiles, int format, void *stream) {
  LM_REQUIRE(experts >= 0 && n > 0 && k > 0 && n % 16 == 0 && k % 64 == 0, LM_EINVAL,
             "the tile layout needs n % 16 == 0 and k % 64 == 0");
  LM_REQUIRE(expert_stride >= n * k, LM_EINVAL, "expert stride smaller than n * k");
  LM_REQUIRE(format == LM_TILES_PLAIN || format == LM_TILES_F16, LM_EINVAL,
             "unknown tile format");
  LM_REQUIRE(experts == 0 || (q && tiles), LM_EINVAL, "null pointer");
  const int64_t nb = n / 16, kb = k / 64, blocks = experts * nb * kb;
  if (blocks == 0) return LM_OK;
  LM_REQUIRE((blocks + 3) / 4 < (int64_t(1) << 31), LM_EINVAL, "bank too large for one launch");
  tile_rows_kernel<<<(unsigned)((blocks + 3) / 4), 256, 0, as_stream(stream)>>>(
      q, tiles, blocks, nb, kb, k, expert_stride, format);
  return check_launch("tile_rows_kernel");
}

extern "C" int lm_act_quant_g128(const void *x, int x_dtype, int8_t *q, float *s, int64_t rows,
                                 int64_t k, void *stream) {
  LM_REQUIRE(rows >= 0 && k > 0 && k % 128 == 0, LM_EINVAL,
             "Expected CUDA rows with K divisible by 128");
  LM_REQUIRE(x_dtype == LM_BF16 || x_dtype == LM_FP16, LM_EINVAL,
             "Expected CUDA rows with K divisible by 128");
  LM_REQUIRE(rows == 0 || (x && q && s), LM_EINVAL, "null pointer");
  const int64_t ngroups = rows * (k / 128);
  if (ngroups == 0) return LM_OK;
  const uint16_t *xp = static_cast<const uint16_t *>(x);
  if (x_dtype == LM_BF16)
    act_quant_kernel<BF16><<<act_quant_grid(ngroups), 256, 0, as_stream(stream)>>>(xp, q, s, ngroups);
  else
    act_quant_kernel<FP16><<<act_quant_grid(ngroups), 256, 0, as_stream(stream)>>>(xp, q, s, ngroups);
  return check_launch("act_quant_kernel");
}
