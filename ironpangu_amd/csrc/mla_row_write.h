// The MLA cache row writer shared by the stand-alone writer kernel
// (cache_write.hip) and the fused decode step (mla_decode.hip): C8 tile
// quantization and the RMSNorm + half-rope row of resident_cache_writer.h:5-20.
// Both callers run exactly this code, so their rows are bit-identical.
#pragma once
#include "common.h"

namespace ifattn {

// Symmetric int8 of one group of `width` bf16 values held as 8-element chunks.
// scale = max|x| / 127 (IEEE division), q = rne(x / scale) clamped to +-127.
// A zero group gets scale `zero_scale` and all-zero codes.
__device__ __forceinline__ float c8_scale(float amax, float zero_scale) {
  return amax == 0.0f ? zero_scale : __fdiv_rn(amax, 127.0f);
}
__device__ __forceinline__ int c8_code(float x, float scale) {
  float v = __fdiv_rn(x, scale);
  int q = __float2int_rn(v);
  return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// Fused MLA cache writer (the RMSNorm + half-rope + cache-store step of
// resident_cache_writer.h:5-20): one wave per row of 576 bf16 (512 latent +
// 64 rope). Lane l owns latent values 8l..8l+7. The fp32 operation order is
// fixed (no contraction) so the result is bit-identical to the CPU restatement:
// per-lane in-order sum of squares, xor butterfly over the 64 lanes,
// rstd = 1/sqrt(sum/512 + eps), y = (x*rstd)*gamma; PACKED rows quantize y per
// 128-value tile (16 lanes) like mla_write_c8_kernel, bf16 rows store RNE(y).
// Rope: lanes 0..31 own dims 2l, 2l+1; the partner half (d+32)%64 sits in lane
// (l+16)%32: out = bf16(a*cos + (d<32 ? -b : b)*sin).
// Correctly rounded fp32 square root for x > 0: the hardware estimate (within
// one ulp) is moved to the neighbour whose rounding interval holds sqrt(x); the
// interval ends (s +- ulp/2)^2 are exact in fp64 (25-bit operands).
__device__ __forceinline__ float sqrt_rn(float x) {
  float s = __builtin_amdgcn_sqrtf(x);
  const double dx = double(x);
  for (int it = 0; it < 2; ++it) {
    const float up = __uint_as_float(__float_as_uint(s) + 1u);
    const float dn = __uint_as_float(__float_as_uint(s) - 1u);
    const double hi = 0.5 * (double(s) + double(up)), lo = 0.5 * (double(s) + double(dn));
    if (hi * hi < dx) s = up;
    else if (lo * lo > dx) s = dn;
  }
  return s;
}

// One row by one whole wave (every lane calls it): src [576] bf16 (512 latent
// + 64 rope), gamma [512], cos/sin [64] of this row, dst the cache row.
template <bool PACKED>
__device__ __forceinline__ void mla_norm_rope_row(const uint16_t *__restrict__ src,
                                                  const uint16_t *__restrict__ gamma,
                                                  const uint16_t *__restrict__ cosr,
                                                  const uint16_t *__restrict__ sinr, float eps,
                                                  uint8_t *__restrict__ dst, int lane) {
  // Every product and sum is rounded on its own (no fused multiply-add).
#pragma clang fp contract(off)
  const u32x4 w = load_u32x4(src + lane * 8);
  const u32x4 gw = load_u32x4(gamma + lane * 8);
  float v[8], g[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
    v[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    g[2 * i] = bf16_bits_to_f32(gw[i] & 0xffffu);
    g[2 * i + 1] = bf16_bits_to_f32(gw[i] >> 16);
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float sq = v[i] * v[i];
    ss = ss + sq;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss = ss + __shfl_xor(ss, m, 64);
  const float mean = ss * (1.0f / 512.0f);
  const float rstd = __fdiv_rn(1.0f, sqrt_rn(mean + eps));
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = v[i] * rstd;
    y[i] = t * g[i];
  }
  if constexpr (PACKED) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(y[i]));
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) amax = wave_max_xor(amax, m);  // within 16 lanes
    const float scale = c8_scale(amax, 0.0f);
    uint32_t lo = 0, hi = 0;
    if (scale != 0.0f) {
#pragma unroll
      for (int i = 0; i < 4; ++i) lo |= (uint32_t(c8_code(y[i], scale)) & 0xffu) << (8 * i);
#pragma unroll
      for (int i = 0; i < 4; ++i) hi |= (uint32_t(c8_code(y[4 + i], scale)) & 0xffu) << (8 * i);
    }
    *reinterpret_cast<u32x2 *>(dst + lane * 8) = u32x2{lo, hi};
    if ((lane & 15) == 0) *reinterpret_cast<float *>(dst + 640 + (lane >> 4) * 4) = scale;
  } else {
    store_u32x4(dst + lane * 16, u32x4{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]),
                                       pack_bf16x2(y[4], y[5]), pack_bf16x2(y[6], y[7])});
  }
  // Rope: every lane takes part in the shuffle; lanes 0..31 store.
  const int rl = lane & 31;
  const uint32_t mine = reinterpret_cast<const uint32_t *>(src + 512)[rl];
  const uint32_t other = __shfl(mine, (rl + 16) & 31, 64);
  if (lane < 32) {
    const uint32_t cw = reinterpret_cast<const uint32_t *>(cosr)[rl];
    const uint32_t sw = reinterpret_cast<const uint32_t *>(sinr)[rl];
    float o2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float a = bf16_bits_to_f32(e ? mine >> 16 : mine & 0xffffu);
      const float b = bf16_bits_to_f32(e ? other >> 16 : other & 0xffffu);
      const float c = bf16_bits_to_f32(e ? cw >> 16 : cw & 0xffffu);
      const float sn = bf16_bits_to_f32(e ? sw >> 16 : sw & 0xffffu);
      const float p0 = a * c;
      const float p1 = (rl < 16 ? -b : b) * sn;
      o2[e] = p0 + p1;
    }
    reinterpret_cast<uint32_t *>(dst + (PACKED ? 512 : 1024))[rl] =
        uint32_t(f32_to_bf16_bits(o2[0])) | (uint32_t(f32_to_bf16_bits(o2[1])) << 16);
  }
}

}  // namespace ifattn
