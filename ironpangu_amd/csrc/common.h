// Shared device helpers for the gfx950 attention-path kernels.
//
// bf16 rounding is round-to-nearest-even on the fp32 bit pattern, the rule the
// reference uses everywhere it narrows to bf16
// (crates/inferfabric-cli/src/npu_probe.rs:151-154,
//  native/kernels/cache_quantization.cpp:9-12). NaN inputs stay quiet NaN here
// (the reference rule would also produce a NaN pattern, but not a canonical one).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ifattn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Two fp32 -> packed bf16 pair (lo in bits 0..15), round-to-nearest-even in
// hardware (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2_t));
}

// Raw v_exp_f32 (2^x); -inf -> 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Buffer resource over [base, base + bytes): loads at offsets past the end
// return zero instead of touching memory. Base must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, int(bytes),
                                           0x00020000);
}
// POL: cache-policy bits of the load (0: default; 2: nontemporal).
template <int POL = 0>
__device__ __forceinline__ u32x4 buf_load_x4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL));
}
__device__ __forceinline__ uint32_t buf_load_x1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Buffer descriptor as four SGPR words, for the direct-to-LDS load below.
__device__ __forceinline__ u32x4 raw_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return u32x4{uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(a))),
               uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(a >> 32) & 0xffffu)),
               uint32_t(__builtin_amdgcn_readfirstlane(bytes)), 0x00020000u};
}
// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return uint32_t(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) char *)(p)));
}
// Direct-to-LDS load (buffer_load_dwordx4 ... lds): lane i's 16 bytes at
// offset voff of the buffer land at LDS byte lds_base + 16*i (lds_base is
// wave-uniform); offsets past the buffer end write zeros. The compiler does not
// see these LDS writes: the caller waits for them with lds_dma_wait<N>() (N =
// direct loads it may leave in flight) and a workgroup barrier before any wave
// reads the bytes, and must not let such a load target bytes a wave may still
// be reading. NT sets the nontemporal cache policy (streamed bytes that no
// other workgroup will read again).
template <bool NT = false>
__device__ __forceinline__ void lds_dma16(u32x4 rsrc, uint32_t voff, uint32_t lds_base) {
  if constexpr (NT)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
                 :
                 : "v"(voff), "s"(rsrc), "{m0}"(lds_base)
                 : "memory");
  else
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "{m0}"(lds_base)
                 : "memory");
}
// Direct-to-LDS dword load: lane i's 4 bytes at offset voff land at LDS byte
// lds_base + 4*i (zeros past the buffer end); same rules as lds_dma16.
__device__ __forceinline__ void lds_dma4(u32x4 rsrc, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "{m0}"(lds_base)
               : "memory");
}
template <int N>
__device__ __forceinline__ void lds_dma_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// v_perm_b32 byte select: result byte i = byte sel[i] of {hi:lo} (lo = bytes 0-3).
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
// Low bf16 halves of two dwords -> one dword {a.lo, b.lo}.
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return perm_b32(b, a, 0x05040100u);
}
// High bf16 halves of two dwords -> one dword {a.hi, b.hi}.
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return perm_b32(b, a, 0x07060302u);
}

__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// 16x16x32 fp16 MFMA, same operand layout as the bf16 one.
__device__ __forceinline__ f32x4 mfma16x16x32_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// Additive offset of i8x4_to_f16_biased: code c reads as c + kI8Bias.
constexpr float kI8Bias = 1152.0f;
// Four int8 codes (one dword, code i in byte i) -> four fp16 values code + 1152,
// exactly, as two packed pairs: with its sign bit flipped a code c is the
// unsigned byte c + 128, and as the low mantissa byte of 0x6400 (fp16 1024.0,
// whose ulp is 1) it reads 1024 + c + 128. Three VALU ops per four codes,
// against a convert per code for the bf16 route.
__device__ __forceinline__ u32x2 i8x4_to_f16_biased(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  return u32x2{perm_b32(0x64646464u, u, 0x05010400u), perm_b32(0x64646464u, u, 0x05030402u)};
}
// Eight int4 codes (two's complement nibbles, element 2b in the low nibble of
// byte b, as if_cache_quantize packs them) -> eight int8 codes (element i in
// byte i of the pair). A nibble v becomes (v ^ 8) + 120 = code + 128, which
// stays within a byte (no carries), and the sign flip makes it the int8 code.
__device__ __forceinline__ u32x2 i4x8_to_i8x8(uint32_t x) {
  const uint32_t e = x & 0x0F0F0F0Fu, o = (x >> 4) & 0x0F0F0F0Fu;
  const uint32_t lo = perm_b32(o, e, 0x05010400u), hi = perm_b32(o, e, 0x07030602u);
  return u32x2{((lo ^ 0x08080808u) + 0x78787878u) ^ 0x80808080u,
               ((hi ^ 0x08080808u) + 0x78787878u) ^ 0x80808080u};
}
__device__ __forceinline__ u32x4 i8x8_to_f16_biased(uint32_t lo, uint32_t hi) {
  const u32x2 a = i8x4_to_f16_biased(lo), b = i8x4_to_f16_biased(hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}
// Eight bf16 values -> fp16 times qs (a power of two), summed into *sum as the
// fp16 values read back (so a biased product sum can drop kI8Bias * sum).
__device__ __forceinline__ u32x4 bf16x8_to_f16(u32x4 v, float qs, float *sum) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 h = {_Float16(bf16_bits_to_f32(v[i] & 0xFFFFu) * qs),
                     _Float16(bf16_bits_to_f32(v[i] >> 16) * qs)};
    *sum += float(h[0]) + float(h[1]);
    r[i] = __builtin_bit_cast(uint32_t, h);
  }
  return r;
}
// Largest |bf16| of eight packed values.
__device__ __forceinline__ float bf16x8_absmax(u32x4 v) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    m = fmaxf(m, fmaxf(fabsf(bf16_bits_to_f32(v[i] & 0xFFFFu)), fabsf(bf16_bits_to_f32(v[i] >> 16))));
  return m;
}
// Power of two 2^-e that brings amax into [2^14, 2^15): inside fp16's range
// with room for the biased product sums, and away from fp16's subnormals, so
// small q keep their 11 significant bits (e is clamped to [-100, 127]; a zero
// or subnormal amax gets 2^100).
__device__ __forceinline__ float f16_range_scale(float amax) {
  int e = int((__float_as_uint(amax) >> 23) & 0xFFu) - 127 - 14;
  e = e < -100 ? -100 : (e > 127 ? 127 : e);
  return __uint_as_float(uint32_t(127 - e) << 23);
}

// 16x16x16 bf16 MFMA: lane l holds row (l & 15) of A and column (l & 15) of B,
// k = 4(l >> 4) .. 4(l >> 4) + 3, as two packed bf16 pairs each.
__device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}
__device__ __forceinline__ float wave_sum_xor(float v, int mask) {
  return v + __shfl_xor(v, mask, 64);
}

// Lane exchange across 16-lane rows (partner lane l ^ 16) and across halves
// (l ^ 32) on the VALU: v_permlane16_swap / v_permlane32_swap return, in both
// partner lanes, {value of the even-row lane, value of the odd-row lane}, so a
// max or sum of the pair is one more VALU op (no LDS round trip, unlike
// ds_bpermute). Both partners get bit-identical results.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <typename T>
__device__ __forceinline__ T uniform(T v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// Load of data no kernel writes while this one runs (plans, lengths, tables
// written by an earlier launch), through the constant address space: at a
// wave-uniform address it becomes a scalar load, which waits on its own
// counter instead of behind the wave's outstanding vector stores.
template <typename T>
__device__ __forceinline__ T ld_const(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

__device__ __forceinline__ u32x4 load_u32x4(const void *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}
__device__ __forceinline__ void store_u32x4(void *p, u32x4 v) {
  *reinterpret_cast<u32x4 *>(p) = v;
}

}  // namespace ifattn
