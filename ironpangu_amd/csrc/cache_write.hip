// Slot-mapped KV-cache writes for gfx950.
//
//  * kv_write_rows: cache[slot[r]] = rows[r] for K and V (and the 576-wide MLA
//    latent row, which is the same operation with one cache). Replaces the two
//    aclnnScatterNdUpdate calls of native/src/inferfabric_acl.cpp:1364-1376 and
//    the aclnnInplaceIndexCopy of native/src/token_executor.h:733-757.
//  * kv_write_c8: the same write, quantizing each (token, kv head) row of
//    head_dim bf16 values to int8 with one fp32 scale (authoring contract
//    per_token_head_symmetric, crates/inferfabric-authoring/src/execution.rs:65-66;
//    arithmetic of native/kernels/cache_quantization.cpp:20-34 with nearest-even
//    rounding in place of ties-away).
//  * mla_write_c8: the 656-byte packed latent row (docs/packed-mla-cache.md:27-43):
//    int8 latent[512] | bf16 rope[64] | f32 scale[4], one scale per 128 values.
//
// Memory: a row is moved with 16-byte vector loads/stores, one lane per 16 B, so
// a wave writes 1 KiB contiguous per instruction; the write is purely HBM-bound
// and bit-exact (no arithmetic on copied rows).
#include <type_traits>

#include "common.h"
#include "ifattn_internal.h"
#include "mla_row_write.h"

namespace ifattn {

// Slots are int64 (reference append/index tensors, inferfabric_acl.h:103-106)
// or int32 (the MLA descriptor, token_executor.h:1304-1311).
template <typename SlotT>
__global__ __launch_bounds__(256) void kv_write_rows_kernel(
    const uint8_t *__restrict__ k_rows, const uint8_t *__restrict__ v_rows,
    uint8_t *__restrict__ k_cache, uint8_t *__restrict__ v_cache,
    const SlotT *__restrict__ slots, int64_t rows, int64_t row_vecs, int64_t num_slots) {
  // One thread per 16-byte vector; blockIdx.y selects K (0) or V (1).
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * row_vecs) return;
  const int64_t r = idx / row_vecs, c = idx - r * row_vecs;
  const int64_t slot = int64_t(slots[r]);
  if (slot < 0 || slot >= num_slots) return;  // padding rows / rejected ids
  const uint8_t *src = blockIdx.y ? v_rows : k_rows;
  uint8_t *dst = blockIdx.y ? v_cache : k_cache;
  store_u32x4(dst + (slot * row_vecs + c) * 16, load_u32x4(src + (r * row_vecs + c) * 16));
}

// One wave per (row, kv head, K|V); head_dim <= 512 handled as 8 values/lane.
template <typename SlotT>
__global__ __launch_bounds__(256) void kv_write_c8_kernel(
    const uint16_t *__restrict__ k_rows, const uint16_t *__restrict__ v_rows,
    int8_t *__restrict__ k_cache, int8_t *__restrict__ v_cache,
    float *__restrict__ k_scale, float *__restrict__ v_scale,
    const SlotT *__restrict__ slots, int64_t rows, int kv_heads, int head_dim,
    int64_t num_slots) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (unit >= rows * kv_heads) return;
  const int64_t r = unit / kv_heads;
  const int h = int(unit - r * kv_heads);
  const int64_t slot = int64_t(slots[r]);
  if (slot < 0 || slot >= num_slots) return;
  const uint16_t *src = (blockIdx.y ? v_rows : k_rows) + (r * kv_heads + h) * head_dim;
  int8_t *dst = (blockIdx.y ? v_cache : k_cache) + (slot * kv_heads + h) * head_dim;
  float *sc = (blockIdx.y ? v_scale : k_scale) + slot * kv_heads + h;
  const bool active = lane * 8 < head_dim;
  float x[8];
  float amax = 0.0f;
  if (active) {
    u32x4 w = load_u32x4(src + lane * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
      x[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = wave_max_xor(amax, m);
  const float scale = c8_scale(amax, 1.0f);
  if (active) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) lo |= (uint32_t(c8_code(x[i], scale)) & 0xffu) << (8 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) hi |= (uint32_t(c8_code(x[4 + i], scale)) & 0xffu) << (8 * i);
    *reinterpret_cast<u32x2 *>(dst + lane * 8) = u32x2{lo, hi};
  }
  if (lane == 0) *sc = scale;
}

// Packed C8 MLA row writer: one wave per token row; 576 bf16 in, 656 B out.
// Lanes 0..63 each own 8 latent values (512 = 64 x 8); lanes 0..7 also copy
// 8 rope values each. Tile t = lanes 16t..16t+15.
template <typename SlotT>
__global__ __launch_bounds__(256) void mla_write_c8_kernel(
    const uint16_t *__restrict__ rows_in, uint8_t *__restrict__ cache,
    const SlotT *__restrict__ slots, int64_t rows, int64_t num_slots) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t slot = int64_t(slots[r]);
  if (slot < 0 || slot >= num_slots) return;
  const uint16_t *src = rows_in + r * 576;
  uint8_t *dst = cache + slot * 656;
  u32x4 w = load_u32x4(src + lane * 8);
  float x[8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
    x[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) amax = wave_max_xor(amax, m);  // within 16 lanes
  // Zero tile: scale 0 and zero codes (docs/packed-mla-cache.md:36-37).
  const float scale = c8_scale(amax, 0.0f);
  uint32_t lo = 0, hi = 0;
  if (scale != 0.0f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) lo |= (uint32_t(c8_code(x[i], scale)) & 0xffu) << (8 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) hi |= (uint32_t(c8_code(x[4 + i], scale)) & 0xffu) << (8 * i);
  }
  *reinterpret_cast<u32x2 *>(dst + lane * 8) = u32x2{lo, hi};
  if (lane < 8) store_u32x4(dst + 512 + lane * 16, load_u32x4(src + 512 + lane * 8));
  if ((lane & 15) == 0) *reinterpret_cast<float *>(dst + 640 + (lane >> 4) * 4) = scale;
}

// Fused MLA cache writer: one wave per row (mla_norm_rope_row, mla_row_write.h).
template <typename SlotT, bool PACKED>
__global__ __launch_bounds__(256) void mla_norm_rope_write_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ gamma,
    const uint16_t *__restrict__ cosv, const uint16_t *__restrict__ sinv,
    const SlotT *__restrict__ slots, int64_t rows, float eps, uint8_t *__restrict__ cache,
    int64_t num_slots) {
  constexpr int64_t STRIDE = PACKED ? 656 : 1152;
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t slot = int64_t(slots[r]);
  if (slot < 0 || slot >= num_slots) return;
  mla_norm_rope_row<PACKED>(x + r * 576, gamma, cosv + r * 64, sinv + r * 64, eps,
                            cache + slot * STRIDE, lane);
}

// ---- legacy launchers (native/include/cache_quantization.h:3-7) -------------
// if_cache_quantize: one bf16 row of `width` values -> packed row `*position`
// with one fp32 scale (cache_quantization.cpp:12-38). bits 8 or 4; INT4 nibbles
// are two's complement, low nibble first. Position is read on the device so a
// captured graph follows later host updates of it.
__global__ __launch_bounds__(256) void cache_quantize_kernel(
    const uint16_t *__restrict__ input, uint8_t *__restrict__ packed,
    float *__restrict__ scales, const int64_t *__restrict__ position,
    uint32_t width, uint32_t capacity, uint32_t bits) {
  __shared__ float red[4];
  const int64_t row = *position;
  if (row < 0 || row >= int64_t(capacity)) return;
  const int limit = bits == 8 ? 127 : 7;
  float amax = 0.0f;
  for (uint32_t j = threadIdx.x; j < width; j += blockDim.x)
    amax = fmaxf(amax, fabsf(bf16_bits_to_f32(input[j])));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = wave_max_xor(amax, m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float scale = amax == 0.0f ? 1.0f : __fdiv_rn(amax, float(limit));
  if (threadIdx.x == 0) scales[row] = scale;
  const uint32_t per_byte = 8 / bits, stride = width * bits / 8;
  for (uint32_t b = threadIdx.x; b < stride; b += blockDim.x) {
    uint32_t byte = 0;
    for (uint32_t k = 0; k < per_byte; ++k) {
      // Reference rounding for this entry point: ties away from zero, formed
      // as int(value +- 0.5f) in fp32 (cache_quantization.cpp:30-32).
      const float value = __fdiv_rn(bf16_bits_to_f32(input[b * per_byte + k]), scale);
      int q = int(__fadd_rn(value, value >= 0.0f ? 0.5f : -0.5f));
      q = q > limit ? limit : (q < -limit ? -limit : q);
      byte |= (uint32_t(q) & (bits == 8 ? 0xffu : 0xfu)) << (k * bits);
    }
    packed[int64_t(row) * stride + b] = uint8_t(byte);
  }
}

// if_cache_dequantize: rows 0..*position reconstructed to bf16, rows after it
// written as zero (cache_quantization.cpp:39-57).
__global__ __launch_bounds__(256) void cache_dequantize_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ scales,
    uint16_t *__restrict__ output, const int64_t *__restrict__ position,
    uint32_t width, uint32_t capacity, uint32_t bits) {
  const int64_t last = *position;
  const uint64_t total = uint64_t(width) * capacity;
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * blockDim.x) {
    const uint64_t row = i / width, j = i - row * width;
    float v = 0.0f;
    if (int64_t(row) <= last) {
      const uint8_t byte = packed[row * (width * bits / 8) + j * bits / 8];
      int q = bits == 8 ? int(int8_t(byte)) : int((byte >> ((j & 1) * 4)) & 15);
      if (bits == 4 && q >= 8) q -= 16;
      v = float(q) * scales[row];
    }
    output[i] = uint16_t(f32_to_bf16_bits(v));
  }
}

// Causal candidate ids i<=pos ? i : -1 and length pos+1 per row
// (cache_quantization.cpp:70-85). One thread per (row, candidate).
__global__ __launch_bounds__(256) void packed_attention_metadata_kernel(
    const int64_t *__restrict__ positions, int32_t *__restrict__ indices,
    int32_t *__restrict__ lengths, uint32_t capacity, uint32_t rows) {
  const uint64_t total = uint64_t(rows) * capacity;
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * blockDim.x) {
    const uint64_t row = i / capacity, c = i - row * capacity;
    const int64_t pos = positions[row];
    indices[i] = int64_t(c) <= pos ? int32_t(c) : -1;
    if (c == 0) lengths[row] = int32_t(pos + 1);
  }
}

}  // namespace ifattn

using namespace ifattn;

namespace {
int32_t check_slot_dtype(int32_t dt) {
  if (dt != IFATTN_DTYPE_I32 && dt != IFATTN_DTYPE_I64)
    return fail(IFATTN_EINVAL, "slot mapping dtype must be I32 (4) or I64 (5)");
  return IFATTN_OK;
}
}  // namespace

extern "C" int32_t ifattn_kv_cache_write(const void *k_rows, const void *v_rows, void *k_cache,
                                         void *v_cache, const void *slot_mapping,
                                         int32_t slot_dtype, int64_t rows, int64_t row_bytes,
                                         int64_t num_slots, void *stream) {
  if (check_slot_dtype(slot_dtype)) return IFATTN_EINVAL;
  if (rows < 0 || row_bytes <= 0 || row_bytes % 16 || num_slots <= 0)
    return fail(IFATTN_EINVAL, "kv write: rows>=0, row_bytes>0 multiple of 16, num_slots>0");
  if (!k_rows || !k_cache || !slot_mapping || (!v_rows) != (!v_cache))
    return fail(IFATTN_EINVAL, "kv write: null pointer (V pair must be both set or both null)");
  if (!aligned16(k_rows) || !aligned16(k_cache) || (v_rows && (!aligned16(v_rows) || !aligned16(v_cache))))
    return fail(IFATTN_EINVAL, "kv write: rows and caches must be 16-byte aligned");
  if (rows == 0) return IFATTN_OK;
  const int64_t vecs = row_bytes / 16, total = rows * vecs;
  dim3 grid(unsigned((total + 255) / 256), v_rows ? 2 : 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (slot_dtype == IFATTN_DTYPE_I64)
    kv_write_rows_kernel<int64_t><<<grid, 256, 0, s>>>(
        (const uint8_t *)k_rows, (const uint8_t *)v_rows, (uint8_t *)k_cache, (uint8_t *)v_cache,
        (const int64_t *)slot_mapping, rows, vecs, num_slots);
  else
    kv_write_rows_kernel<int32_t><<<grid, 256, 0, s>>>(
        (const uint8_t *)k_rows, (const uint8_t *)v_rows, (uint8_t *)k_cache, (uint8_t *)v_cache,
        (const int32_t *)slot_mapping, rows, vecs, num_slots);
  return launch_status("kv write");
}

extern "C" int32_t ifattn_kv_cache_write_c8(const void *k_rows, const void *v_rows, void *k_cache,
                                            void *v_cache, void *k_scale, void *v_scale,
                                            const void *slot_mapping, int32_t slot_dtype,
                                            int64_t rows, int32_t kv_heads, int32_t head_dim,
                                            int64_t num_slots, void *stream) {
  if (check_slot_dtype(slot_dtype)) return IFATTN_EINVAL;
  if (rows < 0 || kv_heads <= 0 || head_dim <= 0 || head_dim > 512 || head_dim % 8 || num_slots <= 0)
    return fail(IFATTN_EINVAL, "c8 write: head_dim must be a multiple of 8 in [8,512]");
  if (!k_rows || !k_cache || !k_scale || !slot_mapping || (!v_rows) != (!v_cache) ||
      (!v_cache) != (!v_scale))
    return fail(IFATTN_EINVAL, "c8 write: null pointer");
  if (!aligned16(k_rows) || (v_rows && !aligned16(v_rows)) || !aligned8(k_cache) ||
      (v_cache && !aligned8(v_cache)))
    return fail(IFATTN_EINVAL, "c8 write: rows need 16-byte and caches 8-byte alignment");
  if (rows == 0) return IFATTN_OK;
  const int64_t units = rows * kv_heads;
  dim3 grid(unsigned((units + 3) / 4), v_rows ? 2 : 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (slot_dtype == IFATTN_DTYPE_I64)
    kv_write_c8_kernel<int64_t><<<grid, 256, 0, s>>>(
        (const uint16_t *)k_rows, (const uint16_t *)v_rows, (int8_t *)k_cache, (int8_t *)v_cache,
        (float *)k_scale, (float *)v_scale, (const int64_t *)slot_mapping, rows, kv_heads, head_dim,
        num_slots);
  else
    kv_write_c8_kernel<int32_t><<<grid, 256, 0, s>>>(
        (const uint16_t *)k_rows, (const uint16_t *)v_rows, (int8_t *)k_cache, (int8_t *)v_cache,
        (float *)k_scale, (float *)v_scale, (const int32_t *)slot_mapping, rows, kv_heads, head_dim,
        num_slots);
  return launch_status("c8 write");
}

extern "C" int32_t ifattn_mla_cache_write_c8(const void *rows_in, void *cache, const void *slot_mapping,
                                             int32_t slot_dtype, int64_t rows, int64_t num_slots,
                                             void *stream) {
  if (check_slot_dtype(slot_dtype)) return IFATTN_EINVAL;
  if (!rows_in || !cache || !slot_mapping || rows < 0 || num_slots <= 0)
    return fail(IFATTN_EINVAL, "mla c8 write: null pointer or bad extent");
  if (!aligned16(rows_in) || !aligned16(cache))
    return fail(IFATTN_EINVAL, "mla c8 write: rows and cache must be 16-byte aligned");
  if (rows == 0) return IFATTN_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = unsigned((rows + 3) / 4);
  if (slot_dtype == IFATTN_DTYPE_I64)
    mla_write_c8_kernel<int64_t><<<grid, 256, 0, s>>>((const uint16_t *)rows_in, (uint8_t *)cache,
                                                      (const int64_t *)slot_mapping, rows, num_slots);
  else
    mla_write_c8_kernel<int32_t><<<grid, 256, 0, s>>>((const uint16_t *)rows_in, (uint8_t *)cache,
                                                      (const int32_t *)slot_mapping, rows, num_slots);
  return launch_status("mla c8 write");
}

extern "C" int32_t ifattn_mla_norm_rope_cache_write(const void *x, const void *gamma,
                                                    const void *cos, const void *sin,
                                                    const void *slot_mapping, int32_t slot_dtype,
                                                    int64_t rows, float eps, void *cache,
                                                    int32_t packed, int64_t num_slots,
                                                    void *stream) {
  if (check_slot_dtype(slot_dtype)) return IFATTN_EINVAL;
  if (!x || !gamma || !cos || !sin || !slot_mapping || !cache || num_slots <= 0)
    return fail(IFATTN_EINVAL, "mla norm/rope write: null pointer or bad extent");
  if (rows < 1 || rows > 4096)
    return fail(IFATTN_EINVAL, "mla norm/rope write: rows must be 1..4096");
  if (!aligned16(x) || !aligned16(gamma) || !aligned4(cos) || !aligned4(sin) || !aligned16(cache))
    return fail(IFATTN_EINVAL, "mla norm/rope write: x, gamma, cache 16-byte and cos/sin 4-byte aligned");
  if (!(eps > 0.0f) || eps > 1.0f)
    return fail(IFATTN_EINVAL, "mla norm/rope write: eps must be in (0, 1]");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = unsigned((rows + 3) / 4);
  auto go = [&](auto slot_tag, auto packed_tag) {
    using SlotT = decltype(slot_tag);
    mla_norm_rope_write_kernel<SlotT, decltype(packed_tag)::value><<<grid, 256, 0, s>>>(
        (const uint16_t *)x, (const uint16_t *)gamma, (const uint16_t *)cos, (const uint16_t *)sin,
        (const SlotT *)slot_mapping, rows, eps, (uint8_t *)cache, num_slots);
  };
  if (slot_dtype == IFATTN_DTYPE_I64) {
    if (packed) go(int64_t{}, std::true_type{}); else go(int64_t{}, std::false_type{});
  } else {
    if (packed) go(int32_t{}, std::true_type{}); else go(int32_t{}, std::false_type{});
  }
  return launch_status("mla norm/rope write");
}

// Legacy signatures return void like the reference's launchers; failures are
// recorded in ifattn_last_error().
extern "C" void if_cache_quantize(void *input, void *packed, void *scales, void *position,
                                  uint32_t width, uint32_t capacity, uint32_t bits, void *stream) {
  if (!input || !packed || !scales || !position || !width || !capacity ||
      (bits != 8 && bits != 4) || (bits == 4 && (width & 1))) {
    fail(IFATTN_EINVAL, "if_cache_quantize: bad arguments");
    return;
  }
  cache_quantize_kernel<<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(
      (const uint16_t *)input, (uint8_t *)packed, (float *)scales, (const int64_t *)position, width,
      capacity, bits);
  launch_status("if_cache_quantize");
}

extern "C" void if_cache_dequantize(void *packed, void *scales, void *output, void *position,
                                    uint32_t width, uint32_t capacity, uint32_t bits, void *stream) {
  if (!packed || !scales || !output || !position || !width || !capacity ||
      (bits != 8 && bits != 4) || (bits == 4 && (width & 1))) {
    fail(IFATTN_EINVAL, "if_cache_dequantize: bad arguments");
    return;
  }
  const uint64_t total = uint64_t(width) * capacity;
  const unsigned grid = unsigned(total / 256 + 1 < 4096 ? total / 256 + 1 : 4096);
  cache_dequantize_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      (const uint8_t *)packed, (const float *)scales, (uint16_t *)output, (const int64_t *)position,
      width, capacity, bits);
  launch_status("if_cache_dequantize");
}

extern "C" void if_packed_attention_metadata_batch(void *position, void *indices, void *length,
                                                   uint32_t capacity, uint32_t rows, void *stream) {
  if (!position || !indices || !length || !capacity || !rows) {
    fail(IFATTN_EINVAL, "if_packed_attention_metadata: bad arguments");
    return;
  }
  const uint64_t total = uint64_t(rows) * capacity;
  const unsigned grid = unsigned(total / 256 + 1 < 2048 ? total / 256 + 1 : 2048);
  packed_attention_metadata_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      (const int64_t *)position, (int32_t *)indices, (int32_t *)length, capacity, rows);
  launch_status("if_packed_attention_metadata");
}

extern "C" void if_packed_attention_metadata(void *position, void *indices, void *length,
                                             uint32_t capacity, void *stream) {
  if_packed_attention_metadata_batch(position, indices, length, capacity, 1, stream);
}
