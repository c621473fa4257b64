/* Legacy cache storage launchers, same symbols and argument order as the
 * reference's native/include/cache_quantization.h:3-7, implemented for gfx950.
 *
 * if_cache_quantize(input, packed, scales, position, width, capacity, bits, stream)
 *   one bf16 row -> packed INT8/INT4 row *position plus one fp32 scale
 *   (scale = max|x|/limit, 1.0 for a zero row; ties-away rounding, as
 *   native/kernels/cache_quantization.cpp:20-34).
 * if_cache_dequantize(packed, scales, output, position, width, capacity, bits, stream)
 *   rows <= *position reconstructed to bf16, later rows zero (:39-57).
 * if_packed_attention_metadata[_batch](position, indices, length, capacity, [rows,] stream)
 *   causal candidates i<=pos ? i : -1 and length pos+1 (:70-91).
 * position is a device int64 read at run time (graph-replay safe). They return
 * void like the originals; a rejected call records ifattn_last_error().
 */
#ifndef IFATTN_CACHE_QUANTIZATION_H
#define IFATTN_CACHE_QUANTIZATION_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
void if_cache_quantize(void *input, void *packed, void *scales, void *position, uint32_t width,
                       uint32_t capacity, uint32_t bits, void *stream);
void if_cache_dequantize(void *packed, void *scales, void *output, void *position, uint32_t width,
                         uint32_t capacity, uint32_t bits, void *stream);
void if_packed_attention_metadata(void *position, void *indices, void *length, uint32_t capacity,
                                  void *stream);
void if_packed_attention_metadata_batch(void *position, void *indices, void *length,
                                        uint32_t capacity, uint32_t rows, void *stream);
#ifdef __cplusplus
}
#endif
#endif
