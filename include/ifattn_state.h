/* ifattn attention state: one MLA attention layer's cache, page binding,
 * block table and side buffers as one object, the counterpart of the
 * reference's AttentionState (native/src/openpangu_decoder_state.h:16-48).
 *
 * Unlike the rest of the C ABI this object owns device memory: its buffers are
 * allocated with hipMalloc on the current device the first time a call needs
 * them (ifattn_attention_state_buffers, _upload_table, _set_length, _attend)
 * and freed by ifattn_attention_state_destroy. Host-only calls (_geometry,
 * _pages, _append, _blocks) never touch the device. Status codes and
 * ifattn_last_error() are those of ifattn.h.
 */
#ifndef IFATTN_STATE_H
#define IFATTN_STATE_H
#include <stdint.h>

#include "ifattn_host.h"
#ifdef __cplusplus
extern "C" {
#endif

typedef struct ifattn_attention_state ifattn_attention_state;

/* Cache formats, as AttentionState(bits, capacity, packed, ...) picks them. */
#define IFATTN_STATE_BF16 0     /* bits 16: bf16 rows of 576, 16-token pages      */
#define IFATTN_STATE_PACKED_C8 1 /* packed: 656-byte C8 rows, 32-token pages      */
#define IFATTN_STATE_ROW_QUANT 2 /* bits 8 or 4: if_cache_quantize rows + scales */

typedef struct {
  uint32_t format;         /* IFATTN_STATE_* */
  uint32_t page_tokens;    /* 16 (bf16, row-quantized) or 32 (packed C8) */
  uint32_t row_bytes;      /* 1152, 656, or 576 * bits / 8 */
  uint32_t num_blocks;     /* pages of the cache over all residents (0 for row-quantized) */
  uint32_t table_entries;  /* block-table row: capacity/page, or ceil(context/16) with a context */
  uint32_t heads;          /* query heads of the layer (the query and output buffers) */
  uint64_t cache_bytes;
} ifattn_attention_state_geometry;

typedef struct {
  void *cache;       /* geometry.cache_bytes */
  int32_t *table;    /* [1, table_entries] int32 */
  float *scales;     /* [capacity] fp32, row-quantized caches only (else NULL) */
  uint16_t *query;   /* [1, heads, 576] bf16 */
  uint16_t *out;     /* [1, heads, 512] bf16 */
  int32_t *indices;  /* [1, 512] int32 candidate positions (packed C8 sparse attention) */
  int32_t *kv_len;   /* [1] int32 keys of the query row (_set_length) */
  uint16_t *sink_keys;   /* [128, 576] bf16, zero-initialized */
  uint16_t *sink_values; /* [128, 512] bf16, zero-initialized */
} ifattn_attention_state_buffers;

/* AttentionState(bits, capacity, packed, residents, shared, context)
 * (openpangu_decoder_state.h:24-40) with `heads` query heads (the reference's
 * TP share is 6). packed selects the C8 row; otherwise bits 16 is bf16 and
 * bits 8 or 4 the row-quantized cache (one resident only). capacity is the
 * cached tokens per resident; context > 0 makes the table a ring of
 * ceil(context / 16) absolute logical pages over the resident's pages. */
int32_t ifattn_attention_state_create(uint32_t bits, uint32_t capacity, int32_t packed,
                                      uint32_t residents, int32_t shared, uint32_t context,
                                      uint32_t heads, ifattn_attention_state **out);
void ifattn_attention_state_destroy(ifattn_attention_state *state);
int32_t ifattn_attention_state_geometry_of(const ifattn_attention_state *state,
                                           ifattn_attention_state_geometry *out);
/* The page binding (ResidentPages(page, capacity, residents, shared)); select,
 * bind and release it with the ifattn_pages_* calls. Owned by the state. */
int32_t ifattn_attention_state_pages(ifattn_attention_state *state, ifattn_pages **out);
/* AttentionState::append (openpangu_decoder_state.h:41-44): the physical row of
 * an absolute position for the selected resident (position mod capacity when
 * the state has a context; positions at or past the context are rejected). */
int32_t ifattn_attention_state_append(const ifattn_attention_state *state, uint32_t position,
                                      uint64_t *physical);
/* AttentionState::blocks (openpangu_decoder_state.h:45-47): the selected
 * resident's table row, ring mode when the state has a context. *entries
 * receives table_entries; table may be NULL to query it. */
int32_t ifattn_attention_state_blocks(const ifattn_attention_state *state, int32_t *table,
                                      uint32_t capacity, uint32_t *entries);
/* Device buffers (allocated on the first call). */
int32_t ifattn_attention_state_buffers_of(ifattn_attention_state *state,
                                          ifattn_attention_state_buffers *out);
/* Upload blocks() into the device table on `stream`. */
int32_t ifattn_attention_state_upload_table(ifattn_attention_state *state, void *stream);
/* Write kv_len into the device length (a one-thread kernel, graph safe). */
int32_t ifattn_attention_state_set_length(ifattn_attention_state *state, int32_t kv_len,
                                          void *stream);
/* Attention of the query buffer into the output buffer over the device table
 * and length: bf16 states run the window attention (window 0 = every cached
 * key), packed C8 states the sparse attention over the indices buffer; with
 * sinks != 0 the 128 sink rows join the softmax. Row-quantized states run the
 * window attention over their int8 / int4 codes and row scales directly
 * (ifattn_mla_window_attention_rowq), where the reference first dequantizes
 * the cache to bf16 (token_executor.h:806-822). Scale 1/sqrt(192). */
int32_t ifattn_attention_state_attend(ifattn_attention_state *state, int32_t window,
                                      int32_t sinks, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* IFATTN_STATE_H */
