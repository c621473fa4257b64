/* ifattn host metadata C ABI: page ownership, slot mapping, block tables and
 * the packed varlen batch layout that feed the device kernels.
 *
 * These replace the reference's host C++ classes on the same path; every call
 * validates its whole input first and leaves state unchanged on rejection.
 * Status codes and ifattn_last_error() are those of ifattn.h.
 */
#ifndef IFATTN_HOST_H
#define IFATTN_HOST_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct ifattn_pages ifattn_pages;

/* ResidentPages(page_tokens, logical_tokens, slots, shared)
 * (native/src/page_binding.h:65-82). */
int32_t ifattn_pages_create(uint32_t page_tokens, uint32_t logical_tokens, uint32_t slots,
                            int32_t shared, ifattn_pages **out);
void ifattn_pages_destroy(ifattn_pages *pages);
/* ResidentPages::select (page_binding.h:83-86). */
int32_t ifattn_pages_select(ifattn_pages *pages, uint32_t slot);
/* ResidentPages::bind for the selected resident (page_binding.h:87-106). */
int32_t ifattn_pages_bind(ifattn_pages *pages, const int32_t *ids, uint64_t count);
/* The selected resident (ResidentPages::select's argument; 0 initially). */
int32_t ifattn_pages_selected(const ifattn_pages *pages, uint32_t *slot);
/* ResidentPages::release (page_binding.h:107-111). */
int32_t ifattn_pages_release(ifattn_pages *pages, uint32_t slot);
/* Owned pages of a resident; *count receives the number, ids may be NULL to query it. */
int32_t ifattn_pages_owned(const ifattn_pages *pages, uint32_t slot, int32_t *ids,
                           uint64_t capacity, uint64_t *count);
/* ResidentPages::append(slot, position): physical token row
 * table[pos/page]*page + pos%page (page_binding.h:115-126). slot UINT32_MAX
 * means the selected resident. */
int32_t ifattn_pages_append(const ifattn_pages *pages, uint32_t slot, uint32_t position,
                            uint64_t *physical);
/* Slot mapping of a packed batch: out[r] = append(row_residents[r], positions[r])
 * for every row (the per-row loop of native/src/token_executor.h:1334-1348). */
int32_t ifattn_pages_slot_mapping(const ifattn_pages *pages, const int32_t *row_residents,
                                  const int32_t *positions, uint64_t rows, int64_t *out);
/* ResidentPages::batch_table (page_binding.h:146-160): [count, entries] int32. */
int32_t ifattn_pages_batch_table(const ifattn_pages *pages, const int32_t *residents,
                                 uint64_t count, uint32_t entries, int32_t ring, int32_t *out);

/* StateCopyRange / PageSpan (page_binding.h:14-35,161-187). ranges receive
 * {source, destination, bytes} triples; spans receive {offset, bytes} pairs.
 * *count is the number produced; capacity is in entries. */
int32_t ifattn_pages_copy_plan(const ifattn_pages *pages, uint32_t source, uint32_t destination,
                               uint32_t completed_tokens, int32_t windowed, uint64_t field_bytes,
                               uint64_t *ranges, uint64_t capacity, uint64_t *count);
int32_t ifattn_page_spans(const int32_t *ids, uint64_t count, uint64_t page_bytes,
                          uint64_t field_bytes, uint64_t *spans, uint64_t capacity,
                          uint64_t *span_count);

/* SequenceBatch::make (native/include/sequence_batch.h:23-59). */
typedef struct {
  uint32_t resident, position, tokens;
  int32_t sample;
} ifattn_sequence_slice;

/* Outputs (caller-sized): starts[count+1] (== cu_seqlens_q), query_ends[count],
 * prior_lengths[count], kv_lengths[count], residents[count]; per row
 * positions[rows], row_residents[rows], lengths[rows] (int64); sample_rows /
 * sample_residents[count]. rows_capacity must be >= the total token count, which
 * is returned in *rows; *samples receives the number of sampled rows. Any
 * output pointer may be NULL. */
int32_t ifattn_sequence_batch_make(const ifattn_sequence_slice *slices, uint64_t count,
                                   uint32_t resident_capacity, uint32_t token_budget,
                                   uint32_t context, uint64_t rows_capacity, int32_t *starts,
                                   int32_t *query_ends, int32_t *prior_lengths,
                                   int32_t *kv_lengths, int32_t *residents, int32_t *positions,
                                   int32_t *row_residents, int64_t *lengths,
                                   uint32_t *sample_rows, uint32_t *sample_residents,
                                   uint64_t *rows, uint64_t *samples);

/* Sliding-window page ring (SlidingWindowLayout, native/include/sliding_window_layout.h:9-33):
 * a window of `window` tokens whose chunk of `chunk` rows is written before it
 * is queried keeps physical_pages pages of page_tokens tokens; the block table
 * has table_entries absolute logical pages, logical page l -> ring page
 * l % physical_pages. Rejects a zero argument, chunk > context and overflow. */
int32_t ifattn_window_layout(uint32_t context, uint32_t window, uint32_t chunk,
                             uint32_t page_tokens, uint32_t *physical_pages,
                             uint32_t *table_entries);
/* Block-table row [table_entries]: ring page ids, or owned[ring page] when the
 * resident owns `owned` (physical_pages distinct ids). */
int32_t ifattn_window_table(uint32_t context, uint32_t window, uint32_t chunk,
                            uint32_t page_tokens, const int32_t *owned, uint64_t owned_count,
                            int32_t *table);
/* Physical token row of each absolute position (the append of
 * sliding_window_layout.h:28-31 through the same page ids as the table). */
int32_t ifattn_window_slots(uint32_t context, uint32_t window, uint32_t chunk,
                            uint32_t page_tokens, const int32_t *owned, uint64_t owned_count,
                            const uint32_t *positions, uint64_t count, int64_t *slots);

#ifdef __cplusplus
}
#endif
#endif /* IFATTN_HOST_H */
