// C-ABI shim over the REFERENCE's own host metadata headers, compiled in place
// from /root/reference (native/src/page_binding.h, native/include/sequence_batch.h,
// native/include/sliding_window_layout.h) into oracle/_ref/libref_meta.so.
// TEST INFRASTRUCTURE ONLY: used to check the product's host metadata and to
// write the golden fixtures under tests/golden/. No reference source is copied.
#include <cstring>
#include <exception>

#include "include/sequence_batch.h"
#include "include/sliding_window_layout.h"
#include "src/page_binding.h"

using inferfabric::execution::SequenceBatch;
using inferfabric::execution::SequenceSlice;
using inferfabric::state::ResidentPages;

namespace {
template <typename F>
int guarded(F &&f) {
  try {
    f();
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}
}  // namespace

extern "C" {
struct RefSlice {
  uint32_t resident, position, tokens;
  int32_t sample;
};

int ref_pages_create(uint32_t page_tokens, uint32_t logical, uint32_t slots, int shared, void **out) {
  return guarded([&] { *out = new ResidentPages(page_tokens, logical, slots, shared != 0); });
}
void ref_pages_destroy(void *p) { delete static_cast<ResidentPages *>(p); }
int ref_pages_select(void *p, uint32_t slot) {
  return guarded([&] { static_cast<ResidentPages *>(p)->select(slot); });
}
int ref_pages_bind(void *p, const int32_t *ids, uint64_t n) {
  return guarded([&] { static_cast<ResidentPages *>(p)->bind(std::vector<int32_t>(ids, ids + n)); });
}
int ref_pages_release(void *p, uint32_t slot) {
  return guarded([&] { static_cast<ResidentPages *>(p)->release(slot); });
}
int ref_pages_append(void *p, uint32_t slot, uint32_t pos, uint64_t *out) {
  return guarded([&] {
    auto *r = static_cast<ResidentPages *>(p);
    *out = slot == UINT32_MAX ? r->append(pos) : r->append(slot, pos);
  });
}
int ref_pages_batch_table(void *p, const int32_t *res, uint64_t n, uint32_t entries, int ring,
                          int32_t *out) {
  return guarded([&] {
    auto t = static_cast<ResidentPages *>(p)->batch_table(std::vector<int32_t>(res, res + n),
                                                          entries, ring != 0);
    std::memcpy(out, t.data(), t.size() * 4);
  });
}
int ref_pages_copy_plan(void *p, uint32_t src, uint32_t dst, uint32_t completed, int windowed,
                        uint64_t field_bytes, uint64_t *ranges, uint64_t cap, uint64_t *count) {
  return guarded([&] {
    auto plan = static_cast<ResidentPages *>(p)->copy_plan(src, dst, completed, windowed != 0,
                                                           field_bytes);
    *count = plan.size();
    for (size_t i = 0; i < plan.size() && i < cap; ++i) {
      ranges[3 * i] = plan[i].source;
      ranges[3 * i + 1] = plan[i].destination;
      ranges[3 * i + 2] = plan[i].bytes;
    }
  });
}
int ref_page_spans(const int32_t *ids, uint64_t n, uint64_t page_bytes, uint64_t field_bytes,
                   uint64_t *spans, uint64_t cap, uint64_t *count) {
  return guarded([&] {
    auto s = inferfabric::state::page_spans(std::vector<int32_t>(ids, ids + n), page_bytes, field_bytes);
    *count = s.size();
    for (size_t i = 0; i < s.size() && i < cap; ++i) {
      spans[2 * i] = s[i].offset;
      spans[2 * i + 1] = s[i].bytes;
    }
  });
}
int ref_sequence_batch(const RefSlice *sl, uint64_t n, uint32_t cap, uint32_t budget,
                       uint32_t context, uint64_t rows_cap, int32_t *starts, int32_t *query_ends,
                       int32_t *prior, int32_t *kv, int32_t *residents, int32_t *positions,
                       int32_t *row_res, int64_t *lengths, uint32_t *sample_rows,
                       uint32_t *sample_res, uint64_t *rows, uint64_t *samples) {
  return guarded([&] {
    std::vector<SequenceSlice> v;
    for (uint64_t i = 0; i < n; ++i)
      v.push_back({sl[i].resident, sl[i].position, sl[i].tokens, sl[i].sample != 0});
    auto b = SequenceBatch::make(v, cap, budget, context);
    if (b.positions.size() > rows_cap) throw std::runtime_error("rows");
    auto put = [](auto *d, const auto &x) { if (d && !x.empty()) std::memcpy(d, x.data(), x.size() * sizeof(x[0])); };
    put(starts, b.starts); put(query_ends, b.query_ends); put(prior, b.prior_lengths);
    put(kv, b.kv_lengths); put(residents, b.residents); put(positions, b.positions);
    put(row_res, b.row_residents); put(lengths, b.lengths); put(sample_rows, b.sample_rows);
    put(sample_res, b.sample_residents);
    *rows = b.positions.size();
    *samples = b.sample_rows.size();
  });
}

int ref_window_layout(uint32_t context, uint32_t window, uint32_t chunk, uint32_t page,
                      uint32_t *pages, uint32_t *entries) {
  return guarded([&] {
    inferfabric::state::SlidingWindowLayout l(context, window, chunk, page);
    *pages = l.physical_pages;
    *entries = l.table_entries();
  });
}
int ref_window_append(uint32_t context, uint32_t window, uint32_t chunk, uint32_t page,
                      uint32_t position, uint32_t *slot) {
  return guarded([&] {
    inferfabric::state::SlidingWindowLayout l(context, window, chunk, page);
    *slot = l.append(position);
  });
}
}
