// C ABI over the host metadata classes of page_table.h. Exceptions never cross
// the boundary: each call maps them to IFATTN_EINVAL plus the message.
#include <cstring>
#include <exception>
#include <new>

#include "../../include/ifattn_host.h"
#include "ifattn_internal.h"
#include "page_table.h"

struct ifattn_pages {
  ifattn::host::ResidentPageTable table;
};

namespace {
template <typename F>
int32_t guarded(F &&f) {
  try {
    f();
    return IFATTN_OK;
  } catch (const std::exception &e) {
    return ifattn::fail(IFATTN_EINVAL, e.what());
  } catch (...) {
    return ifattn::fail(IFATTN_EINVAL, "unknown host metadata failure");
  }
}
void require(bool ok, const char *what) {
  if (!ok) throw std::runtime_error(what);
}
}  // namespace

extern "C" int32_t ifattn_pages_create(uint32_t page_tokens, uint32_t logical_tokens,
                                       uint32_t slots, int32_t shared, ifattn_pages **out) {
  return guarded([&] {
    require(out != nullptr, "null output handle");
    *out = nullptr;
    *out = new ifattn_pages{ifattn::host::ResidentPageTable(page_tokens, logical_tokens, slots,
                                                            shared != 0)};
  });
}

extern "C" void ifattn_pages_destroy(ifattn_pages *pages) { delete pages; }

extern "C" int32_t ifattn_pages_select(ifattn_pages *pages, uint32_t slot) {
  return guarded([&] {
    require(pages != nullptr, "null page table");
    pages->table.select(slot);
  });
}

extern "C" int32_t ifattn_pages_bind(ifattn_pages *pages, const int32_t *ids, uint64_t count) {
  return guarded([&] {
    require(pages != nullptr && (ids != nullptr || count == 0), "null page table or ids");
    pages->table.bind(std::vector<int32_t>(ids, ids + count));
  });
}

extern "C" int32_t ifattn_pages_release(ifattn_pages *pages, uint32_t slot) {
  return guarded([&] {
    require(pages != nullptr, "null page table");
    pages->table.release(slot);
  });
}

extern "C" int32_t ifattn_pages_owned(const ifattn_pages *pages, uint32_t slot, int32_t *ids,
                                      uint64_t capacity, uint64_t *count) {
  return guarded([&] {
    require(pages != nullptr && count != nullptr, "null page table or count");
    const auto &own = pages->table.pages(slot);
    *count = own.size();
    if (ids) {
      require(capacity >= own.size(), "owned page output too small");
      std::memcpy(ids, own.data(), own.size() * sizeof(int32_t));
    }
  });
}

extern "C" int32_t ifattn_pages_append(const ifattn_pages *pages, uint32_t slot,
                                       uint32_t position, uint64_t *physical) {
  return guarded([&] {
    require(pages != nullptr && physical != nullptr, "null page table or output");
    const uint32_t s = slot == UINT32_MAX ? pages->table.active() : slot;
    *physical = pages->table.slot_of(s, position);
  });
}

extern "C" int32_t ifattn_pages_slot_mapping(const ifattn_pages *pages,
                                             const int32_t *row_residents,
                                             const int32_t *positions, uint64_t rows,
                                             int64_t *out) {
  return guarded([&] {
    require(pages != nullptr && (rows == 0 || (row_residents && positions && out)),
            "null slot mapping argument");
    // Resolve every row before writing any output.
    std::vector<int64_t> tmp(rows);
    for (uint64_t r = 0; r < rows; ++r) {
      require(row_residents[r] >= 0 && positions[r] >= 0, "negative resident or position");
      tmp[r] = int64_t(pages->table.slot_of(uint32_t(row_residents[r]), uint32_t(positions[r])));
    }
    if (rows) std::memcpy(out, tmp.data(), rows * sizeof(int64_t));
  });
}

extern "C" int32_t ifattn_pages_batch_table(const ifattn_pages *pages, const int32_t *residents,
                                            uint64_t count, uint32_t entries, int32_t ring,
                                            int32_t *out) {
  return guarded([&] {
    require(pages != nullptr && out != nullptr && (residents != nullptr || count == 0),
            "null batch table argument");
    auto t = pages->table.batch_table(std::vector<int32_t>(residents, residents + count), entries,
                                      ring != 0);
    std::memcpy(out, t.data(), t.size() * sizeof(int32_t));
  });
}

extern "C" int32_t ifattn_pages_copy_plan(const ifattn_pages *pages, uint32_t source,
                                          uint32_t destination, uint32_t completed_tokens,
                                          int32_t windowed, uint64_t field_bytes,
                                          uint64_t *ranges, uint64_t capacity, uint64_t *count) {
  return guarded([&] {
    require(pages != nullptr && count != nullptr, "null copy plan argument");
    auto plan = pages->table.copy_plan(source, destination, completed_tokens, windowed != 0,
                                       field_bytes);
    *count = plan.size();
    if (ranges) {
      require(capacity >= plan.size(), "copy plan output too small");
      for (size_t i = 0; i < plan.size(); ++i) {
        ranges[3 * i] = plan[i].source;
        ranges[3 * i + 1] = plan[i].destination;
        ranges[3 * i + 2] = plan[i].bytes;
      }
    }
  });
}

extern "C" int32_t ifattn_page_spans(const int32_t *ids, uint64_t count, uint64_t page_bytes,
                                     uint64_t field_bytes, uint64_t *spans, uint64_t capacity,
                                     uint64_t *span_count) {
  return guarded([&] {
    require(span_count != nullptr && (ids != nullptr || count == 0), "null page span argument");
    auto out = ifattn::host::coalesce_page_spans(std::vector<int32_t>(ids, ids + count), page_bytes,
                                                 field_bytes);
    *span_count = out.size();
    if (spans) {
      require(capacity >= out.size(), "page span output too small");
      for (size_t i = 0; i < out.size(); ++i) {
        spans[2 * i] = out[i].offset;
        spans[2 * i + 1] = out[i].bytes;
      }
    }
  });
}

extern "C" int32_t ifattn_sequence_batch_make(
    const ifattn_sequence_slice *slices, uint64_t count, uint32_t resident_capacity,
    uint32_t token_budget, uint32_t context, uint64_t rows_capacity, int32_t *starts,
    int32_t *query_ends, int32_t *prior_lengths, int32_t *kv_lengths, int32_t *residents,
    int32_t *positions, int32_t *row_residents, int64_t *lengths, uint32_t *sample_rows,
    uint32_t *sample_residents, uint64_t *rows, uint64_t *samples) {
  return guarded([&] {
    require(slices != nullptr || count == 0, "null slices");
    std::vector<ifattn::host::PackedSlice> in(count);
    for (uint64_t i = 0; i < count; ++i)
      in[i] = {slices[i].resident, slices[i].position, slices[i].tokens, slices[i].sample != 0};
    auto b = ifattn::host::PackedBatch::make(in, resident_capacity, token_budget, context);
    require(b.positions.size() <= rows_capacity, "row outputs too small for the batch");
    auto put = [](auto *dst, const auto &v) {
      if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(v[0]));
    };
    put(starts, b.starts);
    put(query_ends, b.query_ends);
    put(prior_lengths, b.prior_lengths);
    put(kv_lengths, b.kv_lengths);
    put(residents, b.residents);
    put(positions, b.positions);
    put(row_residents, b.row_residents);
    put(lengths, b.lengths);
    put(sample_rows, b.sample_rows);
    put(sample_residents, b.sample_residents);
    if (rows) *rows = b.positions.size();
    if (samples) *samples = b.sample_rows.size();
  });
}

extern "C" int32_t ifattn_window_layout(uint32_t context, uint32_t window, uint32_t chunk,
                                        uint32_t page_tokens, uint32_t *physical_pages,
                                        uint32_t *table_entries) {
  return guarded([&] {
    const ifattn::host::WindowRing ring(context, window, chunk, page_tokens);
    if (physical_pages) *physical_pages = ring.pages;
    if (table_entries) *table_entries = ring.entries();
  });
}

extern "C" int32_t ifattn_window_table(uint32_t context, uint32_t window, uint32_t chunk,
                                       uint32_t page_tokens, const int32_t *owned,
                                       uint64_t owned_count, int32_t *table) {
  return guarded([&] {
    const ifattn::host::WindowRing ring(context, window, chunk, page_tokens);
    require(table != nullptr, "null table output");
    require(owned == nullptr || owned_count == ring.pages, "owned pages must number the ring pages");
    if (owned) {
      require(!ifattn::host::has_duplicates(std::vector<int32_t>(owned, owned + owned_count)),
              "owned pages alias");
      for (uint64_t i = 0; i < owned_count; ++i) require(owned[i] >= 0, "negative page id");
    }
    for (uint32_t l = 0; l < ring.entries(); ++l) {
      const uint32_t ph = ring.physical_page(l);
      table[l] = owned ? owned[ph] : int32_t(ph);
    }
  });
}

extern "C" int32_t ifattn_window_slots(uint32_t context, uint32_t window, uint32_t chunk,
                                       uint32_t page_tokens, const int32_t *owned,
                                       uint64_t owned_count, const uint32_t *positions,
                                       uint64_t count, int64_t *slots) {
  return guarded([&] {
    const ifattn::host::WindowRing ring(context, window, chunk, page_tokens);
    require(slots != nullptr && (positions != nullptr || count == 0), "null slot argument");
    require(owned == nullptr || owned_count == ring.pages, "owned pages must number the ring pages");
    for (uint64_t i = 0; i < count; ++i) require(positions[i] < context, "sliding append bounds");
    for (uint64_t i = 0; i < count; ++i) {
      const uint32_t s = ring.slot(positions[i]);
      const uint32_t ph = s / page_tokens;
      slots[i] = int64_t(owned ? owned[ph] : int32_t(ph)) * page_tokens + s % page_tokens;
    }
  });
}
