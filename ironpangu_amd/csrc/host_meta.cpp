// Host metadata that feeds the cache-write and attention kernels: page
// ownership, slot mappings, block tables, page spans, state-copy plans and the
// packed varlen (cu_seqlens) layout. Cache contents never visit the host.
//
// Design: one flat page map per pool and no per-resident objects. Each call
// validates its whole input in a first pass and then emits its result in a
// second pass straight into the caller's buffers, so a rejected call writes
// nothing and leaves the pool as it was. No exception crosses the boundary;
// errors are a status plus ifattn_last_error().
//
// Observable behaviour (results and the conditions that reject a call) is the
// contract of the reference's host metadata, pinned bit for bit by
// tests/test_host_meta.py against that code compiled in place:
//   pool, bind, release, slot  native/src/page_binding.h:37-126
//   tables                     native/src/page_binding.h:132-160
//   copy plans, page spans     native/src/page_binding.h:19-35,161-187
//   packed batch               native/include/sequence_batch.h:23-59
//   window ring                native/include/sliding_window_layout.h:9-33
#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/ifattn_host.h"
#include "ifattn_internal.h"

// Pool of R residents x P pages per resident (P = logical_tokens / page_tokens).
//  map[r * P + i]  physical page backing logical page i of resident r
//  held[r]         logical pages of r that are backed: always P in fixed mode,
//                  0..P in shared mode (a partial reservation is allowed)
//  owner[page]     resident holding a physical page, -1 when free
// Fixed mode keeps resident r on pages [rP, rP + P) and only lets it permute
// them; shared mode lets it claim any free pages.
struct ifattn_pages {
  uint32_t page_tokens = 0, logical_tokens = 0, per_resident = 0, residents = 0, selected = 0;
  bool shared = false;
  std::vector<int32_t> map;
  std::vector<uint32_t> held;
  std::vector<int8_t> owner;
  // Alias detection without sorting: page p was seen in the current check when
  // seen[p] == epoch.
  std::vector<uint32_t> seen;
  uint32_t epoch = 0;

  uint32_t pool_pages() const { return per_resident * residents; }
  const int32_t *row(uint32_t r) const { return map.data() + size_t(r) * per_resident; }
  uint32_t next_epoch() {
    if (++epoch == 0) {  // wrapped: restart the stamps
      std::fill(seen.begin(), seen.end(), 0u);
      epoch = 1;
    }
    return epoch;
  }
  // Physical token row of (resident, position), or -1 when the position is
  // outside the resident's backed pages.
  int64_t physical_row(uint32_t r, uint32_t position) const {
    if (position >= logical_tokens) return -1;
    const uint32_t logical = position / page_tokens;
    if (logical >= held[r]) return -1;
    return int64_t(row(r)[logical]) * page_tokens + position % page_tokens;
  }
};

namespace {

using ifattn::fail;

constexpr uint32_t kMaxResidents = 64;
constexpr uint64_t kIdLimit = 0x7fffffffu;

int32_t reject(const char *what) { return fail(IFATTN_EINVAL, what); }

// Sliding-window page ring: a window whose chunk rows are written before the
// chunk is queried has window + chunk - 1 tokens live at once, which touch at
// most ceil((window + chunk - 2) / page) + 1 pages; never more than the whole
// context needs. Logical page l lives in ring page l % pages.
struct Ring {
  uint32_t context = 0, page_tokens = 0, pages = 0, entries = 0;
};
int32_t make_ring(uint32_t context, uint32_t window, uint32_t chunk, uint32_t page, Ring *out) {
  if (!context || !window || !chunk || !page || chunk > context)
    return reject("window ring: zero argument or chunk longer than the context");
  const uint64_t live = uint64_t(window) + chunk - 1;
  const uint64_t touched = (live + page - 2) / page + 1;
  const uint64_t whole = (uint64_t(context) + page - 1) / page;
  const uint64_t pages = std::min(touched, whole);
  if (pages * page > 0xffffffffull) return reject("window ring: capacity overflows 32 bits");
  out->context = context;
  out->page_tokens = page;
  out->pages = uint32_t(pages);
  out->entries = uint32_t(whole);
  return IFATTN_OK;
}

}  // namespace

// ------------------------------------------------------------------ pool

extern "C" int32_t ifattn_pages_create(uint32_t page_tokens, uint32_t logical_tokens,
                                       uint32_t slots, int32_t shared, ifattn_pages **out) {
  if (!out) return reject("pages: null output handle");
  *out = nullptr;
  if (!slots || slots > kMaxResidents || !page_tokens || !logical_tokens ||
      logical_tokens % page_tokens)
    return reject("pages: need 1..64 residents and a context of whole pages");
  const uint32_t per = logical_tokens / page_tokens;
  if (uint64_t(per) * slots > kIdLimit) return reject("pages: pool exceeds 2^31-1 pages");
  auto *p = new (std::nothrow) ifattn_pages;
  if (!p) return fail(IFATTN_EINVAL, "pages: out of host memory");
  p->page_tokens = page_tokens;
  p->logical_tokens = logical_tokens;
  p->per_resident = per;
  p->residents = slots;
  p->shared = shared != 0;
  const uint32_t n = per * slots;
  // Every resident starts on its own partition, in order.
  p->map.resize(n);
  p->owner.resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    p->map[i] = int32_t(i);
    p->owner[i] = int8_t(i / per);
  }
  p->held.assign(slots, per);
  p->seen.assign(n, 0u);
  *out = p;
  return IFATTN_OK;
}

extern "C" void ifattn_pages_destroy(ifattn_pages *pages) { delete pages; }

extern "C" int32_t ifattn_pages_select(ifattn_pages *pages, uint32_t slot) {
  if (!pages) return reject("pages: null pool");
  if (slot >= pages->residents) return reject("pages: no such resident");
  pages->selected = slot;
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_selected(const ifattn_pages *pages, uint32_t *slot) {
  if (!pages || !slot) return reject("pages: null pool or output");
  *slot = pages->selected;
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_bind(ifattn_pages *p, const int32_t *ids, uint64_t count) {
  if (!p || (!ids && count)) return reject("pages: null pool or page list");
  const uint32_t r = p->selected, per = p->per_resident;
  // Pass 1: every page legal for this resident and named once.
  if (p->shared ? (count == 0 || count > per) : count != per)
    return reject(p->shared ? "pages: a claim names 1..P pages"
                            : "pages: a fixed binding names exactly P pages");
  const uint32_t stamp = p->next_epoch();
  for (uint64_t i = 0; i < count; ++i) {
    const int32_t id = ids[i];
    if (id < 0 || uint32_t(id) >= p->pool_pages()) return reject("pages: page id outside the pool");
    if (p->shared ? (p->owner[id] != -1 && p->owner[id] != int8_t(r)) : uint32_t(id) / per != r)
      return reject(p->shared ? "pages: page held by another resident"
                              : "pages: page outside the resident's partition");
    if (p->seen[id] == stamp) return reject("pages: page named twice");
    p->seen[id] = stamp;
  }
  // Pass 2: commit.
  int32_t *dst = p->map.data() + size_t(r) * per;
  if (p->shared) {
    for (uint32_t i = 0; i < p->held[r]; ++i) p->owner[dst[i]] = -1;
    for (uint64_t i = 0; i < count; ++i) p->owner[ids[i]] = int8_t(r);
  }
  std::memcpy(dst, ids, count * sizeof(int32_t));
  p->held[r] = uint32_t(count);
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_release(ifattn_pages *p, uint32_t slot) {
  if (!p) return reject("pages: null pool");
  if (!p->shared || slot >= p->residents)
    return reject("pages: release needs a shared pool and an existing resident");
  const int32_t *own = p->row(slot);
  for (uint32_t i = 0; i < p->held[slot]; ++i) p->owner[own[i]] = -1;
  p->held[slot] = 0;
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_owned(const ifattn_pages *p, uint32_t slot, int32_t *ids,
                                      uint64_t capacity, uint64_t *count) {
  if (!p || !count) return reject("pages: null pool or count");
  if (slot >= p->residents) return reject("pages: no such resident");
  *count = p->held[slot];
  if (ids) {
    if (capacity < p->held[slot]) return reject("pages: owned-page output too small");
    std::memcpy(ids, p->row(slot), p->held[slot] * sizeof(int32_t));
  }
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_append(const ifattn_pages *p, uint32_t slot, uint32_t position,
                                       uint64_t *physical) {
  if (!p || !physical) return reject("pages: null pool or output");
  const uint32_t r = slot == UINT32_MAX ? p->selected : slot;
  if (r >= p->residents) return reject("pages: no such resident");
  const int64_t row = p->physical_row(r, position);
  if (row < 0) return reject("pages: position outside the resident's pages");
  *physical = uint64_t(row);
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_slot_mapping(const ifattn_pages *p, const int32_t *row_residents,
                                             const int32_t *positions, uint64_t rows,
                                             int64_t *out) {
  if (!p || (rows && (!row_residents || !positions || !out)))
    return reject("slot mapping: null argument");
  for (uint64_t i = 0; i < rows; ++i) {
    const int32_t r = row_residents[i], pos = positions[i];
    if (r < 0 || uint32_t(r) >= p->residents || pos < 0 || p->physical_row(uint32_t(r), uint32_t(pos)) < 0)
      return reject("slot mapping: a row's position is outside its resident's pages");
  }
  for (uint64_t i = 0; i < rows; ++i)
    out[i] = p->physical_row(uint32_t(row_residents[i]), uint32_t(positions[i]));
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_batch_table(const ifattn_pages *p, const int32_t *residents,
                                            uint64_t count, uint32_t entries, int32_t ring,
                                            int32_t *out) {
  if (!p || !out || (!residents && count)) return reject("block table: null argument");
  if (count == 0 || count > p->residents) return reject("block table: 1..R residents");
  uint64_t used = 0;  // residents are <= 64: a bit mask finds repeats
  for (uint64_t i = 0; i < count; ++i) {
    const int32_t r = residents[i];
    if (r < 0 || uint32_t(r) >= p->residents || (used >> r & 1u))
      return reject("block table: unknown or repeated resident");
    used |= uint64_t(1) << r;
  }
  const uint32_t per = p->per_resident;
  if (entries == 0 || (!ring && entries != per))
    return reject("block table: P entries, or any nonzero count in ring mode");
  // Entry i holds logical page i (ring: i mod P); logical pages the resident
  // does not back read as page 0.
  for (uint64_t k = 0; k < count; ++k) {
    const int32_t *own = p->row(uint32_t(residents[k]));
    const uint32_t held = p->held[residents[k]];
    int32_t *dst = out + k * entries;
    for (uint32_t base = 0; base < entries; base += per) {
      const uint32_t n = std::min(per, entries - base);
      const uint32_t live = std::min(n, held);
      std::memcpy(dst + base, own, live * sizeof(int32_t));
      std::fill(dst + base + live, dst + base + n, 0);
    }
  }
  return IFATTN_OK;
}

extern "C" int32_t ifattn_pages_copy_plan(const ifattn_pages *p, uint32_t source,
                                          uint32_t destination, uint32_t completed_tokens,
                                          int32_t windowed, uint64_t field_bytes,
                                          uint64_t *ranges, uint64_t capacity, uint64_t *count) {
  if (!p || !count) return reject("copy plan: null argument");
  const uint32_t page = p->page_tokens;
  if (source == destination || completed_tokens == 0 || completed_tokens % page ||
      (!windowed && completed_tokens > p->logical_tokens))
    return reject("copy plan: two residents and a nonzero whole-page token count");
  if (source >= p->residents || destination >= p->residents)
    return reject("copy plan: no such resident");
  const uint64_t pool = p->pool_pages();
  if (field_bytes == 0 || field_bytes % pool) return reject("copy plan: field is not whole pages");
  const uint64_t page_bytes = field_bytes / pool;
  // A windowed copy of more tokens than a resident holds copies every ring page.
  const uint32_t n = std::min(completed_tokens / page, p->per_resident);
  if (p->held[source] < n || p->held[destination] < n)
    return reject("copy plan: a resident backs fewer pages than the copy needs");
  // Runs of pages that are consecutive on both sides become one range; the
  // runs are counted before any output is written.
  const int32_t *from = p->row(source), *to = p->row(destination);
  auto run_end = [&](uint32_t i) {
    uint32_t j = i + 1;
    while (j < n && from[j] == from[j - 1] + 1 && to[j] == to[j - 1] + 1) ++j;
    return j;
  };
  uint64_t runs = 0;
  for (uint32_t i = 0; i < n; i = run_end(i)) ++runs;
  if (ranges && capacity < runs) return reject("copy plan: output too small");
  if (ranges) {
    uint64_t k = 0;
    for (uint32_t i = 0, j; i < n; i = j, ++k) {
      j = run_end(i);
      ranges[3 * k] = uint64_t(from[i]) * page_bytes;
      ranges[3 * k + 1] = uint64_t(to[i]) * page_bytes;
      ranges[3 * k + 2] = uint64_t(j - i) * page_bytes;
    }
  }
  *count = runs;
  return IFATTN_OK;
}

extern "C" int32_t ifattn_page_spans(const int32_t *ids, uint64_t count, uint64_t page_bytes,
                                     uint64_t field_bytes, uint64_t *spans, uint64_t capacity,
                                     uint64_t *span_count) {
  if (!span_count || (!ids && count)) return reject("page spans: null argument");
  if (page_bytes == 0 || field_bytes == 0 || field_bytes % page_bytes)
    return reject("page spans: field is not whole pages");
  const uint64_t pages = field_bytes / page_bytes;
  std::vector<int32_t> order(ids, ids + count);
  std::sort(order.begin(), order.end());
  for (uint64_t i = 0; i < count; ++i)
    if (order[i] < 0 || uint64_t(order[i]) >= pages || (i && order[i] == order[i - 1]))
      return reject("page spans: page outside the field or named twice");
  // Physical order, one span per run of adjacent pages.
  auto run_end = [&](uint64_t i) {
    uint64_t j = i + 1;
    while (j < count && order[j] == order[j - 1] + 1) ++j;
    return j;
  };
  uint64_t runs = 0;
  for (uint64_t i = 0; i < count; i = run_end(i)) ++runs;
  if (spans && capacity < runs) return reject("page spans: output too small");
  if (spans) {
    uint64_t k = 0;
    for (uint64_t i = 0, j; i < count; i = j, ++k) {
      j = run_end(i);
      spans[2 * k] = uint64_t(order[i]) * page_bytes;
      spans[2 * k + 1] = (j - i) * page_bytes;
    }
  }
  *span_count = runs;
  return IFATTN_OK;
}

// ------------------------------------------------------------------ packed batch

extern "C" int32_t ifattn_sequence_batch_make(
    const ifattn_sequence_slice *slices, uint64_t count, uint32_t resident_capacity,
    uint32_t token_budget, uint32_t context, uint64_t rows_capacity, int32_t *starts,
    int32_t *query_ends, int32_t *prior_lengths, int32_t *kv_lengths, int32_t *residents,
    int32_t *positions, int32_t *row_residents, int64_t *lengths, uint32_t *sample_rows,
    uint32_t *sample_residents, uint64_t *rows, uint64_t *samples) {
  if (!slices && count) return reject("packed batch: null slices");
  if (count == 0 || !resident_capacity || !token_budget || !context ||
      resident_capacity > kIdLimit || token_budget > kIdLimit || context > kIdLimit)
    return reject("packed batch: empty batch or limits outside 1..2^31-1");
  // Pass 1: members valid, residents distinct, the running total within budget.
  std::vector<uint32_t> ids(count);
  uint64_t total = 0;
  for (uint64_t i = 0; i < count; ++i) {
    const ifattn_sequence_slice &s = slices[i];
    if (s.resident >= resident_capacity || s.tokens == 0 ||
        uint64_t(s.position) + s.tokens > context)
      return reject("packed batch: member outside the resident or context limits");
    ids[i] = s.resident;
    total += s.tokens;
    if (total > token_budget) return reject("packed batch: token budget exceeded");
  }
  std::sort(ids.begin(), ids.end());
  if (std::adjacent_find(ids.begin(), ids.end()) != ids.end())
    return reject("packed batch: a resident appears twice");
  if (total > rows_capacity) return reject("packed batch: row outputs too small");
  // Pass 2: emit. Row t of member k is position position_k + t; its
  // attention length is that position + 1; the member's sample row is its last.
  uint64_t row = 0, nsample = 0;
  if (starts) starts[0] = 0;
  for (uint64_t k = 0; k < count; ++k) {
    const ifattn_sequence_slice &s = slices[k];
    for (uint32_t t = 0; t < s.tokens; ++t, ++row) {
      if (positions) positions[row] = int32_t(s.position + t);
      if (row_residents) row_residents[row] = int32_t(s.resident);
      if (lengths) lengths[row] = int64_t(s.position) + t + 1;
    }
    if (starts) starts[k + 1] = int32_t(row);
    if (query_ends) query_ends[k] = int32_t(row);
    if (prior_lengths) prior_lengths[k] = int32_t(s.position);
    if (kv_lengths) kv_lengths[k] = int32_t(s.position + s.tokens);
    if (residents) residents[k] = int32_t(s.resident);
    if (s.sample) {
      if (sample_rows) sample_rows[nsample] = uint32_t(row - 1);
      if (sample_residents) sample_residents[nsample] = s.resident;
      ++nsample;
    }
  }
  if (rows) *rows = total;
  if (samples) *samples = nsample;
  return IFATTN_OK;
}

// ------------------------------------------------------------------ window ring

extern "C" int32_t ifattn_window_layout(uint32_t context, uint32_t window, uint32_t chunk,
                                        uint32_t page_tokens, uint32_t *physical_pages,
                                        uint32_t *table_entries) {
  Ring g;
  if (const int32_t st = make_ring(context, window, chunk, page_tokens, &g)) return st;
  if (physical_pages) *physical_pages = g.pages;
  if (table_entries) *table_entries = g.entries;
  return IFATTN_OK;
}

namespace {
// The resident's ring pages: `owned` (g.pages distinct, non-negative ids) or,
// without it, ring page numbers themselves.
int32_t check_owned(const Ring &g, const int32_t *owned, uint64_t owned_count) {
  if (!owned) return IFATTN_OK;
  if (owned_count != g.pages) return reject("window ring: owned pages must number the ring pages");
  std::vector<int32_t> s(owned, owned + owned_count);
  std::sort(s.begin(), s.end());
  if (s.front() < 0 || std::adjacent_find(s.begin(), s.end()) != s.end())
    return reject("window ring: negative or repeated owned page");
  return IFATTN_OK;
}
}  // namespace

extern "C" int32_t ifattn_window_table(uint32_t context, uint32_t window, uint32_t chunk,
                                       uint32_t page_tokens, const int32_t *owned,
                                       uint64_t owned_count, int32_t *table) {
  Ring g;
  if (const int32_t st = make_ring(context, window, chunk, page_tokens, &g)) return st;
  if (!table) return reject("window ring: null table output");
  if (const int32_t st = check_owned(g, owned, owned_count)) return st;
  for (uint32_t l = 0; l < g.entries; ++l) {
    const uint32_t ph = l % g.pages;
    table[l] = owned ? owned[ph] : int32_t(ph);
  }
  return IFATTN_OK;
}

extern "C" int32_t ifattn_window_slots(uint32_t context, uint32_t window, uint32_t chunk,
                                       uint32_t page_tokens, const int32_t *owned,
                                       uint64_t owned_count, const uint32_t *positions,
                                       uint64_t count, int64_t *slots) {
  Ring g;
  if (const int32_t st = make_ring(context, window, chunk, page_tokens, &g)) return st;
  if (!slots || (!positions && count)) return reject("window ring: null slot argument");
  if (const int32_t st = check_owned(g, owned, owned_count)) return st;
  for (uint64_t i = 0; i < count; ++i)
    if (positions[i] >= context) return reject("window ring: position beyond the context");
  for (uint64_t i = 0; i < count; ++i) {
    const uint32_t ph = (positions[i] / page_tokens) % g.pages;
    slots[i] = int64_t(owned ? owned[ph] : int32_t(ph)) * page_tokens + positions[i] % page_tokens;
  }
  return IFATTN_OK;
}
