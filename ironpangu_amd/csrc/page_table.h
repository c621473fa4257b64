// Host metadata that feeds the cache-write and attention kernels: per-resident
// page ownership, slot mapping and block tables, plus the packed varlen
// (cu_seqlens) batch layout. Cache contents never visit the host.
//
// Behaviour follows the reference's host classes:
//  * PageMap      ~ PageBinding       (native/src/page_binding.h:37-62)
//  * ResidentPageTable ~ ResidentPages (native/src/page_binding.h:65-188)
//  * PackedBatch  ~ SequenceBatch::make (native/include/sequence_batch.h:23-59)
//  * coalesce_page_spans ~ page_spans (native/src/page_binding.h:19-35)
//  * WindowRing   ~ SlidingWindowLayout (native/include/sliding_window_layout.h:9-33)
// Every mutating call validates its whole input before changing state, so a
// rejected update leaves the previous mapping intact (page_binding_test.cpp:17-22).
#pragma once
#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <vector>

namespace ifattn::host {

struct ByteRange {
  uint64_t source, destination, bytes;
};
struct Span {
  uint64_t offset, bytes;
};

// Sort the owned pages and merge physically adjacent ones into byte spans.
inline std::vector<Span> coalesce_page_spans(std::vector<int32_t> pages, uint64_t page_bytes,
                                             uint64_t field_bytes) {
  if (page_bytes == 0 || field_bytes == 0 || field_bytes % page_bytes != 0)
    throw std::runtime_error("page span field layout");
  const uint64_t count = field_bytes / page_bytes;
  std::sort(pages.begin(), pages.end());
  for (size_t i = 0; i < pages.size(); ++i) {
    if (pages[i] < 0 || uint64_t(pages[i]) >= count || (i > 0 && pages[i] == pages[i - 1]))
      throw std::runtime_error("page span bounds/alias");
  }
  std::vector<Span> out;
  for (int32_t page : pages) {
    const uint64_t off = uint64_t(page) * page_bytes;
    if (!out.empty() && out.back().offset + out.back().bytes == off)
      out.back().bytes += page_bytes;
    else
      out.push_back({off, page_bytes});
  }
  return out;
}

// Page ring of a sliding-window cache whose chunk writes precede the chunk's
// queries: the window plus the later rows of a chunk span window + chunk - 1
// tokens, which can touch one page more than they fill, so that many physical
// pages (never more than the context needs) hold every live row. Block-table
// entries stay absolute logical pages; logical page l lives in physical page
// l % pages, so the attention kernels read the window through an ordinary table.
class WindowRing {
 public:
  uint32_t context, window, chunk, page_tokens, pages;
  WindowRing(uint32_t c, uint32_t w, uint32_t q, uint32_t p)
      : context(c), window(w), chunk(q), page_tokens(p), pages(0) {
    if (c == 0 || w == 0 || q == 0 || p == 0 || q > c)
      throw std::runtime_error("invalid sliding window layout");
    const uint64_t span = uint64_t(w) + q - 1;       // tokens live at once
    uint64_t need = (span + p - 2) / p + 1;           // pages such a span can touch
    const uint64_t all = (uint64_t(c) + p - 1) / p;   // pages of the whole context
    need = need < all ? need : all;
    if (need * p > UINT32_MAX) throw std::runtime_error("sliding window capacity overflow");
    pages = uint32_t(need);
  }
  uint32_t entries() const { return uint32_t((uint64_t(context) + page_tokens - 1) / page_tokens); }
  uint32_t physical_page(uint32_t logical) const {
    if (logical >= entries()) throw std::runtime_error("sliding page bounds");
    return logical % pages;
  }
  uint32_t slot(uint32_t position) const {
    if (position >= context) throw std::runtime_error("sliding append bounds");
    return physical_page(position / page_tokens) * page_tokens + position % page_tokens;
  }
};

// True when `ids` names some value twice (sort-based, no allocation sized by
// the id range).
template <typename T>
inline bool has_duplicates(std::vector<T> ids) {
  std::sort(ids.begin(), ids.end());
  return std::adjacent_find(ids.begin(), ids.end()) != ids.end();
}

// One logical sequence of `logical_tokens` tokens mapped onto whole pages of a
// pool of `physical_pages` pages.
class PageMap {
  uint32_t page_tokens_, logical_tokens_, physical_pages_;
  std::vector<int32_t> pages_;

 public:
  PageMap(uint32_t page_tokens, uint32_t logical_tokens, uint32_t physical_pages)
      : page_tokens_(page_tokens), logical_tokens_(logical_tokens), physical_pages_(physical_pages) {
    if (page_tokens == 0 || logical_tokens == 0 || physical_pages > uint32_t(INT32_MAX) ||
        logical_tokens % page_tokens != 0 || logical_tokens / page_tokens > physical_pages)
      throw std::runtime_error("invalid page binding capacity");
    pages_.resize(logical_tokens / page_tokens);
    for (size_t i = 0; i < pages_.size(); ++i) pages_[i] = int32_t(i);
  }
  void bind(const std::vector<int32_t> &pages) {
    if (pages.size() != pages_.size()) throw std::runtime_error("page binding length");
    for (int32_t page : pages)
      if (page < 0 || uint32_t(page) >= physical_pages_)
        throw std::runtime_error("page binding bounds/alias");
    if (has_duplicates(pages)) throw std::runtime_error("page binding bounds/alias");
    pages_ = pages;
  }
  // Physical token row of a logical position.
  uint64_t slot(uint32_t position) const {
    if (position >= logical_tokens_) throw std::runtime_error("page append bounds");
    return uint64_t(pages_[position / page_tokens_]) * page_tokens_ + position % page_tokens_;
  }
  const std::vector<int32_t> &pages() const { return pages_; }
};

// Up to 64 residents. Fixed mode: resident r owns partition
// [r*P, (r+1)*P) of the pool and may only permute pages inside it. Shared
// mode: residents claim any unowned pages (a partial reservation is allowed).
class ResidentPageTable {
  uint32_t page_tokens_, logical_tokens_, pages_per_slot_, active_ = 0;
  bool shared_;
  std::vector<PageMap> fixed_;
  std::vector<std::vector<int32_t>> claimed_;
  std::vector<int32_t> owner_;

  void check_slot(uint32_t slot, const char *what) const {
    if (slot >= fixed_.size()) throw std::runtime_error(what);
  }

 public:
  ResidentPageTable(uint32_t page_tokens, uint32_t logical_tokens, uint32_t slots, bool shared)
      : page_tokens_(page_tokens), logical_tokens_(logical_tokens),
        pages_per_slot_(page_tokens ? logical_tokens / page_tokens : 0), shared_(shared) {
    if (slots == 0 || slots > 64 || page_tokens == 0 || logical_tokens == 0 ||
        logical_tokens % page_tokens != 0 || uint64_t(pages_per_slot_) * slots > uint64_t(INT32_MAX))
      throw std::runtime_error("resident page capacity");
    const uint32_t pool = pages_per_slot_ * slots;
    owner_.assign(pool, -1);
    for (uint32_t s = 0; s < slots; ++s) {
      fixed_.emplace_back(page_tokens, logical_tokens, pool);
      std::vector<int32_t> own(pages_per_slot_);
      for (uint32_t i = 0; i < pages_per_slot_; ++i) {
        own[i] = int32_t(s * pages_per_slot_ + i);
        owner_[own[i]] = int32_t(s);
      }
      fixed_.back().bind(own);
      claimed_.push_back(own);
    }
  }
  uint32_t slots() const { return uint32_t(fixed_.size()); }
  uint32_t pages_per_slot() const { return pages_per_slot_; }
  uint32_t active() const { return active_; }
  bool shared() const { return shared_; }

  void select(uint32_t slot) {
    check_slot(slot, "resident page slot");
    active_ = slot;
  }
  void bind(const std::vector<int32_t> &pages) {
    if (!shared_) {
      for (int32_t page : pages)
        if (page < 0 || uint32_t(page) / pages_per_slot_ != active_)
          throw std::runtime_error("page binding crosses resident partition");
      fixed_[active_].bind(pages);
      return;
    }
    if (pages.empty() || pages.size() > pages_per_slot_)
      throw std::runtime_error("shared page binding length");
    for (int32_t page : pages)
      if (page < 0 || size_t(page) >= owner_.size() ||
          (owner_[page] != -1 && owner_[page] != int32_t(active_)))
        throw std::runtime_error("shared page bounds/owner/alias");
    if (has_duplicates(pages)) throw std::runtime_error("shared page bounds/owner/alias");
    release(active_);
    claimed_[active_] = pages;
    for (int32_t page : pages) owner_[page] = int32_t(active_);
  }
  void release(uint32_t slot) {
    if (!shared_ || slot >= fixed_.size())
      throw std::runtime_error("shared page release policy/slot");
    for (int32_t page : claimed_[slot]) owner_[page] = -1;
    claimed_[slot].clear();
  }
  const std::vector<int32_t> &pages(uint32_t slot) const {
    check_slot(slot, "page lookup slot");
    return shared_ ? claimed_[slot] : fixed_[slot].pages();
  }
  // Physical token row of (resident, logical position); does not change the
  // selected resident.
  uint64_t slot_of(uint32_t slot, uint32_t position) const {
    check_slot(slot, "page append slot");
    if (!shared_) return fixed_[slot].slot(position);
    const auto &own = claimed_[slot];
    if (position >= logical_tokens_ || position / page_tokens_ >= own.size())
      throw std::runtime_error("append outside reserved shared pages");
    return uint64_t(own[position / page_tokens_]) * page_tokens_ + position % page_tokens_;
  }
  // Block table row; unowned entries are 0, ring mode repeats the owned pages.
  std::vector<int32_t> table(uint32_t slot, uint32_t entries, bool ring) const {
    const auto &own = pages(slot);
    if (entries == 0 || (!ring && entries != pages_per_slot_))
      throw std::runtime_error("resident table extent");
    std::vector<int32_t> row(entries, 0);
    for (uint32_t i = 0; i < entries; ++i) {
      const uint32_t ordinal = ring ? i % pages_per_slot_ : i;
      if (ordinal < own.size()) row[i] = own[ordinal];
    }
    return row;
  }
  std::vector<int32_t> batch_table(const std::vector<int32_t> &residents, uint32_t entries,
                                   bool ring) const {
    if (residents.empty() || residents.size() > fixed_.size())
      throw std::runtime_error("resident batch table count");
    for (int32_t r : residents)
      if (r < 0 || uint32_t(r) >= fixed_.size())
        throw std::runtime_error("resident batch table slot");
    if (has_duplicates(residents)) throw std::runtime_error("resident batch table slot");
    std::vector<int32_t> out;
    out.reserve(size_t(entries) * residents.size());
    for (int32_t r : residents) {
      auto row = table(uint32_t(r), entries, ring);
      out.insert(out.end(), row.begin(), row.end());
    }
    return out;
  }
  // Byte ranges copying `completed` tokens of pages from one resident to
  // another (page_binding.h:161-187): whole pages, ring ordinals, adjacent
  // ranges merged.
  std::vector<ByteRange> copy_plan(uint32_t source, uint32_t destination, uint32_t completed,
                                   bool windowed, uint64_t field_bytes) const {
    if (source == destination || completed == 0 || completed % page_tokens_ != 0 ||
        (!windowed && completed > logical_tokens_))
      throw std::runtime_error("state copy requires distinct slots and a complete page boundary");
    const auto &from = pages(source);
    const auto &to = pages(destination);
    const uint64_t pool = uint64_t(pages_per_slot_) * fixed_.size();
    if (field_bytes == 0 || field_bytes % pool != 0)
      throw std::runtime_error("state copy field disagrees with physical page layout");
    const uint64_t page_bytes = field_bytes / pool;
    const size_t count = std::min<uint64_t>(completed / page_tokens_, pages_per_slot_);
    if (from.size() < count || to.size() < count)
      throw std::runtime_error("state copy exceeds reserved source/destination pages");
    std::vector<ByteRange> out;
    for (size_t i = 0; i < count; ++i) {
      const ByteRange next{uint64_t(from[i]) * page_bytes, uint64_t(to[i]) * page_bytes, page_bytes};
      if (!out.empty() && out.back().source + out.back().bytes == next.source &&
          out.back().destination + out.back().bytes == next.destination)
        out.back().bytes += page_bytes;
      else
        out.push_back(next);
    }
    return out;
  }
};

struct PackedSlice {
  uint32_t resident, position, tokens;
  bool sample;
};

// Control-only packed varlen layout. starts == cu_seqlens_q.
struct PackedBatch {
  std::vector<int32_t> starts{0}, residents, positions, row_residents;
  std::vector<int32_t> query_ends, prior_lengths, kv_lengths;
  std::vector<int64_t> lengths;
  std::vector<uint32_t> sample_rows, sample_residents;

  static PackedBatch make(const std::vector<PackedSlice> &seqs, uint32_t resident_capacity,
                          uint32_t token_budget, uint32_t context) {
    if (seqs.empty() || resident_capacity == 0 || token_budget == 0 || context == 0 ||
        resident_capacity > uint32_t(INT32_MAX) || token_budget > uint32_t(INT32_MAX) ||
        context > uint32_t(INT32_MAX))
      throw std::runtime_error("invalid sequence batch limits");
    // Members are checked in order, as submitted: the first invalid member or
    // the first prefix over budget rejects the batch.
    uint64_t total = 0;
    std::vector<uint32_t> ids;
    for (const auto &s : seqs) {
      ids.push_back(s.resident);
      if (s.resident >= resident_capacity || has_duplicates(ids) || s.tokens == 0 ||
          uint64_t(s.position) + s.tokens > context)
        throw std::runtime_error("invalid sequence batch member");
      total += s.tokens;
      if (total > token_budget) throw std::runtime_error("sequence batch token budget exceeded");
    }
    PackedBatch b;
    b.positions.reserve(total);
    b.row_residents.reserve(total);
    b.lengths.reserve(total);
    for (const auto &s : seqs) {
      b.residents.push_back(int32_t(s.resident));
      for (uint32_t i = 0; i < s.tokens; ++i) {
        b.positions.push_back(int32_t(s.position + i));
        b.row_residents.push_back(int32_t(s.resident));
        b.lengths.push_back(int64_t(s.position) + i + 1);
      }
      const int32_t end = int32_t(b.positions.size());
      b.starts.push_back(end);
      b.query_ends.push_back(end);
      b.prior_lengths.push_back(int32_t(s.position));
      b.kv_lengths.push_back(int32_t(s.position + s.tokens));
      if (s.sample) {
        b.sample_rows.push_back(uint32_t(end - 1));
        b.sample_residents.push_back(s.resident);
      }
    }
    return b;
  }
};

}  // namespace ifattn::host
