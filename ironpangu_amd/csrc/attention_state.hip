// One MLA attention layer's state as an object: cache, page binding, block
// table, query/output/index/length buffers and the learned sink rows, the
// counterpart of the reference's AttentionState
// (native/src/openpangu_decoder_state.h:16-48). Geometry and the host metadata
// (append, blocks) follow that class; attention runs the gfx950 MLA kernels of
// mla_decode.hip over the state's own buffers.
#include <cstdlib>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/ifattn_state.h"
#include "common.h"
#include "ifattn_internal.h"

namespace {
using ifattn::fail;

constexpr uint32_t kSinks = 128;  // sink rows of the reference state (openpangu_decoder_state.h:30)
constexpr int32_t kTopK = 512;    // candidate list of the reference state ([1, 1, 512])

__global__ void state_store_i32(int32_t *dst, int32_t v) { *dst = v; }

int32_t reject(const char *what) { return fail(IFATTN_EINVAL, what); }
}  // namespace

struct ifattn_attention_state {
  ifattn_attention_state_geometry geo{};
  uint32_t capacity = 0, residents = 0, context = 0, bits = 16;
  ifattn_pages *pages = nullptr;
  ifattn_attention_state_buffers buf{};
  void *workspace = nullptr;
  uint64_t workspace_bytes = 0;
  int device = -1;
  bool ready = false;  // every device buffer allocated and initialised
  std::mutex alloc_mutex;
  std::vector<int32_t> host_table;

  ~ifattn_attention_state() {
    free_buffers();
    ifattn_pages_destroy(pages);
  }
  void free_buffers() {
    void *ptrs[] = {buf.cache, buf.table, buf.scales, buf.query, buf.out, buf.indices,
                    buf.kv_len, buf.sink_keys, buf.sink_values, workspace};
    for (void *p : ptrs)
      if (p) (void)hipFree(p);
    buf = ifattn_attention_state_buffers{};
    workspace = nullptr;
    workspace_bytes = 0;
    ready = false;
  }
  bool sparse() const { return geo.format == IFATTN_STATE_PACKED_C8; }
  uint32_t max_context() const { return geo.table_entries * geo.page_tokens; }

  // Device buffers on the current device, once. A failure part way frees
  // what was allocated, so the next call starts again from nothing.
  int32_t ensure_buffers() {
    std::lock_guard<std::mutex> lock(alloc_mutex);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(IFATTN_ELAUNCH, "attention state: no device");
    if (ready) {
      if (dev != device) return reject("attention state: buffers live on another device");
      return IFATTN_OK;
    }
    const int32_t st = allocate_buffers();
    if (st != IFATTN_OK) {
      free_buffers();
      return st;
    }
    device = dev;
    ready = true;
    return IFATTN_OK;
  }
  int32_t allocate_buffers() {
    struct Req {
      void **ptr;
      uint64_t bytes;
    };
    const uint64_t q_bytes = uint64_t(geo.heads) * 576 * 2, o_bytes = uint64_t(geo.heads) * 512 * 2;
    std::vector<Req> reqs = {{&buf.cache, geo.cache_bytes},
                             {reinterpret_cast<void **>(&buf.table), uint64_t(geo.table_entries) * 4},
                             {reinterpret_cast<void **>(&buf.query), q_bytes},
                             {reinterpret_cast<void **>(&buf.out), o_bytes},
                             {reinterpret_cast<void **>(&buf.indices), uint64_t(kTopK) * 4},
                             {reinterpret_cast<void **>(&buf.kv_len), 16},
                             {reinterpret_cast<void **>(&buf.sink_keys), uint64_t(kSinks) * 576 * 2},
                             {reinterpret_cast<void **>(&buf.sink_values), uint64_t(kSinks) * 512 * 2}};
    if (geo.format == IFATTN_STATE_ROW_QUANT)
      reqs.push_back({reinterpret_cast<void **>(&buf.scales), uint64_t(capacity) * 4});
    workspace_bytes = ifattn_mla_attention_workspace_size(1, int32_t(geo.heads), int32_t(max_context()),
                                                          0, sparse() ? kTopK : 0, int32_t(kSinks),
                                                          int32_t(geo.page_tokens));
    reqs.push_back({&workspace, workspace_bytes});
    // Test hook: IFATTN_STATE_FAIL_ALLOCATION=i fails the i-th allocation, so
    // a test can force the clean-up path from the host.
    const char *hook = getenv("IFATTN_STATE_FAIL_ALLOCATION");
    const int fail_allocation_at = hook ? atoi(hook) : -1;
    for (auto &r : reqs) {
      if (fail_allocation_at >= 0 && int(&r - reqs.data()) == fail_allocation_at)
        return fail(IFATTN_ELAUNCH, "attention state: device allocation failed");
      if (hipMalloc(r.ptr, r.bytes ? r.bytes : 16) != hipSuccess) {
        *r.ptr = nullptr;
        return fail(IFATTN_ELAUNCH, "attention state: device allocation failed");
      }
      if (hipMemset(*r.ptr, 0, r.bytes ? r.bytes : 16) != hipSuccess)
        return fail(IFATTN_ELAUNCH, "attention state: device allocation failed");
    }
    // The reference's initial table: entry i -> page i mod (capacity / page).
    std::vector<int32_t> blocks(geo.table_entries);
    const uint32_t per = capacity / geo.page_tokens;
    for (uint32_t i = 0; i < geo.table_entries; ++i) blocks[i] = int32_t(i % per);
    if (hipMemcpy(buf.table, blocks.data(), blocks.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return fail(IFATTN_ELAUNCH, "attention state: table upload failed");
    std::vector<int32_t> none(kTopK, -1);
    if (hipMemcpy(buf.indices, none.data(), none.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return fail(IFATTN_ELAUNCH, "attention state: index upload failed");
    return IFATTN_OK;
  }
};

extern "C" int32_t ifattn_attention_state_create(uint32_t bits, uint32_t capacity, int32_t packed,
                                                 uint32_t residents, int32_t shared,
                                                 uint32_t context, uint32_t heads,
                                                 ifattn_attention_state **out) {
  if (!out) return reject("attention state: null output handle");
  *out = nullptr;
  if (heads == 0 || heads > 16) return reject("attention state: 1..16 heads");
  const bool row_quant = !packed && bits != 16;
  if (row_quant && bits != 8 && bits != 4)
    return reject("attention state: bits 16 (bf16), or 8 / 4 (row-quantized)");
  if (row_quant && residents > 1)
    return reject("attention state: resident row-quantized cache unsupported");
  const uint32_t page = packed ? 32 : 16;
  if (capacity == 0 || capacity % page || residents == 0)
    return reject("attention state: capacity must be whole pages and residents >= 1");
  auto *s = new (std::nothrow) ifattn_attention_state;
  if (!s) return reject("attention state: out of host memory");
  if (const int32_t st = ifattn_pages_create(page, capacity, residents, shared, &s->pages)) {
    delete s;
    return st;
  }
  s->capacity = capacity;
  s->residents = residents;
  s->context = context;
  s->bits = bits;
  auto &g = s->geo;
  g.format = packed ? IFATTN_STATE_PACKED_C8 : (row_quant ? IFATTN_STATE_ROW_QUANT : IFATTN_STATE_BF16);
  g.page_tokens = page;
  g.heads = heads;
  if (packed) {
    g.row_bytes = 656;
    g.num_blocks = residents * capacity / 32;
    g.table_entries = capacity / 32;
  } else {
    g.row_bytes = row_quant ? 576 * bits / 8 : 1152;
    g.num_blocks = row_quant ? 0 : residents * capacity / 16;
    g.table_entries = context ? (context + 15) / 16 : capacity / 16;
  }
  g.cache_bytes = row_quant ? uint64_t(capacity) * g.row_bytes
                            : uint64_t(g.num_blocks) * page * g.row_bytes;
  *out = s;
  return IFATTN_OK;
}

extern "C" void ifattn_attention_state_destroy(ifattn_attention_state *state) { delete state; }

extern "C" int32_t ifattn_attention_state_geometry_of(const ifattn_attention_state *state,
                                                      ifattn_attention_state_geometry *out) {
  if (!state || !out) return reject("attention state: null argument");
  *out = state->geo;
  return IFATTN_OK;
}

extern "C" int32_t ifattn_attention_state_pages(ifattn_attention_state *state, ifattn_pages **out) {
  if (!state || !out) return reject("attention state: null argument");
  *out = state->pages;
  return IFATTN_OK;
}

extern "C" int32_t ifattn_attention_state_append(const ifattn_attention_state *state,
                                                 uint32_t position, uint64_t *physical) {
  if (!state || !physical) return reject("attention state: null argument");
  if (state->context && position >= state->context)
    return reject("attention state: absolute position past the context");
  const uint32_t p = state->context ? position % state->capacity : position;
  return ifattn_pages_append(state->pages, UINT32_MAX, p, physical);
}

extern "C" int32_t ifattn_attention_state_blocks(const ifattn_attention_state *state,
                                                 int32_t *table, uint32_t capacity,
                                                 uint32_t *entries) {
  if (!state || !entries) return reject("attention state: null argument");
  *entries = state->geo.table_entries;
  if (!table) return IFATTN_OK;
  if (capacity < state->geo.table_entries) return reject("attention state: table output too small");
  uint32_t sel = 0;
  if (const int32_t st = ifattn_pages_selected(state->pages, &sel)) return st;
  const int32_t r = int32_t(sel);
  return ifattn_pages_batch_table(state->pages, &r, 1, state->geo.table_entries,
                                  state->context != 0, table);
}

extern "C" int32_t ifattn_attention_state_buffers_of(ifattn_attention_state *state,
                                                     ifattn_attention_state_buffers *out) {
  if (!state || !out) return reject("attention state: null argument");
  if (const int32_t st = state->ensure_buffers()) return st;
  *out = state->buf;
  return IFATTN_OK;
}

extern "C" int32_t ifattn_attention_state_upload_table(ifattn_attention_state *state, void *stream) {
  if (!state) return reject("attention state: null state");
  if (const int32_t st = state->ensure_buffers()) return st;
  auto &t = state->host_table;
  t.resize(state->geo.table_entries);
  uint32_t n = 0;
  if (const int32_t st = ifattn_attention_state_blocks(state, t.data(), uint32_t(t.size()), &n)) return st;
  // Ordered after the stream's earlier work; returns once the table is in
  // place (the reference's DeviceTensor::upload is synchronous too).
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(state->buf.table, t.data(), t.size() * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(IFATTN_ELAUNCH, "attention state: table upload failed");
  return IFATTN_OK;
}

extern "C" int32_t ifattn_attention_state_set_length(ifattn_attention_state *state, int32_t kv_len,
                                                     void *stream) {
  if (!state) return reject("attention state: null state");
  if (kv_len < 0 || uint32_t(kv_len) > state->max_context())
    return reject("attention state: length outside the table's reach");
  if (const int32_t st = state->ensure_buffers()) return st;
  state_store_i32<<<1, 1, 0, static_cast<hipStream_t>(stream)>>>(state->buf.kv_len, kv_len);
  return ifattn::launch_status("attention state length");
}

extern "C" int32_t ifattn_attention_state_attend(ifattn_attention_state *state, int32_t window,
                                                 int32_t sinks, void *stream) {
  if (!state) return reject("attention state: null state");
  if (window < 0) return reject("attention state: window must be >= 0");
  if (const int32_t st = state->ensure_buffers()) return st;
  const auto &b = state->buf;
  const auto &g = state->geo;
  const float scale = 0.07216878364870322f;  // 1/sqrt(192)
  const int32_t n_sinks = sinks ? int32_t(kSinks) : 0;
  if (g.format == IFATTN_STATE_ROW_QUANT)  // codes dequantized in registers
    return ifattn_mla_window_attention_rowq(
        b.query, b.cache, b.scales, int32_t(state->bits), b.table, int32_t(g.table_entries), nullptr,
        b.kv_len, 1, 1, window, sinks ? b.sink_keys : nullptr, sinks ? b.sink_values : nullptr,
        n_sinks, b.out, int32_t(g.heads), int32_t(g.page_tokens),
        int64_t(state->capacity / g.page_tokens), int32_t(state->max_context()), scale,
        state->workspace, state->workspace_bytes, stream);
  if (state->sparse())
    return ifattn_mla_sparse_attention_c8(
        b.query, b.cache, b.indices, kTopK, b.table, int32_t(g.table_entries), nullptr, b.kv_len, 1,
        1, sinks ? b.sink_keys : nullptr, sinks ? b.sink_values : nullptr, n_sinks, b.out,
        int32_t(g.heads), int32_t(g.page_tokens), int64_t(g.num_blocks), int32_t(state->max_context()),
        scale, state->workspace, state->workspace_bytes, stream);
  return ifattn_mla_window_attention_bf16(
      b.query, b.cache, b.table, int32_t(g.table_entries), nullptr, b.kv_len, 1, 1, window,
      sinks ? b.sink_keys : nullptr, sinks ? b.sink_values : nullptr, n_sinks, b.out,
      int32_t(g.heads), int32_t(g.page_tokens), int64_t(g.num_blocks), int32_t(state->max_context()),
      scale, state->workspace, state->workspace_bytes, stream);
}
