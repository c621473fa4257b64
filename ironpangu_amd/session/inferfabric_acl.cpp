// libinferfabric_acl.so: the reference's session ABI (native/include/inferfabric_acl.h)
// over one HIP device, for callers that bind it by name — the Rust loader
// (crates/inferfabric-native/src/ffi.rs:36-70) and the Qwen attention probe
// (crates/inferfabric-cli/src/npu_probe/attention.rs:66-200).
//
// A session is a HIP device, one default-priority stream and four id tables
// (buffers, operations, graphs, and the owned workspaces behind operations).
// An operation is a fixed list of launches over device addresses resolved when
// it is prepared, plus child operations for sequences; nothing is planned at
// execute time, so a captured graph replays exactly the launches an eager run
// makes. The launches themselves are the gfx950 kernels of libifattn_hip.so,
// entered through its C ABI (include/ifattn.h).
//
// Conventions kept from the reference implementation
// (native/src/inferfabric_acl.cpp): status 0 / -1 with a thread-local message
// (:46-58), ids counting up from 1 (:294), calls only on the opening thread
// (:297-299), a session refuses further work after a failed capture (:300-301,
// :790-797), execute / replay / read / write complete before returning
// (:592-597, :636-648, :756-768), operations and graphs live until close
// (:1751-1790).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <exception>
#include <functional>
#include <limits>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/ifattn.h"
#include "../../include/inferfabric_acl.h"

namespace {

thread_local std::string g_error;

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void hip(hipError_t e, const char *what) {
  if (e != hipSuccess) throw Failure(std::string(what) + ": " + hipGetErrorString(e));
}
// A status of the ifattn C ABI; its message is on this thread.
void ifattn_ok(int32_t status, const char *what) {
  if (status != IFATTN_OK) throw Failure(std::string(what) + ": " + ifattn_last_error());
}

template <class F>
int32_t guarded(F &&f) noexcept {
  try {
    f();
    g_error.clear();
    return 0;
  } catch (const std::exception &e) {
    g_error = e.what();
  } catch (...) {
    g_error = "unknown C++ exception";
  }
  return -1;
}

int32_t not_served(const char *entry) {
  g_error = std::string(entry) +
            ": not in this library (the MI355X build serves the session, sequences and the "
            "Qwen attention path: attention_qk_prepare, paged_attention_prepare)";
  return -1;
}

}  // namespace

struct inferfabric_acl_session {
  struct Buffer {
    void *ptr;
    uint64_t bytes;
    bool owned;
  };
  struct Operation {
    std::vector<Operation *> children;                 // run first, in order
    std::vector<std::function<void(hipStream_t)>> launches;
    std::vector<void *> owned;                         // workspaces, freed at close
    uint64_t workspace_bytes = 0;
    void run(hipStream_t s) const {
      for (const Operation *c : children) c->run(s);
      for (const auto &l : launches) l(s);
    }
  };
  struct Graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
  };

  int device = 0;
  hipStream_t stream = nullptr;
  std::thread::id thread = std::this_thread::get_id();
  uint64_t next = 1;
  bool poisoned = false;
  std::map<uint64_t, Buffer> buffers;
  std::map<uint64_t, std::unique_ptr<Operation>> operations;
  std::map<uint64_t, Graph> graphs;
  uint64_t budget = 0, reserve = 0, baseline_free = 0, minimum_free = UINT64_MAX;

  void enter() {
    if (thread != std::this_thread::get_id()) throw Failure("wrong device thread");
    if (poisoned) throw Failure("session poisoned after capture failure");
    hip(hipSetDevice(device), "hipSetDevice");
  }
  void *region(uint64_t id, uint64_t offset, uint64_t bytes) {
    auto it = buffers.find(id);
    if (it == buffers.end() || offset > it->second.bytes || bytes > it->second.bytes - offset)
      throw Failure("invalid allocation region");
    return static_cast<char *>(it->second.ptr) + offset;
  }
  std::pair<uint64_t, uint64_t> observe() {
    size_t free = 0, total = 0;
    hip(hipMemGetInfo(&free, &total), "HBM memory info");
    minimum_free = std::min<uint64_t>(minimum_free, free);
    return {free, total};
  }
  // Budget rule of the reference (inferfabric_acl.cpp:149-161): device memory in
  // use since the budget was set, plus this request, stays within the budget,
  // and the reserve stays free.
  void check_allocation(uint64_t bytes) {
    if (!budget) return;
    const uint64_t free = observe().first;
    const uint64_t used = baseline_free > free ? baseline_free - free : 0;
    if (used > budget || bytes > budget - used || free < reserve || bytes > free - reserve)
      throw Failure("HBM budget exceeded: observed_used=" + std::to_string(used) +
                    " allocation=" + std::to_string(bytes) + " budget=" + std::to_string(budget));
  }
  void *device_alloc(uint64_t bytes, const char *what) {
    check_allocation(bytes);
    void *p = nullptr;
    hip(hipMalloc(&p, bytes ? bytes : 16), what);
    if (budget) observe();
    return p;
  }
  uint64_t add_operation(std::unique_ptr<Operation> op) {
    const uint64_t id = next++;
    operations.emplace(id, std::move(op));
    return id;
  }
  uint64_t add_graph(Graph g) {
    const uint64_t id = next++;
    graphs.emplace(id, g);
    return id;
  }
  void fence(const char *what) { hip(hipStreamSynchronize(stream), what); }
  // Records `body` (launches on `stream`) into a graph. A failure inside the
  // capture leaves the session poisoned, as the reference does.
  Graph capture(const std::function<void()> &body) {
    hip(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "capture begin");
    std::exception_ptr error;
    try {
      body();
    } catch (...) {
      error = std::current_exception();
    }
    Graph g;
    const hipError_t end = hipStreamEndCapture(stream, &g.graph);
    hipError_t inst = hipSuccess;
    if (!error && end == hipSuccess) inst = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
    if (error || end != hipSuccess || inst != hipSuccess) {
      poisoned = true;
      if (g.exec) hipGraphExecDestroy(g.exec);
      if (g.graph) hipGraphDestroy(g.graph);
      if (error) std::rethrow_exception(error);
      hip(end, "capture end");
      hip(inst, "graph instantiate");
    }
    return g;
  }
  void release() {
    for (auto &kv : graphs) {
      if (kv.second.exec) hipGraphExecDestroy(kv.second.exec);
      if (kv.second.graph) hipGraphDestroy(kv.second.graph);
    }
    graphs.clear();
    for (auto &kv : operations)
      for (void *p : kv.second->owned) hipFree(p);
    operations.clear();
    for (auto &kv : buffers)
      if (kv.second.owned) hipFree(kv.second.ptr);
    buffers.clear();
    if (stream) hipStreamDestroy(stream);
    stream = nullptr;
  }
};

using Session = inferfabric_acl_session;

extern "C" {

uint32_t inferfabric_acl_abi_version(void) { return 2; }
const char *inferfabric_acl_last_error(void) { return g_error.c_str(); }

int32_t inferfabric_acl_open(int32_t device, inferfabric_acl_session **out) {
  return guarded([&] {
    if (!out) throw Failure("null session output");
    *out = nullptr;
    int count = 0;
    hip(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) throw Failure("invalid device " + std::to_string(device));
    auto s = std::make_unique<Session>();
    s->device = device;
    hip(hipSetDevice(device), "hipSetDevice");
    hip(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
    *out = s.release();
  });
}

int32_t inferfabric_acl_close(inferfabric_acl_session *s) {
  return guarded([&] {
    if (!s) return;
    if (s->thread != std::this_thread::get_id()) throw Failure("wrong close thread");
    hip(hipSetDevice(s->device), "close device");
    if (s->stream) hip(hipStreamSynchronize(s->stream), "close fence");
    s->release();
    delete s;
  });
}

int32_t inferfabric_acl_set_memory_budget(inferfabric_acl_session *s, uint64_t bytes,
                                          uint64_t reserve) {
  return guarded([&] {
    if (!s || !bytes) throw Failure("invalid memory budget");
    s->enter();
    const auto [free, total] = s->observe();
    if (bytes > total || free <= reserve) throw Failure("insufficient free HBM for memory reserve");
    s->budget = std::min<uint64_t>(bytes, free - reserve);
    s->reserve = reserve;
    s->baseline_free = free;
    s->minimum_free = free;
  });
}

int32_t inferfabric_acl_memory_snapshot(inferfabric_acl_session *s,
                                        inferfabric_acl_memory_stats *out) {
  return guarded([&] {
    if (!s || !out) throw Failure("invalid memory snapshot");
    s->enter();
    s->fence("memory snapshot fence");
    const auto [free, total] = s->observe();
    *out = {};
    out->free_bytes = free;
    out->total_bytes = total;
    out->observed_peak_bytes = s->baseline_free > s->minimum_free ? s->baseline_free - s->minimum_free : 0;
    out->budget_bytes = s->budget;
    out->graphs = s->graphs.size();
    for (const auto &kv : s->buffers)
      if (kv.second.owned) out->buffer_bytes += kv.second.bytes;
    for (const auto &kv : s->operations) out->workspace_bytes += kv.second->workspace_bytes;
    s->check_allocation(0);
  });
}

int32_t inferfabric_acl_allocation_snapshot(inferfabric_acl_session *s,
                                            inferfabric_acl_allocation_stats *out) {
  return guarded([&] {
    if (!s || !out) throw Failure("invalid allocation snapshot");
    s->enter();
    *out = {};
    out->dedicated_workspaces = 1;
    for (const auto &kv : s->operations) {
      out->logical_workspace_bytes += kv.second->workspace_bytes;
      out->workspace_blocks += kv.second->owned.size();
    }
    for (const auto &kv : s->buffers) {
      if (kv.second.owned)
        ++out->owned_buffers;
      else
        ++out->buffer_views;
    }
  });
}

int32_t inferfabric_acl_allocate(inferfabric_acl_session *s, uint64_t bytes, uint64_t *handle) {
  return guarded([&] {
    if (!s || !handle || bytes == 0 || bytes > std::numeric_limits<size_t>::max())
      throw Failure("invalid allocation");
    s->enter();
    void *p = s->device_alloc(bytes, "hipMalloc");
    const uint64_t id = s->next++;
    s->buffers.emplace(id, Session::Buffer{p, bytes, true});
    *handle = id;
  });
}

int32_t inferfabric_acl_buffer_view(inferfabric_acl_session *s, uint64_t parent, uint64_t offset,
                                    uint64_t bytes, uint64_t *handle) {
  return guarded([&] {
    if (!s || !handle || !bytes || offset % 512) throw Failure("invalid aligned buffer view");
    s->enter();
    void *p = s->region(parent, offset, bytes);
    const uint64_t id = s->next++;
    s->buffers.emplace(id, Session::Buffer{p, bytes, false});
    *handle = id;
  });
}

int32_t inferfabric_acl_write(inferfabric_acl_session *s, uint64_t handle, uint64_t offset,
                              const void *host, uint64_t bytes) {
  return guarded([&] {
    if (!s || !host) throw Failure("null write argument");
    s->enter();
    void *dst = s->region(handle, offset, bytes);
    hip(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, s->stream), "write H2D");
    s->fence("write fence");
  });
}

int32_t inferfabric_acl_read(inferfabric_acl_session *s, uint64_t handle, uint64_t offset,
                             void *host, uint64_t bytes) {
  return guarded([&] {
    if (!s || !host) throw Failure("null read argument");
    s->enter();
    void *src = s->region(handle, offset, bytes);
    hip(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, s->stream), "read D2H");
    s->fence("read fence");
  });
}

int32_t inferfabric_acl_copy_region(inferfabric_acl_session *s, uint64_t src, uint64_t src_offset,
                                    uint64_t dst, uint64_t dst_offset, uint64_t bytes) {
  return guarded([&] {
    if (!s) throw Failure("null copy session");
    s->enter();
    void *d = s->region(dst, dst_offset, bytes);
    void *from = s->region(src, src_offset, bytes);
    hip(hipMemcpyAsync(d, from, bytes, hipMemcpyDeviceToDevice, s->stream), "copy region");
    s->fence("copy region fence");
  });
}

int32_t inferfabric_acl_capture_copy(inferfabric_acl_session *s, uint64_t source,
                                     uint64_t destination, uint64_t bytes, uint64_t *graph) {
  return guarded([&] {
    if (!s || !graph || source == destination || bytes == 0) throw Failure("invalid graph arguments");
    s->enter();
    void *src = s->region(source, 0, bytes);
    void *dst = s->region(destination, 0, bytes);
    hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s->stream), "warmup copy");
    s->fence("warmup fence");
    Session::Graph g = s->capture([&] {
      hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s->stream), "captured copy");
    });
    *graph = s->add_graph(g);
  });
}

int32_t inferfabric_acl_replay(inferfabric_acl_session *s, uint64_t graph) {
  return guarded([&] {
    if (!s) throw Failure("null session");
    s->enter();
    auto it = s->graphs.find(graph);
    if (it == s->graphs.end()) throw Failure("unknown graph");
    hip(hipGraphLaunch(it->second.exec, s->stream), "graph replay");
    s->fence("replay fence");
    s->check_allocation(0);
  });
}

int32_t inferfabric_acl_operation_execute(inferfabric_acl_session *s, uint64_t operation) {
  return guarded([&] {
    if (!s) throw Failure("null session");
    s->enter();
    auto it = s->operations.find(operation);
    if (it == s->operations.end()) throw Failure("unknown operation");
    it->second->run(s->stream);
    s->fence("operation fence");
  });
}

int32_t inferfabric_acl_operation_capture(inferfabric_acl_session *s, uint64_t operation,
                                          uint64_t *graph) {
  return guarded([&] {
    if (!s || !graph) throw Failure("null capture argument");
    s->enter();
    auto it = s->operations.find(operation);
    if (it == s->operations.end()) throw Failure("unknown operation");
    const Session::Operation &op = *it->second;
    op.run(s->stream);  // eager warm-up, as the reference runs before capturing
    s->fence("operation warmup fence");
    Session::Graph g = s->capture([&] { op.run(s->stream); });
    *graph = s->add_graph(g);
  });
}

int32_t inferfabric_acl_sequence_prepare(inferfabric_acl_session *s, const uint64_t *ids,
                                         uint64_t count, uint64_t *operation) {
  return guarded([&] {
    if (!s || !ids || !operation || count == 0 || count > 4096) throw Failure("invalid sequence");
    s->enter();
    auto op = std::make_unique<Session::Operation>();
    for (uint64_t i = 0; i < count; ++i) {
      auto it = s->operations.find(ids[i]);
      if (it == s->operations.end()) throw Failure("unknown child operation");
      op->children.push_back(it->second.get());
    }
    *operation = s->add_operation(std::move(op));
  });
}

int32_t inferfabric_acl_attention_qk_prepare(inferfabric_acl_session *s, uint64_t packed_q,
                                             uint64_t kin, uint64_t qgamma, uint64_t kgamma,
                                             uint64_t positions, uint64_t qout, uint64_t kout,
                                             uint64_t gate, int64_t batch, uint64_t *operation) {
  return guarded([&] {
    if (!s || !operation || batch <= 0 || batch > 64) throw Failure("invalid QK batch");
    s->enter();
    const uint64_t b = uint64_t(batch);
    const void *pq = s->region(packed_q, 0, b * 4096 * 2);
    const void *k = s->region(kin, 0, b * 512 * 2);
    const float *qg = static_cast<const float *>(s->region(qgamma, 0, 256 * 4));
    const float *kg = static_cast<const float *>(s->region(kgamma, 0, 256 * 4));
    const int64_t *pos = static_cast<const int64_t *>(s->region(positions, 0, b * 8));
    void *qo = s->region(qout, 0, b * 2048 * 2);
    void *ko = s->region(kout, 0, b * 512 * 2);
    void *go = s->region(gate, 0, b * 2048 * 2);
    auto op = std::make_unique<Session::Operation>();
    op->launches.push_back([=](hipStream_t st) {
      ifattn_ok(ifattn_qk_norm_rope_gate_bf16(pq, k, qg, kg, pos, qo, ko, go, batch, st),
                "attention qk");
    });
    *operation = s->add_operation(std::move(op));
  });
}

int32_t inferfabric_acl_paged_attention_prepare(inferfabric_acl_session *s, uint64_t q, uint64_t k,
                                                uint64_t v, uint64_t gate, uint64_t keys,
                                                uint64_t values, uint64_t append, uint64_t table,
                                                uint64_t mask, uint64_t out, int64_t batch,
                                                int64_t slots, int64_t context,
                                                uint64_t *operation) {
  return guarded([&] {
    if (!s || !operation || batch <= 0 || batch > 64 || slots <= 0 || slots > 1048576 ||
        context <= 0 || context > 262144)
      throw Failure("invalid attention capacity");
    s->enter();
    const uint64_t b = uint64_t(batch), n = uint64_t(slots), c = uint64_t(context);
    const void *qp = s->region(q, 0, b * 2048 * 2);
    const void *kp = s->region(k, 0, b * 512 * 2);
    const void *vp = s->region(v, 0, b * 512 * 2);
    void *kc = s->region(keys, 0, n * 512 * 2);
    void *vc = s->region(values, 0, n * 512 * 2);
    const int64_t *ap = static_cast<const int64_t *>(s->region(append, 0, b * 8));
    const int64_t *tp = static_cast<const int64_t *>(s->region(table, 0, b * c * 8));
    const float *mp = static_cast<const float *>(s->region(mask, 0, b * c * 4));
    const void *gp = s->region(gate, 0, b * 2048 * 2);
    void *op_out = s->region(out, 0, b * 2048 * 2);
    auto op = std::make_unique<Session::Operation>();
    const uint64_t ws_bytes = ifattn_gated_paged_attention_workspace_size(batch, context);
    void *ws = s->device_alloc(ws_bytes, "attention workspace");
    op->owned.push_back(ws);
    op->workspace_bytes = ws_bytes;
    op->launches.push_back([=](hipStream_t st) {
      ifattn_ok(ifattn_gated_paged_attention_bf16(qp, kp, vp, gp, kc, vc, ap, tp, mp, op_out, batch,
                                                  slots, context, ws, ws_bytes, st),
                "paged attention");
    });
    try {
      *operation = s->add_operation(std::move(op));
    } catch (...) {
      hipFree(ws);
      throw;
    }
  });
}

int32_t inferfabric_acl_linear_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                       int64_t, int64_t, int64_t, uint64_t *) {
  return not_served("inferfabric_acl_linear_prepare");
}
int32_t inferfabric_acl_linear_execute(inferfabric_acl_session *s, uint64_t operation) {
  return inferfabric_acl_operation_execute(s, operation);
}
int32_t inferfabric_acl_linear_capture(inferfabric_acl_session *s, uint64_t operation,
                                       uint64_t *graph) {
  return inferfabric_acl_operation_capture(s, operation, graph);
}
int32_t inferfabric_acl_rms_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                    int64_t, int64_t, uint64_t *) {
  return not_served("inferfabric_acl_rms_prepare");
}
int32_t inferfabric_acl_delta_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                      uint64_t, uint64_t, uint64_t, uint64_t, int64_t, int64_t,
                                      int64_t, uint64_t *) {
  return not_served("inferfabric_acl_delta_prepare");
}
int32_t inferfabric_acl_conv_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                     uint64_t, int64_t, int64_t, uint64_t *) {
  return not_served("inferfabric_acl_conv_prepare");
}
int32_t inferfabric_acl_pointwise_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                          int64_t, int32_t, uint64_t *) {
  return not_served("inferfabric_acl_pointwise_prepare");
}
int32_t inferfabric_acl_delta_transforms_prepare(inferfabric_acl_session *, uint64_t, uint64_t,
                                                 uint64_t, uint64_t, uint64_t, uint64_t, uint64_t,
                                                 uint64_t, uint64_t, uint64_t, int64_t,
                                                 uint64_t *) {
  return not_served("inferfabric_acl_delta_transforms_prepare");
}
int32_t inferfabric_acl_gated_rms_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                          uint64_t, int64_t, int64_t, uint64_t *) {
  return not_served("inferfabric_acl_gated_rms_prepare");
}
int32_t inferfabric_acl_embedding_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                          int64_t, int64_t, uint64_t *) {
  return not_served("inferfabric_acl_embedding_prepare");
}
int32_t inferfabric_acl_model_layer_prepare(inferfabric_acl_session *, int32_t, const uint64_t *,
                                            uint64_t, uint64_t, uint64_t, uint64_t, uint64_t,
                                            uint64_t, uint64_t, int64_t, int64_t, uint64_t *,
                                            uint64_t *, uint64_t *) {
  return not_served("inferfabric_acl_model_layer_prepare");
}
int32_t inferfabric_acl_embedding_batch_prepare(inferfabric_acl_session *, uint64_t, uint64_t,
                                                int64_t, int64_t, int64_t, uint64_t *) {
  return not_served("inferfabric_acl_embedding_batch_prepare");
}
int32_t inferfabric_acl_model_layer_batch_prepare(inferfabric_acl_session *, int32_t,
                                                  const uint64_t *, uint64_t, uint64_t, uint64_t,
                                                  uint64_t, uint64_t, uint64_t, uint64_t, int64_t,
                                                  int64_t, int64_t, uint64_t, uint64_t *,
                                                  uint64_t *, uint64_t *) {
  return not_served("inferfabric_acl_model_layer_batch_prepare");
}
int32_t inferfabric_acl_sampler_prepare(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                        uint64_t, uint64_t, uint64_t, uint64_t, uint64_t, uint64_t,
                                        int64_t, int64_t, int32_t, uint64_t *) {
  return not_served("inferfabric_acl_sampler_prepare");
}
int32_t inferfabric_acl_random_fill(inferfabric_acl_session *, uint64_t, int64_t, uint64_t) {
  return not_served("inferfabric_acl_random_fill");
}

int32_t inferfabric_acl_device_count(uint32_t *count) {
  return guarded([&] {
    if (!count) throw Failure("null device count");
    int n = 0;
    hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    *count = uint32_t(n);
  });
}
uint64_t inferfabric_acl_tp_root_size(void) { return 0; }
int32_t inferfabric_acl_tp_root(void *, uint64_t) {
  g_error = "inferfabric_acl_tp_root: not in this library (one GPU, no collectives)";
  return -1;
}
int32_t inferfabric_acl_tp_init(inferfabric_acl_session *, uint32_t, uint32_t, const void *,
                                uint64_t) {
  g_error = "inferfabric_acl_tp_init: not in this library (one GPU, no collectives)";
  return -1;
}

}  // extern "C"
