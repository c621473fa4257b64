// Stand-alone C++ host driver of the attention path: no Python, no PyTorch.
// It binds libifattn_hip.so and one operator plug-in with dlopen/dlsym, the
// way the reference's hosts bind their native libraries (Rust libloading in
// crates/inferfabric-native/src/ffi.rs:36-70, C++ CompiledKernel in
// native/src/compiled_kernel.cpp:39-57), and runs one continuous-batching
// decode workload end to end:
//   host metadata (ResidentPages partitions, block tables, slot mapping) via
//   the host C ABI -> device buffers with hipMalloc -> the fused step
//   (slot-mapped K/V write + paged GQA decode) via the direct C ABI ->
//   the same step through the IFKernelV1 plug-ins (write, then decode) ->
//   bitwise comparison of the two outputs and caches -> timing with HIP events.
// Prints one JSON line. Usage:
//   ifattn_drive [--seqs N] [--lo L] [--hi H] [--steps K] [--seed S] [--libdir DIR]
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ifattn.h"
#include "../../include/ifattn_host.h"
#include "../../include/inferfabric_kernel_v1.h"

namespace {

[[noreturn]] void die(const std::string &what) {
  std::fprintf(stdout, "{\"status\": \"error\", \"error\": \"%s\"}\n", what.c_str());
  std::exit(1);
}
void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) die(std::string(what) + ": " + hipGetErrorString(e));
}

struct Lib {
  void *h = nullptr;
  template <typename F>
  F sym(const char *name) {
    void *p = dlsym(h, name);
    if (!p) die(std::string("missing symbol ") + name);
    return reinterpret_cast<F>(p);
  }
};

uint64_t g_rng = 0x9E3779B97F4A7C15ull;
uint64_t next_u64() {  // xorshift64*
  g_rng ^= g_rng >> 12;
  g_rng ^= g_rng << 25;
  g_rng ^= g_rng >> 27;
  return g_rng * 0x2545F4914F6CDD1Dull;
}
float uniform01() { return float(next_u64() >> 40) / float(1 << 24); }
float normal() {  // Box-Muller
  const float u = uniform01() + 1e-7f, v = uniform01();
  return std::sqrt(-2.0f * std::log(u)) * std::cos(6.28318530718f * v);
}
uint16_t bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

IFKernelTensorV1 desc(void *data, uint32_t dtype, uint32_t access, std::vector<int64_t> shape,
                      uint64_t elem) {
  IFKernelTensorV1 t{};
  t.struct_bytes = sizeof(IFKernelTensorV1);
  t.dtype = dtype;
  t.access = access;
  t.rank = uint32_t(shape.size());
  t.data = data;
  int64_t stride = 1;
  for (int i = int(shape.size()) - 1; i >= 0; --i) {
    t.shape[i] = shape[i];
    t.strides[i] = stride;
    stride *= shape[i];
  }
  t.allocation_bytes = uint64_t(stride) * elem;
  return t;
}

}  // namespace

int main(int argc, char **argv) {
  int seqs = 8, lo = 16, hi = 512, steps = 20;
  uint64_t seed = 1;
  std::string libdir;
  {
    std::string self = argv[0];
    const size_t slash = self.rfind('/');
    libdir = slash == std::string::npos ? "." : self.substr(0, slash);
  }
  for (int i = 1; i + 1 < argc; i += 2) {
    const std::string k = argv[i];
    if (k == "--seqs") seqs = std::atoi(argv[i + 1]);
    else if (k == "--lo") lo = std::atoi(argv[i + 1]);
    else if (k == "--hi") hi = std::atoi(argv[i + 1]);
    else if (k == "--steps") steps = std::atoi(argv[i + 1]);
    else if (k == "--seed") seed = std::strtoull(argv[i + 1], nullptr, 10);
    else if (k == "--libdir") libdir = argv[i + 1];
    else die("unknown argument " + k);
  }
  if (seqs < 1 || seqs > 64 || lo < 1 || hi < lo || steps < 1)
    die("need 1 <= seqs <= 64 (ResidentPages slots) and 1 <= lo <= hi");
  g_rng ^= seed * 0xD1B54A32D192ED03ull;

  Lib lib{dlopen((libdir + "/libifattn_hip.so").c_str(), RTLD_NOW | RTLD_GLOBAL)};
  if (!lib.h) die(std::string("dlopen libifattn_hip.so: ") + dlerror());
  auto last_error = lib.sym<const char *(*)()>("ifattn_last_error");
  auto status = [&](int32_t st, const char *what) {
    if (st != 0) die(std::string(what) + ": " + last_error());
  };
  auto pages_create = lib.sym<decltype(&ifattn_pages_create)>("ifattn_pages_create");
  auto pages_select = lib.sym<decltype(&ifattn_pages_select)>("ifattn_pages_select");
  auto pages_bind = lib.sym<decltype(&ifattn_pages_bind)>("ifattn_pages_bind");
  auto pages_owned = lib.sym<decltype(&ifattn_pages_owned)>("ifattn_pages_owned");
  auto slot_mapping = lib.sym<decltype(&ifattn_pages_slot_mapping)>("ifattn_pages_slot_mapping");
  auto batch_table = lib.sym<decltype(&ifattn_pages_batch_table)>("ifattn_pages_batch_table");
  auto pages_destroy = lib.sym<decltype(&ifattn_pages_destroy)>("ifattn_pages_destroy");
  auto ws_size = lib.sym<decltype(&ifattn_paged_decode_workspace_size)>(
      "ifattn_paged_decode_workspace_size");
  auto step = lib.sym<decltype(&ifattn_paged_decode_step_bf16)>("ifattn_paged_decode_step_bf16");

  // ---- model shape of the reference's GQA config (16 q / 2 kv heads, 128 dims, 128-token pages)
  const int hq = 16, hkv = 2, hd = 128, page = 128;
  const int pages_per_seq = (hi + page - 1) / page;
  const int logical = pages_per_seq * page;
  const int64_t num_blocks = int64_t(pages_per_seq) * seqs;
  const int64_t nslot = num_blocks * page;
  const int64_t row = int64_t(hkv) * hd;  // bf16 per cache row (K or V)

  // ---- host metadata: every sequence owns a fixed partition, pages permuted inside it
  ifattn_pages *pages = nullptr;
  status(pages_create(page, logical, seqs, 0, &pages), "ResidentPages");
  std::vector<int32_t> lens(seqs), residents(seqs), positions(seqs);
  for (int s = 0; s < seqs; ++s) {
    status(pages_select(pages, s), "select");
    std::vector<int32_t> own(pages_per_seq);
    uint64_t n = 0;
    status(pages_owned(pages, s, own.data(), own.size(), &n), "owned");
    for (int i = pages_per_seq - 1; i > 0; --i) std::swap(own[i], own[next_u64() % (i + 1)]);
    status(pages_bind(pages, own.data(), own.size()), "bind");
    lens[s] = lo + int(next_u64() % uint64_t(hi - lo + 1));
    residents[s] = s;
    positions[s] = lens[s] - 1;  // the step's new token
  }
  std::vector<int32_t> table(size_t(seqs) * pages_per_seq);
  status(batch_table(pages, residents.data(), seqs, pages_per_seq, 0, table.data()), "batch table");
  std::vector<int64_t> slots(seqs);
  status(slot_mapping(pages, residents.data(), positions.data(), seqs, slots.data()), "slot mapping");
  pages_destroy(pages);

  // ---- synthetic bf16 data, N(0,1)
  auto randn_bf16 = [](size_t n) {
    std::vector<uint16_t> v(n);
    for (auto &x : v) x = bf16_rne(normal());
    return v;
  };
  const auto hk = randn_bf16(size_t(nslot) * row), hv = randn_bf16(size_t(nslot) * row);
  const auto hq_ = randn_bf16(size_t(seqs) * hq * hd);
  const auto hkn = randn_bf16(size_t(seqs) * row), hvn = randn_bf16(size_t(seqs) * row);

  // ---- device buffers
  auto dalloc = [](size_t bytes) {
    void *p = nullptr;
    hip_check(hipMalloc(&p, bytes), "hipMalloc");
    return p;
  };
  auto up = [&](const void *h, size_t bytes) {
    void *d = dalloc(bytes);
    hip_check(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice), "upload");
    return d;
  };
  const size_t cache_b = size_t(nslot) * row * 2;
  void *k1 = up(hk.data(), cache_b), *v1 = up(hv.data(), cache_b);
  void *k2 = up(hk.data(), cache_b), *v2 = up(hv.data(), cache_b);
  void *q = up(hq_.data(), hq_.size() * 2), *kn = up(hkn.data(), hkn.size() * 2),
       *vn = up(hvn.data(), hvn.size() * 2);
  void *dt = up(table.data(), table.size() * 4), *dl = up(lens.data(), lens.size() * 4),
       *ds = up(slots.data(), slots.size() * 8);
  const size_t out_b = size_t(seqs) * hq * hd * 2;
  void *o1 = dalloc(out_b), *o2 = dalloc(out_b);
  const int max_ctx = pages_per_seq * page;
  const uint64_t wsb = ws_size(seqs, hq, hd, max_ctx);
  void *ws = dalloc(wsb ? wsb : 16);
  hipStream_t stream;
  hip_check(hipStreamCreate(&stream), "stream");
  const float scale = 1.0f / std::sqrt(float(hd));

  // ---- direct C ABI: fused step
  auto run_step = [&]() {
    status(step(q, kn, vn, k1, v1, ds, IFATTN_DTYPE_I64, seqs, static_cast<const int32_t *>(dt),
                pages_per_seq, static_cast<const int32_t *>(dl), o1, seqs, hq, hkv, hd, page,
                num_blocks, max_ctx, scale, ws, wsb, stream),
           "ifattn_paged_decode_step_bf16");
  };
  run_step();
  hip_check(hipStreamSynchronize(stream), "step");

  // ---- plug-ins: write, then decode (the reference loader's calling sequence)
  auto plugin = [&](const char *file) {
    void *h = dlopen((libdir + "/" + file).c_str(), RTLD_NOW);
    if (!h) die(std::string("dlopen ") + file + ": " + dlerror());
    auto entry = reinterpret_cast<IFKernelEntryV1>(dlsym(h, "inferfabric_kernel_v1"));
    if (!entry) die(std::string("no inferfabric_kernel_v1 in ") + file);
    const IFKernelV1 *k1 = entry(1);  // the reference loader's request
    if (!k1 || k1->abi_version != 1) die("version-1 handshake");
    const IFKernelV1 *k = entry(2);
    if (!k || k->abi_version != 2 || std::strcmp(k->target, "gfx950") != 0) die("plug-in handshake");
    return k;
  };
  auto enqueue = [&](const IFKernelV1 *k, std::vector<IFKernelTensorV1> in,
                     std::vector<IFKernelTensorV1> out) {
    IFKernelPreparedV1 p{};
    status(k->prepare(in.data(), uint32_t(in.size()), out.data(), uint32_t(out.size()), &p),
           k->contract);
    void *w = p.workspace_bytes ? dalloc(p.workspace_bytes) : nullptr;
    status(k->enqueue(p.state, w, p.workspace_bytes, stream), k->contract);
    hip_check(hipStreamSynchronize(stream), k->contract);
    k->release(p.state);
    if (w) hip_check(hipFree(w), "hipFree");
  };
  constexpr uint32_t R = IF_KERNEL_ACCESS_READ, W = IF_KERNEL_ACCESS_WRITE,
                     RW = IF_KERNEL_ACCESS_READ_WRITE;
  const std::vector<int64_t> cache_shape{num_blocks, page, hkv, hd};
  enqueue(plugin("libifk_kv_cache_write_bf16.so"),
          {desc(kn, 2, R, {seqs, hkv, hd}, 2), desc(vn, 2, R, {seqs, hkv, hd}, 2),
           desc(ds, 5, R, {seqs}, 8)},
          {desc(k2, 2, RW, cache_shape, 2), desc(v2, 2, RW, cache_shape, 2)});
  enqueue(plugin("libifk_paged_decode_gqa_bf16.so"),
          {desc(q, 2, R, {seqs, hq, hd}, 2), desc(k2, 2, R, cache_shape, 2),
           desc(v2, 2, R, cache_shape, 2), desc(dt, 4, R, {seqs, pages_per_seq}, 4),
           desc(dl, 4, R, {seqs}, 4)},
          {desc(o2, 2, W, {seqs, hq, hd}, 2)});
  auto fetch = [](void *d, size_t bytes) {
    std::vector<uint8_t> h(bytes);
    hip_check(hipMemcpy(h.data(), d, bytes, hipMemcpyDeviceToHost), "download");
    return h;
  };
  const bool same_out = fetch(o1, out_b) == fetch(o2, out_b);
  const bool same_k = fetch(k1, cache_b) == fetch(k2, cache_b);
  const bool same_v = fetch(v1, cache_b) == fetch(v2, cache_b);

  // ---- timing of the fused step (the same rows rewritten each step)
  hipEvent_t e0, e1;
  hip_check(hipEventCreate(&e0), "event");
  hip_check(hipEventCreate(&e1), "event");
  for (int i = 0; i < 3; ++i) run_step();
  hip_check(hipEventRecord(e0, stream), "record");
  for (int i = 0; i < steps; ++i) run_step();
  hip_check(hipEventRecord(e1, stream), "record");
  hip_check(hipEventSynchronize(e1), "sync");
  float ms = 0.0f;
  hip_check(hipEventElapsedTime(&ms, e0, e1), "elapsed");
  ms /= float(steps);
  int64_t ctx = 0, blocks_read = 0;
  for (int s = 0; s < seqs; ++s) {
    ctx += lens[s];
    blocks_read += (lens[s] + page - 1) / page;
  }
  const double bytes = double(ctx) * 2 * row * 2 + double(seqs) * hq * hd * 2 * 2 +
                       double(blocks_read) * 4 + double(seqs) * 4 + double(seqs) * (2 * row * 2 * 2 + 8);
  std::printf(
      "{\"status\": \"%s\", \"driver\": \"C++ dlopen, hipMalloc, no Python\", \"seqs\": %d, "
      "\"context_tokens\": %lld, \"plugin_equals_direct\": {\"out\": %s, \"k_cache\": %s, "
      "\"v_cache\": %s}, \"ms_per_step\": %.5f, \"GBps\": %.2f}\n",
      (same_out && same_k && same_v) ? "ok" : "mismatch", seqs, (long long)ctx,
      same_out ? "true" : "false", same_k ? "true" : "false", same_v ? "true" : "false", ms,
      bytes / (ms * 1e-3) / 1e9);
  return (same_out && same_k && same_v) ? 0 : 2;
}
