// Test driver (no Python in the process): binds libinferfabric_acl.so with
// dlopen/dlsym by the reference's symbol names and replays the call sequence of
// the reference's Qwen attention probe,
// crates/inferfabric-cli/src/npu_probe/attention.rs:82-200:
//   abi_version == 2 check and eager symbol resolution (ffi.rs:36-66), open,
//   allocate every buffer, write the fp32 gammas, attention_qk_prepare,
//   paged_attention_prepare, sequence_prepare of the two, zero inputs, poison
//   the caches, operation_capture, poison again, then per token: write inputs,
//   positions, append rows, table and mask; operation_execute; read out, keys and
//   values; overwrite out with -123; replay the graph; read again and require the
//   replay to equal the eager run bit for bit.
// Default sizes and input formulas are the reference probe's (batch 2, page 4,
// 24 slots, context 12, page maps {4,1,5} and {0,3,2}, six tokens). With --batch,
// --context, --prior and --slots it runs the same sequence at a larger shape:
// each request owns a random set of pages, starts `prior` positions in (those
// rows hold a fixed pattern the test regenerates), and appends one row per token.
// Numerical parity is checked by the calling test against the CPU oracle, from
// the dump this program writes (--dump FILE): per token the inputs, the eager
// output and the appended K/V rows, then the final caches.
// Prints one JSON line.
#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../include/inferfabric_acl.h"

namespace {

[[noreturn]] void die(const std::string &what) {
  std::printf("{\"status\": \"error\", \"error\": \"%s\"}\n", what.c_str());
  std::exit(1);
}

uint16_t bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
// Pattern of rows no token has written: the test regenerates it.
uint16_t pattern(uint64_t slot, uint64_t col) {
  return bf16(float((slot * 131 + col * 7) % 97) / 48.0f - 1.0f);
}

struct Api {
  void *h = nullptr;
  decltype(&inferfabric_acl_abi_version) abi_version;
  decltype(&inferfabric_acl_last_error) last_error;
  decltype(&inferfabric_acl_open) open;
  decltype(&inferfabric_acl_close) close;
  decltype(&inferfabric_acl_allocate) allocate;
  decltype(&inferfabric_acl_write) write;
  decltype(&inferfabric_acl_read) read;
  decltype(&inferfabric_acl_linear_prepare) linear_prepare;
  decltype(&inferfabric_acl_rms_prepare) rms_prepare;
  decltype(&inferfabric_acl_operation_execute) execute;
  decltype(&inferfabric_acl_operation_capture) capture;
  decltype(&inferfabric_acl_replay) replay;
  decltype(&inferfabric_acl_attention_qk_prepare) qk;
  decltype(&inferfabric_acl_paged_attention_prepare) attention;
  decltype(&inferfabric_acl_sequence_prepare) sequence;
  template <typename F>
  void get(F &f, const char *name) {
    f = reinterpret_cast<F>(dlsym(h, name));
    if (!f) die(std::string("missing symbol ") + name);
  }
  void check(int32_t status, const char *what) {
    if (status != 0) die(std::string(what) + ": " + last_error());
  }
};

}  // namespace

int main(int argc, char **argv) {
  std::string lib = "ironpangu_amd/libinferfabric_acl.so", dump;
  int batch = 2, context = 12, prior = 0, tokens = 6, page = 4, device = 0;
  long slots = 24;
  unsigned seed = 1;
  bool reference_shape = true;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto val = [&]() -> const char * {
      if (i + 1 >= argc) die("missing value for " + a);
      return argv[++i];
    };
    if (a == "--lib") lib = val();
    else if (a == "--dump") dump = val();
    else if (a == "--batch") batch = std::atoi(val()), reference_shape = false;
    else if (a == "--context") context = std::atoi(val()), reference_shape = false;
    else if (a == "--prior") prior = std::atoi(val()), reference_shape = false;
    else if (a == "--slots") slots = std::atol(val()), reference_shape = false;
    else if (a == "--page") page = std::atoi(val()), reference_shape = false;
    else if (a == "--tokens") tokens = std::atoi(val());
    else if (a == "--seed") seed = unsigned(std::atoi(val()));
    else die("unknown argument " + a);
  }
  if (batch <= 0 || context <= 0 || page <= 0 || tokens <= 0 || prior < 0 || prior + tokens > context)
    die("bad shape");
  const int pages_per_req = (context + page - 1) / page;
  if (long(batch) * pages_per_req * page > slots) die("pool too small for the requests' pages");

  Api api;
  api.h = dlopen(lib.c_str(), RTLD_NOW | RTLD_LOCAL);
  if (!api.h) die(std::string("dlopen: ") + dlerror());
  api.get(api.abi_version, "inferfabric_acl_abi_version");
  if (api.abi_version() != 2) die("native ABI version mismatch");
  api.get(api.last_error, "inferfabric_acl_last_error");
  api.get(api.open, "inferfabric_acl_open");
  api.get(api.close, "inferfabric_acl_close");
  api.get(api.allocate, "inferfabric_acl_allocate");
  api.get(api.write, "inferfabric_acl_write");
  api.get(api.read, "inferfabric_acl_read");
  api.get(api.linear_prepare, "inferfabric_acl_linear_prepare");
  api.get(api.rms_prepare, "inferfabric_acl_rms_prepare");
  api.get(api.execute, "inferfabric_acl_operation_execute");
  api.get(api.capture, "inferfabric_acl_operation_capture");
  api.get(api.replay, "inferfabric_acl_replay");
  api.get(api.qk, "inferfabric_acl_attention_qk_prepare");
  api.get(api.attention, "inferfabric_acl_paged_attention_prepare");
  api.get(api.sequence, "inferfabric_acl_sequence_prepare");

  inferfabric_acl_session *s = nullptr;
  api.check(api.open(device, &s), "open");
  auto alloc = [&](uint64_t bytes) {
    uint64_t id = 0;
    api.check(api.allocate(s, bytes, &id), "allocate");
    return id;
  };
  auto put = [&](uint64_t id, const void *p, uint64_t bytes) {
    api.check(api.write(s, id, 0, p, bytes), "write");
  };
  auto get = [&](uint64_t id, void *p, uint64_t bytes) {
    api.check(api.read(s, id, 0, p, bytes), "read");
  };
  const uint64_t B = uint64_t(batch), C = uint64_t(context), S = uint64_t(slots);
  const uint64_t qp = alloc(B * 4096 * 2), ki = alloc(B * 512 * 2), vi = alloc(B * 512 * 2);
  const uint64_t q = alloc(B * 2048 * 2), k = alloc(B * 512 * 2), gate = alloc(B * 2048 * 2);
  const uint64_t kg = alloc(256 * 4), qg = alloc(256 * 4);
  // Synthetic norm weights in place of the checkpoint's; gamma = 1 + w.
  std::vector<float> qgamma(256), kgamma(256);
  for (int j = 0; j < 256; ++j) {
    const float wq = float((j * 37) % 29) / 64.0f - 0.2f, wk = float((j * 53) % 31) / 80.0f - 0.15f;
    uint32_t u = uint32_t(bf16(wq)) << 16;
    std::memcpy(&qgamma[j], &u, 4);
    u = uint32_t(bf16(wk)) << 16;
    std::memcpy(&kgamma[j], &u, 4);
    qgamma[j] += 1.0f;
    kgamma[j] += 1.0f;
  }
  put(kg, kgamma.data(), 1024);
  put(qg, qgamma.data(), 1024);
  const uint64_t positions = alloc(B * 8), append = alloc(B * 8);
  const uint64_t table = alloc(B * C * 8), mask = alloc(B * C * 4);
  const uint64_t keys = alloc(S * 512 * 2), values = alloc(S * 512 * 2);
  const uint64_t out = alloc(B * 2048 * 2);

  // linear/rms resolve (the Rust loader binds them) but are not served here.
  uint64_t unused = 0;
  const bool linear_refused = api.linear_prepare(s, qp, k, q, 1, 1, 1, &unused) != 0;

  uint64_t pre = 0, att = 0, op = 0;
  api.check(api.qk(s, qp, ki, qg, kg, positions, q, k, gate, batch, &pre), "attention_qk_prepare");
  api.check(api.attention(s, q, k, vi, gate, keys, values, append, table, mask, out, batch, slots,
                          context, &att),
            "paged_attention_prepare");
  const uint64_t children[2] = {pre, att};
  api.check(api.sequence(s, children, 2, &op), "sequence_prepare");

  // Page maps: the reference probe's two fixed maps, else a random disjoint set
  // of pages per request.
  std::vector<std::vector<long>> maps(batch);
  if (reference_shape) {
    maps = {{4, 1, 5}, {0, 3, 2}};
  } else {
    std::mt19937_64 rng(seed);
    std::vector<long> all(S / page);
    for (size_t i = 0; i < all.size(); ++i) all[i] = long(i);
    std::shuffle(all.begin(), all.end(), rng);
    for (int r = 0; r < batch; ++r)
      maps[r].assign(all.begin() + long(r) * pages_per_req, all.begin() + long(r + 1) * pages_per_req);
  }

  std::vector<uint16_t> zeros(B * 4096, 0);
  put(qp, zeros.data(), B * 4096 * 2);
  put(ki, zeros.data(), B * 512 * 2);
  put(vi, zeros.data(), B * 512 * 2);
  std::vector<int64_t> pos0(B, 0), app0(B);
  for (uint64_t r = 0; r < B; ++r) app0[r] = int64_t(maps[r][0] * page);  // (the reference writes {0, 1})
  if (reference_shape) app0 = {0, 1};
  put(positions, pos0.data(), B * 8);
  put(append, app0.data(), B * 8);
  std::vector<int64_t> table0(B * C, 0);
  put(table, table0.data(), B * C * 8);
  std::vector<float> mask0(B * C, 0.0f);
  put(mask, mask0.data(), B * C * 4);
  std::vector<uint16_t> base(S * 512);
  for (uint64_t i = 0; i < S * 512; ++i)
    base[i] = reference_shape ? bf16(0.75f) : pattern(i / 512, i % 512);
  put(keys, base.data(), S * 1024);
  put(values, base.data(), S * 1024);
  uint64_t graph = 0;
  api.check(api.capture(s, op, &graph), "operation_capture");
  put(keys, base.data(), S * 1024);
  put(values, base.data(), S * 1024);

  FILE *f = nullptr;
  if (!dump.empty()) {
    f = std::fopen(dump.c_str(), "wb");
    if (!f) die("cannot open dump file");
    std::fwrite(qgamma.data(), 4, 256, f);
    std::fwrite(kgamma.data(), 4, 256, f);
  }
  bool graph_equal = true;
  std::vector<uint16_t> qin(B * 4096), kin(B * 512), vin(B * 512), eager(B * 2048), replayed(B * 2048);
  std::vector<uint16_t> ek(S * 512), ev(S * 512), rk(S * 512), rv(S * 512);
  std::vector<int64_t> lookup(B * C), indices(B), pos(B);
  std::vector<float> mvals(B * C);
  for (int token = 0; token < tokens; ++token) {
    for (uint64_t i = 0; i < B * 4096; ++i) qin[i] = bf16(float((i * 13 + token * 7) % 79) / 48.0f - 0.7f);
    for (uint64_t i = 0; i < B * 512; ++i) kin[i] = bf16(float((i * 11 + token * 17) % 67) / 43.0f - 0.8f);
    for (uint64_t i = 0; i < B * 512; ++i) vin[i] = bf16(float((i * 17 + token * 5) % 71) / 41.0f - 0.9f);
    std::fill(lookup.begin(), lookup.end(), 0);
    std::fill(mvals.begin(), mvals.end(), -INFINITY);
    const int p = prior + token;
    for (int r = 0; r < batch; ++r) {
      for (int j = 0; j <= p; ++j) {
        lookup[r * C + j] = maps[r][j / page] * page + j % page;
        mvals[r * C + j] = 0.0f;
      }
      indices[r] = lookup[r * C + p];
      pos[r] = p;
    }
    put(qp, qin.data(), B * 4096 * 2);
    put(ki, kin.data(), B * 512 * 2);
    put(vi, vin.data(), B * 512 * 2);
    put(positions, pos.data(), B * 8);
    put(append, indices.data(), B * 8);
    put(table, lookup.data(), B * C * 8);
    put(mask, mvals.data(), B * C * 4);
    api.check(api.execute(s, op), "operation_execute");
    get(out, eager.data(), B * 4096);
    get(keys, ek.data(), S * 1024);
    get(values, ev.data(), S * 1024);
    std::vector<uint16_t> poison(B * 2048, bf16(-123.0f));
    put(out, poison.data(), B * 4096);
    api.check(api.replay(s, graph), "replay");
    get(out, replayed.data(), B * 4096);
    get(keys, rk.data(), S * 1024);
    get(values, rv.data(), S * 1024);
    graph_equal = graph_equal && replayed == eager && rk == ek && rv == ev;
    if (f) {
      std::fwrite(qin.data(), 2, qin.size(), f);
      std::fwrite(kin.data(), 2, kin.size(), f);
      std::fwrite(vin.data(), 2, vin.size(), f);
      std::fwrite(pos.data(), 8, pos.size(), f);
      std::fwrite(indices.data(), 8, indices.size(), f);
      std::fwrite(lookup.data(), 8, lookup.size(), f);
      std::fwrite(mvals.data(), 4, mvals.size(), f);
      std::fwrite(eager.data(), 2, eager.size(), f);
      std::vector<uint16_t> rows(B * 1024);
      for (uint64_t r = 0; r < B; ++r) {
        std::memcpy(&rows[r * 1024], &ek[uint64_t(indices[r]) * 512], 1024);
        std::memcpy(&rows[r * 1024 + 512], &ev[uint64_t(indices[r]) * 512], 1024);
      }
      std::fwrite(rows.data(), 2, rows.size(), f);
    }
  }
  if (f) {
    std::fwrite(ek.data(), 2, ek.size(), f);
    std::fwrite(ev.data(), 2, ev.size(), f);
    std::fclose(f);
  }
  api.check(api.close(s), "close");
  std::printf(
      "{\"status\": \"ok\", \"abi_version\": %u, \"batch\": %d, \"context\": %d, \"prior\": %d, "
      "\"slots\": %ld, \"page\": %d, \"tokens\": %d, \"graph_equals_eager\": %s, "
      "\"linear_refused\": %s}\n",
      api.abi_version(), batch, context, prior, slots, page, tokens, graph_equal ? "true" : "false",
      linear_refused ? "true" : "false");
  return 0;
}
