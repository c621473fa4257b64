// C-ABI shim over the REFERENCE's own operator plug-in loader
// (native/src/compiled_kernel.cpp, native/include/compiled_kernel.h), compiled
// in place from /root/reference into oracle/_ref/libref_loader.so.
// TEST INFRASTRUCTURE ONLY: the tests load the product's libifk_*.so plug-ins
// through the unmodified reference loader (dlopen, inferfabric_kernel_v1(1),
// descriptor and alias checks, single enqueue). No reference source is copied.
#include <new>
#include <string>
#include <vector>

#include "compiled_kernel.h"

using inferfabric::CompiledKernel;
using inferfabric::PreparedKernel;

namespace {
thread_local std::string g_error;
template <typename F>
int guarded(F &&f) {
  try {
    f();
    return 0;
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  }
}
}  // namespace

extern "C" {
const char *ref_loader_error() { return g_error.c_str(); }

int ref_loader_open(const char *library, const char *contract, const char *target, void **out) {
  *out = nullptr;
  return guarded([&] { *out = new CompiledKernel(library, contract, target); });
}
void ref_loader_close(void *k) { delete static_cast<CompiledKernel *>(k); }

int ref_loader_prepare(void *k, const IFKernelTensorV1 *in, uint32_t nin,
                       const IFKernelTensorV1 *out, uint32_t nout, void **prepared,
                       uint64_t *workspace_bytes) {
  *prepared = nullptr;
  return guarded([&] {
    auto p = static_cast<CompiledKernel *>(k)->prepare(
        std::vector<IFKernelTensorV1>(in, in + nin), std::vector<IFKernelTensorV1>(out, out + nout));
    *workspace_bytes = p.workspace_bytes();
    *prepared = new PreparedKernel(std::move(p));
  });
}
int ref_loader_enqueue(void *prepared, void *workspace, uint64_t capacity, void *stream) {
  return guarded([&] { static_cast<PreparedKernel *>(prepared)->enqueue(workspace, capacity, stream); });
}
void ref_loader_release(void *prepared) { delete static_cast<PreparedKernel *>(prepared); }
}
