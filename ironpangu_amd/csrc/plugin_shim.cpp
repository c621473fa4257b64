// Per-operator plug-in library: exports the reference loader's entry symbol
// (native/src/compiled_kernel.cpp:45-48) and forwards to libifattn_hip.so.
// Built once per contract with -DIFK_CONTRACT_INDEX=<n>.
#include "../../include/inferfabric_kernel_v1.h"

#ifndef IFK_CONTRACT_INDEX
#error "IFK_CONTRACT_INDEX must select the operator contract"
#endif

namespace {
const char *const kContracts[] = {
    "inferfabric.kv_cache_write.bf16.v2",   "inferfabric.kv_cache_write.c8.v2",
    "inferfabric.paged_decode.gqa.bf16.v2", "inferfabric.paged_decode.gqa.c8.v2",
    "inferfabric.varlen_prefill.bf16.v2",   "inferfabric.mla_decode.bf16.v2",
    "inferfabric.mla_decode.c8.v2",         "inferfabric.mla_cache_write.c8.v2",
    "inferfabric.mla_norm_rope_cache.bf16.v2", "inferfabric.mla_norm_rope_cache.c8.v2",
    "inferfabric.mla_window_attention.w512.bf16.v2",
    "inferfabric.mla_window_attention.w2048.bf16.v2",
    "inferfabric.mla_sparse_attention.c8.v2",
};
}

extern "C" __attribute__((visibility("default"))) const IFKernelV1 *inferfabric_kernel_v1(
    uint32_t requested_version) {
  return ifattn_kernel_v1_contract(kContracts[IFK_CONTRACT_INDEX], requested_version);
}
