// Per-operator plug-in library: exports the reference loader's entry symbol
// (native/src/compiled_kernel.cpp:45-48) and forwards to libifattn_hip.so.
// Built once per contract with -DIFK_CONTRACT_INDEX=<n>.
#include "../../include/inferfabric_kernel_v1.h"

#ifndef IFK_CONTRACT_INDEX
#error "IFK_CONTRACT_INDEX must select the operator contract"
#endif

extern "C" const IFKernelV1 *ifattn_kernel_v1_operator(int32_t index, uint32_t requested_version);

// Version 1 (the reference loader's request) or 2; NULL for any other version.
extern "C" __attribute__((visibility("default"))) const IFKernelV1 *inferfabric_kernel_v1(
    uint32_t requested_version) {
  return ifattn_kernel_v1_operator(IFK_CONTRACT_INDEX, requested_version);
}
