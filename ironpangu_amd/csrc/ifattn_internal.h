// Host-side helpers shared by the C-ABI entry points: status codes, the
// thread-local error text (the reference's boundary convention,
// native/src/inferfabric_acl.cpp:46-58), and launch checking.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/ifattn.h"

namespace ifattn {
int32_t fail(int32_t code, const char *message);
// Message "<what>: <message>".
int32_t fail(int32_t code, const char *what, const char *message);
int32_t launch_status(const char *what);
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
inline bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
}  // namespace ifattn
