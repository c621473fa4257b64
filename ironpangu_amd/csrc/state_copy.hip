// Device execution of the host page plans: zeroing the owned page spans of a
// state field when a resident slot is reset (page_spans,
// native/src/page_binding.h:19-35) and copying a resident's pages to another
// slot (copy_plan, page_binding.h:161-187). The plans are read on the device,
// so the launches can be recorded into a HIP graph and replayed with new plans.
//
// Both kernels are HBM-streaming: one grid row of workgroups per span, each
// taking a strided share of its 16-byte vectors, eight per thread per pass
// (nontemporal loads and stores: the bytes are not read again soon; the
// loads measured copy 381 -> 368 us per GiB). Spans whose offset, size or base
// are not 16-byte aligned fall back to a byte loop; spans outside the field
// and copy ranges whose source and destination overlap are skipped. The
// checked entry points validate the whole plan first, in a one-workgroup
// kernel, as the reference validates every copy before issuing it
// (native/src/prepared_execution.h:346-354): an invalid plan moves no byte and
// leaves the 1-based index of its first bad span in a device status word. The span
// sizes live on the device, so the second grid dimension is sized from the
// field's average share per span: a plan mixing one small span into a large
// field launches idle workgroups for it, which exit at once.
#include "common.h"
#include "ifattn_internal.h"
#include "split_k.h"

namespace ifattn {

// spans: {offset, bytes} pairs (reset) or {source, destination, bytes} triples
// (copy). Workgroup (i, j) takes span i and every gridDim.y-th 4 KiB piece of
// it starting at piece j (eight pieces per pass).
// A span the reference rejects: empty, outside the field, or (copies) with
// overlapping source and destination.
template <bool COPY>
__device__ __forceinline__ bool span_bad(uint64_t src, uint64_t dst, uint64_t bytes,
                                         uint64_t field_bytes) {
  return bytes == 0 || src > field_bytes || bytes > field_bytes - src || dst > field_bytes ||
         bytes > field_bytes - dst || (COPY && src < dst + bytes && dst < src + bytes);
}

// Plan check of the checked entry points: *status = 1 + index of the first
// bad span, or 0.
template <bool COPY>
__global__ __launch_bounds__(1024) void state_plan_check_kernel(uint64_t field_bytes,
                                                                const uint64_t *__restrict__ spans,
                                                                uint64_t count, int32_t *status) {
  constexpr int W = COPY ? 3 : 2;
  __shared__ unsigned long long first;
  if (threadIdx.x == 0) first = ~0ull;
  __syncthreads();
  for (uint64_t i = threadIdx.x; i < count; i += blockDim.x) {
    const uint64_t src = spans[W * i], dst = COPY ? spans[W * i + 1] : src;
    if (span_bad<COPY>(src, dst, spans[W * i + W - 1], field_bytes)) {
      atomicMin(&first, (unsigned long long)i);
      break;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) *status = first == ~0ull ? 0 : int32_t(first + 1);
}

template <bool COPY>
__global__ __launch_bounds__(256) void state_span_kernel(uint8_t *__restrict__ field,
                                                         uint64_t field_bytes,
                                                         const uint64_t *__restrict__ spans,
                                                         const int32_t *__restrict__ status) {
  constexpr int W = COPY ? 3 : 2;
  if (status && *status != 0) return;  // checked call with an invalid plan: nothing moves
  const uint64_t i = blockIdx.x;
  const uint64_t src = spans[W * i];
  const uint64_t dst = COPY ? spans[W * i + 1] : src;
  const uint64_t bytes = spans[W * i + W - 1];
  if (bytes == 0 || src > field_bytes || bytes > field_bytes - src || dst > field_bytes ||
      bytes > field_bytes - dst)
    return;
  // A copy range whose source and destination overlap has no defined result
  // under a parallel copy; such ranges are skipped (copy plans move pages
  // between distinct residents, so they never overlap).
  if (COPY && src < dst + bytes && dst < src + bytes) return;
  const uint64_t lanes = uint64_t(gridDim.y) * blockDim.x;
  const uint64_t me = uint64_t(blockIdx.y) * blockDim.x + threadIdx.x;
  if (((src | dst | bytes | reinterpret_cast<uintptr_t>(field)) & 15u) == 0) {
    const uint64_t n = bytes / 16;
    // Eight vectors per thread per pass: all loads issued before the stores.
    constexpr int U = 8;
    uint64_t v = me;
    for (; v + (U - 1) * lanes < n; v += U * lanes) {
      u32x4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        x[u] = COPY ? __builtin_nontemporal_load((const u32x4 *)(field + src + 16 * (v + u * lanes))) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < U; ++u)
        __builtin_nontemporal_store(x[u], reinterpret_cast<u32x4 *>(field + dst + 16 * (v + u * lanes)));
    }
    for (; v < n; v += lanes) {
      const u32x4 x = COPY ? __builtin_nontemporal_load((const u32x4 *)(field + src + 16 * v)) : u32x4{0, 0, 0, 0};
      __builtin_nontemporal_store(x, reinterpret_cast<u32x4 *>(field + dst + 16 * v));
    }
  } else {
    for (uint64_t b = me; b < bytes; b += lanes) field[dst + b] = COPY ? field[src + b] : 0;
  }
}

namespace {
int32_t run_spans(bool copy, void *field, uint64_t field_bytes, const uint64_t *spans,
                  uint64_t count, int32_t *status, void *stream, const char *what) {
  if (!field || (!spans && count) || field_bytes == 0)
    return fail(IFATTN_EINVAL, what, "null field or plan");
  if (!aligned8(spans) || !aligned4(status)) return fail(IFATTN_EINVAL, what, "misaligned plan or status");
  if (count >= (1ull << 31)) return fail(IFATTN_EINVAL, what, "more than 2^31-1 spans");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (status) {
    if (copy) state_plan_check_kernel<true><<<1, 1024, 0, s>>>(field_bytes, spans, count, status);
    else state_plan_check_kernel<false><<<1, 1024, 0, s>>>(field_bytes, spans, count, status);
  }
  if (count == 0) return status ? launch_status(what) : IFATTN_OK;
  // Span sizes live on the device: size the second grid dimension for the
  // average span (one workgroup per 64 KiB of it, up to 1024). Fewer, fuller
  // workgroups measured faster than one per 4 KiB (1 GiB of 20992-B pages:
  // copy 491 -> 377 us, reset 234 -> 205 us with eight vectors per pass).
  const uint64_t avg = field_bytes / count;
  const unsigned split = unsigned(avg / 65536 + 1 < 1024 ? avg / 65536 + 1 : 1024);
  const dim3 grid(unsigned(count), split);
  if (copy)
    state_span_kernel<true><<<grid, 256, 0, s>>>(static_cast<uint8_t *>(field), field_bytes, spans, status);
  else
    state_span_kernel<false><<<grid, 256, 0, s>>>(static_cast<uint8_t *>(field), field_bytes, spans, status);
  return launch_status(what);
}
}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" int32_t ifattn_page_reset(void *field, uint64_t field_bytes, const uint64_t *spans,
                                     uint64_t count, void *stream) {
  return run_spans(false, field, field_bytes, spans, count, nullptr, stream, "page reset");
}

extern "C" int32_t ifattn_state_copy(void *field, uint64_t field_bytes, const uint64_t *ranges,
                                     uint64_t count, void *stream) {
  return run_spans(true, field, field_bytes, ranges, count, nullptr, stream, "state copy");
}

extern "C" int32_t ifattn_page_reset_checked(void *field, uint64_t field_bytes, const uint64_t *spans,
                                             uint64_t count, int32_t *status, void *stream) {
  if (!status) return fail(IFATTN_EINVAL, "page reset: null status");
  return run_spans(false, field, field_bytes, spans, count, status, stream, "page reset");
}

extern "C" int32_t ifattn_state_copy_checked(void *field, uint64_t field_bytes,
                                             const uint64_t *ranges, uint64_t count,
                                             int32_t *status, void *stream) {
  if (!status) return fail(IFATTN_EINVAL, "state copy: null status");
  return run_spans(true, field, field_bytes, ranges, count, status, stream, "state copy");
}
