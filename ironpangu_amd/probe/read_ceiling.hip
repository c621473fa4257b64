// HBM read-ceiling probe for the measurement leg of bench.py (not part of the
// operator library): how fast one MI355X streams reads of whole 64 KiB blocks,
// in a given order, with the default or the nontemporal cache policy. The
// decode kernels read K/V as 64 KiB blocks in block-table order, so this is the
// ceiling their roofline fraction is compared with.
//
// Workgroup w of a grid of G reads blocks order[w], order[w + G], ... (no
// atomics, no barriers); each of its 256 threads issues its 16-byte loads for
// U blocks before using any (16 U loads in flight per lane) and folds them into
// a checksum that is stored only if it matches an impossible value, so no load
// is dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT, int U>
__global__ __launch_bounds__(256) void read_blocks_kernel(const uint8_t *__restrict__ base,
                                                          const int32_t *__restrict__ order,
                                                          int64_t nblocks, u32x4 *sink) {
  u32x4 acc = {0, 0, 0, 0};
  constexpr int kVecs = 65536 / 16 / 256;  // 16 vectors per thread per block
  const int64_t G = gridDim.x;
  for (int64_t i = blockIdx.x; i < nblocks; i += U * G) {
    u32x4 x[U][kVecs];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t b = i + u * G;
      const u32x4 *blk = reinterpret_cast<const u32x4 *>(
          base + int64_t(order[b < nblocks ? b : i]) * 65536);
#pragma unroll
      for (int v = 0; v < kVecs; ++v) {
        const u32x4 *p = blk + v * 256 + threadIdx.x;
        x[u][v] = NT ? __builtin_nontemporal_load(p) : *p;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < kVecs; ++v) acc ^= x[u][v];
  }
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u) sink[threadIdx.x] = acc;
}

extern "C" int32_t ifattn_probe_read_blocks(const void *base, const int32_t *order, int64_t nblocks,
                                            int32_t nontemporal, int32_t unroll, void *sink,
                                            int32_t workgroups, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t *b = static_cast<const uint8_t *>(base);
  u32x4 *k = static_cast<u32x4 *>(sink);
  if (unroll == 2) {
    if (nontemporal) read_blocks_kernel<true, 2><<<workgroups, 256, 0, s>>>(b, order, nblocks, k);
    else read_blocks_kernel<false, 2><<<workgroups, 256, 0, s>>>(b, order, nblocks, k);
  } else {
    if (nontemporal) read_blocks_kernel<true, 1><<<workgroups, 256, 0, s>>>(b, order, nblocks, k);
    else read_blocks_kernel<false, 1><<<workgroups, 256, 0, s>>>(b, order, nblocks, k);
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
