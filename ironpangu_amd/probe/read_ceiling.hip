// HBM read-ceiling probe for the measurement leg of bench.py (not part of the
// operator library): how fast one MI355X streams reads of whole 64 KiB blocks,
// in a given order, with the default or the nontemporal cache policy. The
// decode kernels read K/V as 64 KiB blocks in block-table order, so this is the
// ceiling their roofline fraction is compared with. A second kernel gathers
// short rows (a few hundred bytes at random row offsets), the access of the
// per-position and index-list attention kernels.
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

// Row gather: rows order[0..nrows) of row_bytes bytes (a multiple of 16) at
// base + order[i] * stride, read as 16-byte vectors. Thread t of the grid takes
// vectors t, t + T, ... (T threads), U of them in flight before any is used.
template <bool NT, int U>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t *__restrict__ base,
                                                          const int32_t *__restrict__ order,
                                                          int64_t nrows, int32_t vecs, int64_t stride,
                                                          u32x4 *sink) {
  u32x4 acc = {0, 0, 0, 0};
  const int64_t T = int64_t(gridDim.x) * blockDim.x;
  const int64_t total = nrows * vecs;
  for (int64_t j0 = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; j0 < total; j0 += U * T) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + u * T < total ? j0 + u * T : j0;
      const int64_t r = j / vecs;
      const u32x4 *p = reinterpret_cast<const u32x4 *>(base + int64_t(order[r]) * stride) + (j - r * vecs);
      x[u] = NT ? __builtin_nontemporal_load(p) : *p;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= x[u];
  }
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u) sink[threadIdx.x] = acc;
}

extern "C" int32_t ifattn_probe_gather_rows(const void *base, const int32_t *order, int64_t nrows,
                                            int32_t row_bytes, int64_t stride, int32_t nontemporal,
                                            void *sink, int32_t workgroups, void *stream) {
  if (row_bytes <= 0 || row_bytes % 16 != 0 || nrows <= 0 || workgroups <= 0) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t *b = static_cast<const uint8_t *>(base);
  u32x4 *k = static_cast<u32x4 *>(sink);
  if (nontemporal) gather_rows_kernel<true, 8><<<workgroups, 256, 0, s>>>(b, order, nrows, row_bytes / 16, stride, k);
  else gather_rows_kernel<false, 8><<<workgroups, 256, 0, s>>>(b, order, nrows, row_bytes / 16, stride, k);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
