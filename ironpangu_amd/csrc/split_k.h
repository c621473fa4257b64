// Split-K scheduling shared by the paged decode kernels (GQA and MLA):
// per-call device work list in longest-processing-time order, a work queue
// drained by persistent workgroups, (m, l, O) partials per (sequence,
// partition, head) combined by a merge launch. The prologue kernel that builds
// the work list also performs the step's slot-mapped row writes, so a decode
// step is prologue -> decode -> merge from one host call.
#pragma once
#include <cstdlib>

#include "common.h"

namespace ifattn {

struct DecodeParams {
  const uint16_t *q;
  const uint8_t *k_cache;
  const uint8_t *v_cache;
  const float *k_scale;
  const float *v_scale;
  const int32_t *block_tables;
  const int32_t *seq_lens;
  uint16_t *out;
  int32_t *queue;    // [0] next item (atomic), [1] item count; set by the plan kernel
  uint32_t *items;   // (seq << 12 | part) per (sequence, partition), in sequence order
  float *part_o;     // [num_seqs, max_parts, q_heads, D]
  float *part_ml;    // [num_seqs, max_parts, q_heads, 2]
  // Packed varlen batches: when set, sequence s reads/writes q/out row
  // cu_seqlens[s+1]-1 and only sequences with exactly one query row are
  // scheduled here (longer chunks go to the prefill kernel).
  const int32_t *cu_seqlens;
  int64_t num_blocks;
  int num_seqs, q_heads, kv_heads, group, table_stride, block_size, max_context, max_parts,
      part_tokens;
  int static_items;  // items below this index are not queued (0: the queue hands out every item)
  float scale_log2;  // softmax scale * log2(e)
};

__device__ __forceinline__ int clamp_len(const DecodeParams &p, int seq) {
  const int len = p.seq_lens[seq];
  return len > p.max_context ? p.max_context : len;
}
__device__ __forceinline__ int parts_of(int len, int pt) { return len > 0 ? (len + pt - 1) / pt : 1; }
// q / out row of a sequence (identity for plain decode batches).
__device__ __forceinline__ int64_t q_row_of(const DecodeParams &p, int seq) {
  return p.cu_seqlens ? int64_t(p.cu_seqlens[seq + 1]) - 1 : int64_t(seq);
}
__device__ __forceinline__ bool decode_seq(const DecodeParams &p, int seq) {
  return !p.cu_seqlens || p.cu_seqlens[seq + 1] - p.cu_seqlens[seq] == 1;
}

// Exclusive prefix of bucket[0..nb] (nb < 64 * PL) offset by `start`, by the
// first wave (PL buckets per lane, a shuffle scan across lanes); returns the
// total to lane 0 of that wave. Replaces a serial loop of LDS round trips.
template <int PL = 5>
__device__ __forceinline__ int bucket_prefix(int *bucket, int nb, int start, int tid) {
  int total = 0;
  if (tid < 64) {
    int c[PL], sum = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int b = PL * tid + i;
      c[i] = b <= nb ? bucket[b] : 0;
      sum += c[i];
    }
    int x = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      x += tid >= off ? y : 0;
    }
    int run = start + x - sum;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int b = PL * tid + i;
      if (b <= nb) bucket[b] = run;
      run += c[i];
    }
    total = start + __shfl(x, 63, 64);
  }
  return total;
}

// Builds the compact work list on the device (graph-safe: lengths are read at
// run time) and resets the work queue. Longest-processing-time order: every
// full partition first, then the partial tail partitions by decreasing length
// (a counting sort over 32-token buckets), so the last items pulled from the
// queue are the shortest and the persistent workgroups finish together.
// Sequences with no visible key get one zero-length item at the very end.
// One workgroup of 1024 threads.
// Slot-mapped row writes folded into the prologue (cache[slot[r]] = rows[r]).
struct RowWrite {
  const uint8_t *k_rows, *v_rows;
  uint8_t *k_cache, *v_cache;
  const void *slots;
  int slot_i64;
  int64_t rows, row_vecs, num_slots;
};

__device__ __forceinline__ void prologue_write(const RowWrite &w) {
  const int64_t total = w.rows * w.row_vecs * (w.v_rows ? 2 : 1);
  for (int64_t i = int64_t(blockIdx.x - 1) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x - 1) * blockDim.x) {
    const int64_t per = w.rows * w.row_vecs;
    const bool v = i >= per;
    const int64_t j = v ? i - per : i;
    const int64_t r = j / w.row_vecs, c = j - r * w.row_vecs;
    const int64_t slot = w.slot_i64 ? static_cast<const int64_t *>(w.slots)[r]
                                    : int64_t(static_cast<const int32_t *>(w.slots)[r]);
    if (slot < 0 || slot >= w.num_slots) continue;
    const uint8_t *src = v ? w.v_rows : w.k_rows;
    uint8_t *dst = v ? w.v_cache : w.k_cache;
    store_u32x4(dst + (slot * w.row_vecs + c) * 16, load_u32x4(src + (r * w.row_vecs + c) * 16));
  }
}

// Workgroup 0 plans; workgroups 1.. perform the row writes (if any).
template <int Unused = 0>
__global__ __launch_bounds__(1024) void decode_prologue_kernel(DecodeParams p, RowWrite wr) {
  if (blockIdx.x > 0) {
    prologue_write(wr);
    return;
  }
  constexpr int kBuckets = 257;  // 32-token buckets of PT <= 8192, plus empty rows
  __shared__ int bucket[kBuckets];
  __shared__ int carry;
  const int tid = threadIdx.x;
  const int PT = p.part_tokens;
  const int nb = PT / 32;  // bucket b holds remainders in (PT - 32(b+1), PT - 32b]
  for (int b = tid; b < kBuckets; b += 1024) bucket[b] = 0;
  if (tid == 0) carry = 0;
  __syncthreads();
  // Pass 1: full partitions in sequence order; histogram of partial ones.
  __shared__ int wave_tot[16];
  const int lane = tid & 63, wv = tid >> 6;
  for (int base = 0; base < p.num_seqs; base += 1024) {
    const int seq = base + tid;
    int nfull = 0, bk = -1;
    if (seq < p.num_seqs && decode_seq(p, seq)) {
      const int len = clamp_len(p, seq);
      nfull = len > 0 ? len / PT : 0;
      const int rem = len > 0 ? len - nfull * PT : 0;
      bk = len <= 0 ? nb : (rem > 0 ? (PT - rem) / 32 : -1);
      if (bk >= 0) atomicAdd(&bucket[bk], 1);
    }
    // inclusive scan of nfull: within the wave by shuffles, then across waves
    int x = nfull;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      x += lane >= off ? y : 0;
    }
    if (lane == 63) wave_tot[wv] = x;
    __syncthreads();
    int before = carry;
    for (int w2 = 0; w2 < wv; ++w2) before += wave_tot[w2];
    const int start = before + x - nfull;
    for (int k = 0; k < nfull; ++k) p.items[start + k] = (uint32_t(seq) << 12) | uint32_t(k);
    __syncthreads();
    if (tid == 1023) carry = start + nfull;
    __syncthreads();
  }
  // Exclusive scan of the bucket counts, offset by the full-item count.
  {
    const int run = bucket_prefix(bucket, nb, carry, tid);
    if (tid == 0) {
      p.queue[0] = p.static_items;
      p.queue[1] = run;
    }
  }
  __syncthreads();
  // Pass 2: place each partial / empty item in its bucket.
  for (int base = 0; base < p.num_seqs; base += 1024) {
    const int seq = base + tid;
    if (seq < p.num_seqs && decode_seq(p, seq)) {
      const int len = clamp_len(p, seq);
      const int nfull = len > 0 ? len / PT : 0;
      const int rem = len > 0 ? len - nfull * PT : 0;
      const int bk = len <= 0 ? nb : (rem > 0 ? (PT - rem) / 32 : -1);
      if (bk >= 0) p.items[atomicAdd(&bucket[bk], 1)] = (uint32_t(seq) << 12) | uint32_t(nfull);
    }
  }
}

// Merge the split-K partials of one (sequence, head) over the dims
// [dim0, dim0 + DW) with one wave; lane l owns DW/64 consecutive dims. Up to
// kFast partitions go in one round trip: lane k holds partition k's (m, l) and
// every partial-O slice is loaded before any is used; the weights reach the
// other lanes by shuffle. Longer lists are taken kFast at a time.
template <int D, int DW>
__device__ __forceinline__ void merge_head(const DecodeParams &p, int seq, int h, int nparts,
                                           int dim0, int lane) {
  constexpr int V = DW / 64;
  constexpr int kFast = 16;
  // This sequence's partials: partition k, head h is row k * q_heads + h.
  // Buffer offsets stay 32-bit and rows past nparts read as zero.
  const int64_t seq_row = int64_t(seq) * p.max_parts * p.q_heads;
  const uint32_t rows = uint32_t(nparts) * uint32_t(p.q_heads);
  const auto ro = make_rsrc(p.part_o + seq_row * D, rows * D * 4u);
  const auto rm = make_rsrc(p.part_ml + seq_row * 2, rows * 8u);
  const uint32_t ostride = uint32_t(p.q_heads) * D * 4u;
  const uint32_t obase = (uint32_t(h) * D + uint32_t(dim0 + lane * V)) * 4u;
  auto load_ml = [&](int k) {
    const uint32_t off = (uint32_t(k) * p.q_heads + h) * 8u;
    return make_float2(buf_load_f32(rm, off), buf_load_f32(rm, off + 4));
  };
  // Up to kFast partitions take one round trip: the max comes from the same
  // batch of (m, l) loads as the weights. Longer lists scan the maxima first.
  float mmax = -INFINITY;
  if (nparts > kFast) {
    for (int k = lane; k < nparts; k += 64) mmax = fmaxf(mmax, load_ml(k).x);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mmax = wave_max_xor(mmax, m);
  }
  float lsum = 0.0f;
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  for (int k0 = 0; k0 < nparts; k0 += kFast) {
    const int n = nparts - k0 < kFast ? nparts - k0 : kFast;
    const float2 ml = lane < n ? load_ml(k0 + lane) : make_float2(-INFINITY, 0.0f);
    float o[kFast][V];
#pragma unroll
    for (int u = 0; u < kFast; ++u) {
      const uint32_t off = obase + uint32_t(k0 + u) * ostride;
      if constexpr (V == 2) {
        const u32x2 x = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(ro, off, 0, 0));
        o[u][0] = __uint_as_float(x[0]);
        o[u][1] = __uint_as_float(x[1]);
      } else {
        o[u][0] = buf_load_f32(ro, off);
      }
    }
    if (nparts <= kFast) {
      mmax = ml.x;
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) mmax = wave_max_xor(mmax, m);
    }
    const float w = lane < n ? fast_exp2(ml.x - mmax) : 0.0f;
    lsum += w * ml.y;
#pragma unroll
    for (int u = 0; u < kFast; ++u) {
      const float wu = __shfl(w, u, 64);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += wu * o[u][i];
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) lsum = wave_sum_xor(lsum, m);
  const float inv = 1.0f / lsum;
  uint16_t *op = p.out + (q_row_of(p, seq) * p.q_heads + h) * D + dim0 + lane * V;
  if constexpr (V == 1) {
    op[0] = uint16_t(f32_to_bf16_bits(acc[0] * inv));
  } else {
    *reinterpret_cast<uint32_t *>(op) = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  }
}

// Merge launch: one wave per (sequence, head); only sequences split over more
// than one partition have partials. (An in-kernel merge was measured slower:
// partials written on other XCDs are only visible through an L2 writeback or
// uncached accesses, both costlier than this launch.)
template <int D>
__global__ __launch_bounds__(256) void split_k_merge_kernel(DecodeParams p) {
  constexpr int DW = D < 128 ? D : 128;  // dims per wave
  const int seq = blockIdx.x, h = blockIdx.y;
  if (!decode_seq(p, seq)) return;
  const int nparts = parts_of(clamp_len(p, seq), p.part_tokens);
  if (nparts <= 1) return;
  merge_head<D, DW>(p, seq, h, nparts, (threadIdx.x >> 6) * DW, threadIdx.x & 63);
}

// One workgroup per (sequence, head); one wave per 128 output dims.
template <int D>
inline void launch_merge(const DecodeParams &p, hipStream_t s) {
  if (p.max_parts <= 1) return;
  constexpr int waves = D > 128 ? D / 128 : 1;
  split_k_merge_kernel<D><<<dim3(p.num_seqs, p.q_heads), 64 * waves, 0, s>>>(p);
}

constexpr uint64_t kQueueBytes = 64;

// Tokens per split-K partition (a multiple of the 32-token tile): 2048 for
// bf16 caches, 1536 for C8 caches. The longest-first list ends with the
// partial partitions filling the workgroups' tails, and how well they fit
// depends on the partition size: C8 over 256 sequences of U[1024, 16384]
// tokens measured 234 us at 1536 against 253 us at 1024, 2048, 3072 and 4096;
// bf16 over log-uniform [128, 32768] measured 2048 and 1792 alike, 1216 and
// 2560 slower. The IFATTN_DECODE_PART_TOKENS environment variable overrides
// both for tuning.
inline int part_tokens(bool c8 = false) {
  static int v = [] {
    const char *e = getenv("IFATTN_DECODE_PART_TOKENS");
    int x = e ? atoi(e) : 0;
    return (x >= 32 && x <= 8192 && x % 32 == 0) ? x : 0;
  }();
  return v ? v : (c8 ? 1536 : 2048);
}

inline int max_parts_for(int max_context, bool c8 = false) {
  return (max_context + part_tokens(c8) - 1) / part_tokens(c8);
}
// Partition count the workspace is sized for (either cache type).
inline int max_parts_any(int max_context) {
  const int a = max_parts_for(max_context, false), b = max_parts_for(max_context, true);
  return a > b ? a : b;
}

inline uint64_t align16(uint64_t x) { return (x + 15) & ~uint64_t(15); }

// Compute units of the current device (cached per device).
inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Persistent workgroups per CU. Fewer concurrent row streams keep HBM pages
// open longer; IFATTN_DECODE_WGS_PER_CU overrides the default for tuning.
inline int wgs_per_cu() {
  static int v = [] {
    const char *e = getenv("IFATTN_DECODE_WGS_PER_CU");
    int x = e ? atoi(e) : 0;
    return (x >= 1 && x <= 16) ? x : 2;
  }();
  return v;
}


// Workspace layout: queue words | items | partial O | partial (m, l).
inline uint64_t split_k_workspace_bytes(int num_seqs, int heads, int dims, int max_context) {
  const uint64_t items = uint64_t(num_seqs) * uint64_t(max_parts_any(max_context));
  const uint64_t partials = items > uint64_t(num_seqs)  // single-partition calls keep no partials
                                ? items * heads * (uint64_t(dims) + 2) * sizeof(float)
                                : 0;
  return kQueueBytes + align16(items * 4) + partials;
}
inline void split_k_bind_workspace(DecodeParams &p, void *workspace, int heads, int dims) {
  uint8_t *w = static_cast<uint8_t *>(workspace);
  const uint64_t items = uint64_t(p.num_seqs) * p.max_parts;
  p.queue = reinterpret_cast<int32_t *>(w);
  w += kQueueBytes;
  p.items = reinterpret_cast<uint32_t *>(w);
  w += align16(items * 4);
  p.part_o = reinterpret_cast<float *>(w);
  p.part_ml = p.part_o + items * heads * dims;
}

// Prologue launch: planning workgroup plus enough writer workgroups for `wr`.
inline void launch_prologue(const DecodeParams &p, const RowWrite &wr, hipStream_t s) {
  const int64_t vecs = wr.rows * wr.row_vecs * (wr.v_rows ? 2 : 1);
  const int64_t writers = vecs > 0 ? (vecs + 1023) / 1024 : 0;
  const int grid = 1 + int(writers < 1024 ? writers : 1024);
  decode_prologue_kernel<><<<grid, 1024, 0, s>>>(p, wr);
}

// Launches plan + decode + merge for the single-row sequences of a packed
// varlen batch (defined with the GQA decode kernels).
void launch_varlen_decode_rows(const DecodeParams &p, int head_dim, hipStream_t s);

}  // namespace ifattn
