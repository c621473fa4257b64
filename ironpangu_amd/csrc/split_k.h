// Split-K scheduling of the paged GQA decode, and pieces shared with the MLA
// and prefill planners. The decode splits the call's work into
// contiguous shares: every decode sequence weighs its tokens plus a fixed
// start cost, the prologue kernel prefix-sums the weights on the device and
// cuts the total into `workers` shares of `share` units (one per persistent
// workgroup, fewer for small calls), and the workgroups walk their shares tile
// by tile (bf16 calls give odd workers, on odd XCDs, slightly smaller shares:
// see decode_skew_pm). A sequence lying in one share writes its output
// directly; one spread over several shares writes an (m, l, O) partial per
// share into consecutive slots, which a merge launch combines. No work queue,
// no atomics. The prologue kernel also
// performs the step's slot-mapped row writes, so a decode step is prologue ->
// decode -> merge from one host call. Calls of up to kSelfPlanPerThread
// sequences per decode thread plan inside the decode workgroups instead (the
// same arithmetic), and the prologue then launches only for row writes.
#pragma once
#include <cstdlib>

#include "common.h"

namespace ifattn {

// Tokens per unit of the split: shares end on 32-token tile boundaries.
constexpr int kSplitTile = 32;

struct DecodeParams {
  const uint16_t *q;
  const uint8_t *k_cache;
  const uint8_t *v_cache;
  const float *k_scale;
  const float *v_scale;
  const int32_t *block_tables;
  const int32_t *seq_lens;
  uint16_t *out;
  // Written by the prologue: plan[0] = workers, plan[2..3] = share (int64
  // units per worker).
  int32_t *plan;
  int64_t *seq_pos;    // [num_seqs] first work unit of each sequence
  int2 *seq_slot;      // [num_seqs] (first partial slot, slot count) of a sequence over several
                       // shares, (-1, 0) otherwise
  int32_t *start_seq;  // [grid] first sequence not wholly before each worker's share
  float *part_o;       // [2 * grid, q_heads, D]
  float *part_ml;      // [2 * grid, q_heads, 2]
  // Packed varlen batches: when set, sequence s reads/writes q/out row
  // cu_seqlens[s+1]-1 and only sequences with exactly one query row are
  // scheduled here (longer chunks go to the prefill kernel).
  const int32_t *cu_seqlens;
  int64_t num_blocks;
  int num_seqs, q_heads, kv_heads, group, table_stride, block_size, max_context, head_dim;
  int seq_cost;      // work units charged per sequence on top of its tokens
  int grid;          // persistent decode workgroups (the most workers)
  int self_plan;     // the decode workgroups plan the call themselves (prologue: row writes only)
  int skew_pm;       // share skew d = S * skew_pm / 1000 (see Shares)
  float scale_log2;  // softmax scale * log2(e)
};

__device__ __forceinline__ int clamp_len(const DecodeParams &p, int seq) {
  const int len = ld_const(p.seq_lens + seq);
  return len > p.max_context ? p.max_context : len;
}
// q / out row of a sequence (identity for plain decode batches).
__device__ __forceinline__ int64_t q_row_of(const DecodeParams &p, int seq) {
  return p.cu_seqlens ? int64_t(ld_const(p.cu_seqlens + seq + 1)) - 1 : int64_t(seq);
}
__device__ __forceinline__ bool decode_seq(const DecodeParams &p, int seq) {
  return !p.cu_seqlens || ld_const(p.cu_seqlens + seq + 1) - ld_const(p.cu_seqlens + seq) == 1;
}
__device__ __forceinline__ int64_t share_of(const DecodeParams &p) {
  return ld_const(reinterpret_cast<const int64_t *>(p.plan + 2));
}
// Contiguous shares of S units, worker pairs (2i, 2i + 1) splitting 2S units
// as S + d and S - d: worker v starts at unit v S + (v odd ? d : 0). With
// 0 <= d < S the n = ceil(total / S) workers cover every unit: lo(n) is n S
// (n even) or n S + d (n odd), both >= total.
struct Shares {
  int64_t S, d;
  __device__ int64_t lo(int v) const { return int64_t(v) * S + ((v & 1) ? d : 0); }
  __device__ int worker(int64_t u) const {  // the worker whose share holds unit u
    const int64_t pair = u / (2 * S);
    return int(2 * pair + (u - 2 * S * pair >= S + d ? 1 : 0));
  }
};
__device__ __forceinline__ Shares make_shares(const DecodeParams &p, int64_t share) {
  return Shares{share, share * p.skew_pm / 1000};
}
// Workers holding the first and the last tile of a sequence whose tile 0 sits
// at work unit `first` (tile j at first + 32 j).
__device__ __forceinline__ void seq_workers(int64_t first, int len, const Shares &sh, int &wa, int &wb) {
  const int tiles = (len + kSplitTile - 1) / kSplitTile;
  wa = sh.worker(first);
  wb = sh.worker(first + int64_t(kSplitTile) * (tiles - 1));
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

// Smallest share the plan cuts (units): tiny calls use fewer workers instead of
// spreading every sequence over many one-tile shares.
constexpr int64_t kMinShareUnits = 512;

// Workgroup-wide inclusive scan (sum or max) of one value per thread, 1024
// threads: shuffles within the wave, wave totals through LDS. Returns the
// inclusive value; *total gets the workgroup's total.
template <typename T, bool MAX>
__device__ __forceinline__ T block_scan(T x, T *wave_tot, T *total) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T y = __shfl_up(x, off, 64);
    if (lane >= off) x = MAX ? (y > x ? y : x) : x + y;
  }
  if (lane == 63) wave_tot[wv] = x;
  __syncthreads();
  T before = MAX ? T(-1) : T(0), all = MAX ? T(-1) : T(0);
  for (int w = 0; w < 16; ++w) {
    const T t = wave_tot[w];
    if (w < wv) before = MAX ? (t > before ? t : before) : before + t;
    all = MAX ? (t > all ? t : all) : all + t;
  }
  __syncthreads();  // wave_tot is reused by the next scan
  *total = all;
  return MAX ? (before > x ? before : x) : before + x;
}

// Workgroup 0 plans the split; workgroups 1.. perform the row writes (if any).
// Pass 1: weights (tokens + seq_cost for a decode sequence with keys, 0
// otherwise) -> seq_pos by an exclusive scan; sequences without a visible key
// get their defined zero output here. Then workers = grid, fewer for small
// calls (at least kMinShareUnits per worker), and share = ceil(total /
// workers). Pass 2: a
// sequence whose first and last tiles fall in different shares gets
// consecutive partial slots (one per share it touches); start_seq[v] = the
// first sequence whose last tile lies in share v or later.
template <int Unused = 0>
__global__ __launch_bounds__(1024) void decode_prologue_kernel(DecodeParams p, RowWrite wr) {
  if (blockIdx.x > 0) {
    prologue_write(wr);
    return;
  }
  if (p.self_plan) return;  // the decode workgroups plan for themselves
  __shared__ long long s_tot64[16];
  __shared__ int s_tot32[16];
  __shared__ long long s_pos, s_share;
  __shared__ int s_slot, s_emax, s_workers;
  __shared__ int s_incl[1024];
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_pos = 0;
    s_slot = 0;
    s_emax = -1;
  }
  __syncthreads();
  for (int base = 0; base < p.num_seqs; base += 1024) {
    const int seq = base + tid;
    const bool dec = seq < p.num_seqs && decode_seq(p, seq);
    const int len = dec ? clamp_len(p, seq) : 0;
    if (dec && len <= 0) {  // no visible key: defined zero output
      uint16_t *o = p.out + q_row_of(p, seq) * p.q_heads * p.head_dim;
      for (int i = 0; i < p.q_heads * p.head_dim; i += 8) store_u32x4(o + i, u32x4{0, 0, 0, 0});
    }
    const long long w = len > 0 ? (long long)len + p.seq_cost : 0;
    long long tot;
    const long long incl = block_scan<long long, false>(w, s_tot64, &tot);
    if (seq < p.num_seqs) p.seq_pos[seq] = s_pos + incl - w;
    __syncthreads();
    if (tid == 0) s_pos += tot;
    __syncthreads();
  }
  if (tid == 0) {
    const long long total = s_pos;
    const long long small = (total + kMinShareUnits - 1) / kMinShareUnits;
    long long workers = small < p.grid ? small : p.grid;
    workers = workers < 1 ? 1 : workers;
    const long long share = total > 0 ? (total + workers - 1) / workers : 1;
    s_workers = int(workers);
    s_share = share;
    p.plan[0] = int(workers);
    *reinterpret_cast<int64_t *>(p.plan + 2) = share;
  }
  __syncthreads();
  const long long share = s_share;
  for (int base = 0; base < p.num_seqs; base += 1024) {
    const int seq = base + tid;
    const bool dec = seq < p.num_seqs && decode_seq(p, seq);
    const int len = dec ? clamp_len(p, seq) : 0;
    int cnt = 0, e = -1;
    if (len > 0) {
      int wa, wb;
      seq_workers(p.seq_pos[seq] + p.seq_cost, len, make_shares(p, share), wa, wb);
      cnt = wb > wa ? wb - wa + 1 : 0;
      e = wb;
    }
    int tot;
    const int incl = block_scan<int, false>(cnt, s_tot32, &tot);
    if (seq < p.num_seqs) p.seq_slot[seq] = make_int2(cnt > 0 ? s_slot + incl - cnt : -1, cnt);
    int emax;
    s_incl[tid] = block_scan<int, true>(e, s_tot32, &emax);
    __syncthreads();
    // Largest last-tile worker of the sequences before this one.
    int prev = tid > 0 ? s_incl[tid - 1] : -1;
    prev = prev > s_emax ? prev : s_emax;
    for (int v = prev + 1; v <= e; ++v) p.start_seq[v] = seq;
    __syncthreads();
    if (tid == 0) {
      s_slot += tot;
      s_emax = emax > s_emax ? emax : s_emax;
    }
    __syncthreads();
  }
  for (int v = s_emax + 1 + tid; v < s_workers; v += 1024) p.start_seq[v] = p.num_seqs;
}

// Merge the split-K partials of one (sequence, head) over the dims
// [dim0, dim0 + DW) with one wave; lane l owns DW/64 consecutive dims. Up to
// kFast partitions go in one round trip: lane k holds partition k's (m, l) and
// every partial-O slice is loaded before any is used; the weights reach the
// other lanes by shuffle. Longer lists are taken kFast at a time.
template <int D, int DW>
__device__ __forceinline__ void merge_head(const DecodeParams &p, int seq, int h, int slot0,
                                           int nparts, int dim0, int lane) {
  constexpr int V = DW / 64;
  constexpr int kFast = 16;
  // This sequence's partials: share k (slot slot0 + k), head h is row
  // k * q_heads + h. Buffer offsets stay 32-bit and rows past nparts read as zero.
  const int64_t seq_row = int64_t(slot0) * p.q_heads;
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
  const int2 slots = make_int2(ld_const(&p.seq_slot[seq].x), ld_const(&p.seq_slot[seq].y));
  if (slots.x < 0) return;  // the sequence lies in one share: output written by the decode
  merge_head<D, DW>(p, seq, h, slots.x, slots.y, (threadIdx.x >> 6) * DW, threadIdx.x & 63);
}

// One workgroup per (sequence, head); one wave per 128 output dims.
template <int D>
inline void launch_merge(const DecodeParams &p, hipStream_t s) {
  constexpr int waves = D > 128 ? D / 128 : 1;
  split_k_merge_kernel<D><<<dim3(p.num_seqs, p.q_heads), 64 * waves, 0, s>>>(p);
}

constexpr uint64_t kQueueBytes = 64;

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

// Work units charged per sequence on top of its tokens: the item start of a
// decode workgroup (q and block-id loads, the first tiles' latency) costs about
// as much as streaming this many tokens: 64 for bf16 caches, 192 for C8, whose
// tokens stream twice as fast (config 4: 0.2080 -> 0.2050 ms; 128: 0.2055,
// 256: 0.2061). IFATTN_DECODE_SEQ_COST overrides both.
inline int decode_seq_cost(bool c8 = false) {
  static int v = [] {
    const char *e = getenv("IFATTN_DECODE_SEQ_COST");
    const int x = e ? atoi(e) : -1;
    return (x >= 0 && x <= 65536) ? x : -1;
  }();
  return v >= 0 ? v : (c8 ? 192 : 64);
}
// Share skew (permille) of bf16 decode at head_dim <= 128: workgroups are
// dispatched round-robin over the 8 XCDs, so odd workers run on odd XCDs,
// whose tiles measured 4-8% slower; giving odd workers 3% fewer units ends the
// shares closer together (config-2 step 0.2987 -> 0.2956 ms, 16-token pages
// 1% faster; 1.5% and 4.5% gained less, the opposite skew lost). Head_dim 256
// (1.8% slower with the skew) and C8 (no gain) keep equal shares.
// IFATTN_DECODE_XCD_SKEW (0..200) overrides every variant.
inline int decode_skew_pm(bool c8, int head_dim) {
  static const int v = [] {
    const char *e = getenv("IFATTN_DECODE_XCD_SKEW");
    const int x = e ? atoi(e) : 1000;
    return (x >= 0 && x <= 200) ? x : 1000;
  }();
  return v != 1000 ? v : (c8 || head_dim > 128 ? 0 : 30);
}
inline int decode_grid() { return device_cus() * wgs_per_cu(); }

// Workspace layout: plan words | seq_pos | seq_slot | start_seq | partial O |
// partial (m, l); a sequence over k shares uses k slots, at most 2 per worker.
inline uint64_t split_k_workspace_bytes(int num_seqs, int heads, int dims, int /*max_context*/) {
  const uint64_t workers = uint64_t(decode_grid());
  return kQueueBytes + align16(uint64_t(num_seqs) * 8) + align16(uint64_t(num_seqs) * 8) +
         align16(workers * 4) + 2 * workers * heads * (uint64_t(dims) + 2) * sizeof(float);
}
// Fills the split fields of p (num_seqs set) and binds the workspace.
inline void split_k_bind_workspace(DecodeParams &p, void *workspace, int heads, int dims) {
  p.seq_cost = decode_seq_cost();
  p.grid = decode_grid();
  p.head_dim = dims;
  uint8_t *w = static_cast<uint8_t *>(workspace);
  p.plan = reinterpret_cast<int32_t *>(w);
  w += kQueueBytes;
  p.seq_pos = reinterpret_cast<int64_t *>(w);
  w += align16(uint64_t(p.num_seqs) * 8);
  p.seq_slot = reinterpret_cast<int2 *>(w);
  w += align16(uint64_t(p.num_seqs) * 8);
  p.start_seq = reinterpret_cast<int32_t *>(w);
  w += align16(uint64_t(p.grid) * 4);
  p.part_o = reinterpret_cast<float *>(w);
  p.part_ml = p.part_o + uint64_t(2 * p.grid) * heads * dims;
}

// Prologue launch: planning workgroup plus enough writer workgroups for `wr`
// (none at all for a self-planned call without rows to write).
inline void launch_prologue(const DecodeParams &p, const RowWrite &wr, hipStream_t s) {
  const int64_t vecs = wr.rows * wr.row_vecs * (wr.v_rows ? 2 : 1);
  const int64_t writers = vecs > 0 ? (vecs + 1023) / 1024 : 0;
  if (p.self_plan && writers == 0) return;
  const int grid = 1 + int(writers < 1024 ? writers : 1024);
  decode_prologue_kernel<><<<grid, 1024, 0, s>>>(p, wr);
}

// Self-planned decode calls: at most kSelfPlanPerThread sequences per thread
// of a decode workgroup.
constexpr int kSelfPlanPerThread = 4;
constexpr int kSelfPlanMaxSeqs = kSelfPlanPerThread * 256;
// Host check: may a call of num_seqs sequences on workgroups of `threads`
// threads plan inside the decode kernel (every prefix of units in 32 bits,
// partial slots and workers below 2^16)?
inline bool decode_self_plan(const DecodeParams &p, int threads) {
  return p.num_seqs <= kSelfPlanPerThread * threads &&
         int64_t(p.num_seqs) * (int64_t(p.max_context) + p.seq_cost) < (int64_t(1) << 31) &&
         2 * p.grid < 0xFFFF;
}

// Launches plan + decode + merge for the single-row sequences of a packed
// varlen batch (defined with the GQA decode kernels).
void launch_varlen_decode_rows(const DecodeParams &p, int head_dim, hipStream_t s);

}  // namespace ifattn
