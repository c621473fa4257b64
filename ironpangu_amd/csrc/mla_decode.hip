// Packed-MLA latent-cache attention for gfx950 (bf16 rows, packed C8 rows and
// row-quantized int8 / int4 rows).
//
// For each query row r and head h (all heads share one cache row per key):
//   s_j = scale * q[r,h,0:576] . key_j[0:576]
//   out[r,h] = sum_j softmax(s)_j * key_j[0:512]
// over the row's keys plus optional learned sink rows, fp32 accumulation. This
// is the latent attention of the reference's MLA decoder
// (native/src/token_executor.h:841-906): the BF16 window attention with sinks
// whose CPU oracle is native/probes/sliding_window_probe.cpp:144-163, and the
// packed C8 sparse attention with sinks whose CPU oracle is
// native/probes/packed_cache_probe.cpp:47-66. C8 rows are {int8 latent[512],
// bf16 rope[64], f32 scale[4]} (docs/packed-mla-cache.md:27-43); latent d
// dequantizes as int8 * scale[d/128] (packed_cache_probe.cpp:57).
//
// Keys of a row: rows are packed per sequence (cu_seqlens_q; one row per
// sequence in plain decode). Row t of a sequence with `count` rows and kv_len
// cached keys sees causal = kv_len - count + t + 1 keys
// (openpangu_attention_metadata.h:20-22). Dense rows read positions
// [max(0, causal - window), causal) through the block table (window 0 = all);
// sparse rows read the logical positions of their index list
// (min(causal, topk) candidates, -1 padding; openpangu_attention_metadata.h:13-33).
//
// Decomposition: the plan (a plan launch, or for calls of at most 256 rows
// every attention workgroup itself) cuts the call's work (rows weighted by
// their key tiles, a start cost and their sink block) into contiguous shares,
// one per persistent workgroup of four waves (equal, or weighted by the
// workgroup's dispatch order on the CU), which walks its share row by row. A share's 32-token tiles are copied HBM -> LDS once by direct-to-LDS
// loads (dense: 32 consecutive rows of one
// block; sparse: a gather of 32 rows named by the index list) through a ring
// of slots; wave w then owns latent dims [128w, 128w+128) for QK^T and PV (K
// and V are the same bytes) and waves 0 and 1 one 32-dim step of the rope part.
// Partial score tiles are summed across the waves through LDS, every wave runs
// the same online softmax. With C8 the wave's 128 dims are exactly one scale
// tile, so the per-token tile scale multiplies the wave's partial score and is
// folded into its probabilities for PV. MFMA 16x16x32 bf16 with the heads in
// the N dimension; C8 latent scores use the fp16 MFMA on the codes biased by
// 1152 (three VALU ops per four codes instead of a convert per code), with q
// in fp16 and the bias term removed per head. Row-quantized rows (576 int8 or
// int4 codes and one fp32 scale per row, as if_cache_quantize writes them,
// native/kernels/cache_quantization.cpp:12-38) are gathered row by row with
// their scales staged behind the tile; keys are dequantized in registers to
// the bf16 values if_cache_dequantize would write (the reference attends over
// that dequantized cache, token_executor.h:806-822), V stays in codes with the
// row scale folded into the probabilities. Rows split over several
// shares, and rows with sinks, write (m, l, O) partials; a merge kernel
// combines them with the sink partial. How many workgroups share a CU depends
// on the variant (MlaCfg).
#include <array>

#include "common.h"
#include "ifattn_internal.h"
#include "mla_row_write.h"
#include "split_k.h"

namespace ifattn {

constexpr int kMlaWaves = 4;
constexpr int kMlaSlotsMax = 3;  // most workgroups of one variant per CU
constexpr int kMlaTile = 32;
constexpr int kSparsePart = 1024;  // index-list entries per sparse partition

constexpr int kMaxSinks = 128;

struct MlaParams {
  const uint16_t *q;            // [rows, heads, 576]
  const uint8_t *cache;         // key rows of 1152 (bf16), 656 (C8), 576 (Rq8) or 288 (Rq4) bytes
  const float *row_scales;      // [cache rows] fp32 scales of row-quantized rows
  const int32_t *block_tables;  // [seqs, table_stride]
  const int32_t *kv_lens;       // [seqs] cached keys after this step's writes
  const int32_t *cu_q;          // [seqs + 1] query rows per sequence; null: one row each
  const int32_t *indices;       // [rows, topk] logical key positions (-1 pads); null: dense
  const uint16_t *sink_k;       // [n_sinks, 576] bf16 or null
  const uint16_t *sink_v;       // [n_sinks, 512] bf16
  uint16_t *out;                // [rows, heads, 512]
  // Plan outputs: plan[0] = workers, plan[2..3] = total work units (int64).
  int32_t *plan;
  int64_t *row_pos;             // [rows] first work unit of each row
  int32_t *row_seq;             // [rows] sequence of each row
  int2 *row_slot;               // [rows] (first partial slot, slot count); (-1, 0): the row
                                // writes its output directly
  int32_t *start_row;           // [max_workers] first row not wholly before each worker's share
  uint16_t *part_o;             // [slots, heads, 512] bf16 O / l of each partial
  float *part_ml;               // [slots, heads, 2]
  int64_t num_blocks;
  uint32_t cache_bytes;  // sparse and row-quantized gathers: byte extent of the cache (< 4 GiB - 16)
  uint32_t scale_bytes;  // row-quantized rows: byte extent of row_scales
  int num_seqs, num_rows, heads, table_stride, block_size, max_context, topk, window, n_sinks;
  int row_cost;     // work units charged per row start
  int sink_units;   // work units of a row's sink block (0 without sinks)
  int max_share;    // largest share: sparse segments fit the kSparsePart slot list
  int skew_pm;      // share skew between odd and even workers (MlaShares), permille
  int slot_n;       // dispatch slots with their own share weight (MlaShares), 1: equal shares
  int slot_c;       // workers per dispatch slot (the CUs)
  int slot_w[kMlaSlotsMax];  // share weight of each dispatch slot, permille
  int max_workers;  // workers the workspace holds
  int grid;         // persistent attention workgroups
  int self_plan;    // the attention workgroups plan the call themselves (no plan launch)
  float scale_log2;
};

// Fused decode step (ifattn_mla_decode_step): the step's new latent rows x
// [rows, 576] bf16, normalized and roped into the cache at each sequence's last
// position by the workgroup that reads that position. A kernel argument of its
// own: in MlaParams it cost the plain C8 kernel two spilled registers.
struct MlaStep {
  const uint16_t *x, *gamma, *cos, *sin;
  uint8_t *cache;
  float eps;
};

// Keys of one row: [lo, hi) are positions (dense) or index-list slots
// (sparse); partitions of the row's partition size start at `base` (lo rounded down to a
// tile), so every tile is 32-aligned and never straddles a block.
struct MlaSpan {
  int seq, lo, hi, base;
};

__device__ __forceinline__ int mla_seq_of(const MlaParams &p, int row) {
  if (!p.cu_q) return row;
  int a = 0, b = p.num_seqs - 1;  // last sequence whose first row is <= row
  while (a < b) {
    const int m = (a + b + 1) >> 1;
    if (ld_const(p.cu_q + m) <= row) a = m; else b = m - 1;
  }
  return a;
}

__device__ __forceinline__ MlaSpan mla_span(const MlaParams &p, int row, int seq) {
  const int start = p.cu_q ? ld_const(p.cu_q + seq) : row;
  const int count = p.cu_q ? ld_const(p.cu_q + seq + 1) - start : 1;
  int kv = ld_const(p.kv_lens + seq);
  kv = kv > p.max_context ? p.max_context : kv;
  int causal = kv - count + (row - start) + 1;
  causal = causal < 0 ? 0 : (causal > p.max_context ? p.max_context : causal);
  MlaSpan s;
  s.seq = seq;
  if (p.indices) {
    s.lo = 0;
    s.hi = causal < p.topk ? causal : p.topk;
    s.base = 0;
  } else {
    s.hi = causal;
    s.lo = (p.window > 0 && causal > p.window) ? causal - p.window : 0;
    s.base = s.lo & ~(kMlaTile - 1);
  }
  return s;
}
// Tiles of a row's keys (32-key tiles from `base`).
__device__ __forceinline__ int mla_tiles(const MlaSpan &s) {
  return s.hi > s.lo ? (s.hi - s.base + kMlaTile - 1) / kMlaTile : 0;
}
// Work of row r in units: [row_pos, + sink_units) is its sink block (one
// event, see mla_sink_mid), then row_cost units of start, then its tiles, tile
// j at unit first = row_pos + sink_units + row_cost + 32 j.
struct MlaRowWork {
  int tiles, wa, wb;  // tiles; workers of the first and last tile
  int64_t first;      // unit of tile 0
  int slots;          // partial slots: 1 for the sinks, then one per share the tiles touch
};
// Contiguous shares of a call's work units, one per worker, in worker order.
// Worker v runs on workgroup v % grid; workgroups [k C, (k + 1) C) are the
// k-th workgroup dispatched to each CU (dispatch slot k). Co-resident
// workgroups do not progress at the same rate: the older waves of a CU win
// instruction issue, so on the VALU-bound integer tiles a CU's first
// workgroup ran 2.1, its second 2.5 and its third 3.0 us per tile (C8
// config-5 rows, three per CU), and equal shares ended a third of the way
// apart. When the workers fill the slots exactly, the workers of slot k get
// shares in proportion to its weight; otherwise all shares are equal. Within a
// slot, odd workers (odd XCDs) are d = s * skew_pm / 1000 units shorter than
// even ones. The slots' shares live in a small LDS table (kMlaShareTab
// int64s, written by one thread): kept in registers they pushed the dense C8
// kernel's scalar registers into spills.
constexpr int kMlaShareTab = 2 * kMlaSlotsMax + 3;  // s[3], b[4], c, ns
__device__ __forceinline__ void mla_shares_fill(const MlaParams &p, int64_t total, int workers,
                                                int64_t *tab) {
  if (p.slot_n > 1 && workers == p.slot_n * p.slot_c) {
    int wsum = 0;
    for (int k = 0; k < p.slot_n; ++k) wsum += p.slot_w[k];
    const int64_t den = int64_t(p.slot_c) * wsum;
    int64_t b = 0;
    bool fits = true;  // sparse shares must fit the slot list
    for (int k = 0; k < p.slot_n; ++k) {
      const int64_t sk = (total * p.slot_w[k] + den - 1) / den;
      tab[k] = sk < 1 ? 1 : sk;
      fits = fits && tab[k] <= p.max_share;
      tab[kMlaSlotsMax + k] = b;
      b += int64_t(p.slot_c) * tab[k];
    }
    if (fits) {
      tab[kMlaSlotsMax + p.slot_n] = b;
      tab[2 * kMlaSlotsMax + 1] = p.slot_c;
      tab[2 * kMlaSlotsMax + 2] = p.slot_n;
      return;
    }
  }
  tab[0] = total > 0 ? (total + workers - 1) / workers : 1;
  tab[kMlaSlotsMax] = 0;
  tab[2 * kMlaSlotsMax + 1] = workers + 1;  // one slot: lo(workers) ends the last share
  tab[2 * kMlaSlotsMax + 2] = 1;
}
// TAB false: equal shares of s0 units without the table (the wide variant,
// whose LDS is full; the host gives it no weights).
template <bool TAB = true>
struct MlaShares {
  const int64_t *tab;
  int64_t s0;
  int skew_pm;
  __device__ int64_t lo(int v) const {
    if (!TAB) return int64_t(v) * s0 + ((v & 1) ? s0 * skew_pm / 1000 : 0);
    const int c = int(tab[2 * kMlaSlotsMax + 1]);
    const int k = v / c, i = v - k * c;
    const int64_t s = tab[k];
    return tab[kMlaSlotsMax + k] + int64_t(i) * s + ((i & 1) ? s * skew_pm / 1000 : 0);
  }
  __device__ int worker(int64_t u) const {  // the worker whose share holds unit u
    int k = 0, c = 0;
    int64_t s = s0, b = 0;
    if (TAB) {
      const int ns = int(tab[2 * kMlaSlotsMax + 2]);
      for (int t = 1; t < ns; ++t)
        if (u >= tab[kMlaSlotsMax + t]) k = t;
      s = tab[k];
      b = tab[kMlaSlotsMax + k];
      c = int(tab[2 * kMlaSlotsMax + 1]);
    }
    const int64_t d = s * skew_pm / 1000, q = u - b, pair = q / (2 * s);
    return k * c + int(2 * pair + (q - 2 * s * pair >= s + d ? 1 : 0));
  }
};
// The sink block is one event, run by the worker whose share holds its middle
// unit: a share boundary inside the block then moves at most half of its cost
// to the neighbouring share. (Run at its first unit, a row start a few units
// before a boundary put the whole block, about six tiles of time, on the
// worker before it: window-2048 calls ended 8 us later on odd workers.)
__device__ __forceinline__ int64_t mla_sink_mid(const MlaParams &p, int64_t pos) {
  return pos + p.sink_units / 2;
}
template <bool TAB>
__device__ __forceinline__ MlaRowWork mla_row_work(const MlaParams &p, const MlaSpan &sp, int64_t pos,
                                                   const MlaShares<TAB> &sh) {
  MlaRowWork r;
  r.tiles = mla_tiles(sp);
  r.first = pos + p.sink_units + p.row_cost;
  r.wa = r.wb = 0;
  const int sinks = p.n_sinks > 0 ? 1 : 0;
  r.slots = sinks;
  if (r.tiles > 0) {
    r.wa = sh.worker(r.first);
    r.wb = sh.worker(r.first + int64_t(kMlaTile) * (r.tiles - 1));
    if (sinks || r.wb > r.wa) r.slots += r.wb - r.wa + 1;
  }
  return r;
}

// Work units of a row (0: no keys and no sinks).
__device__ __forceinline__ int64_t mla_row_weight(const MlaParams &p, const MlaSpan &sp) {
  const int tiles = mla_tiles(sp);
  return (tiles > 0 ? int64_t(p.row_cost) + int64_t(kMlaTile) * tiles : 0) + p.sink_units;
}
// Workers of a call of `total` units: the grid, fewer for small calls (at
// least kMinShareUnits each), more for sparse calls whose shares must fit the
// slot list, at most the workspace's max_workers.
__device__ __forceinline__ int mla_split(const MlaParams &p, int64_t total) {
  const int64_t small = (total + kMinShareUnits - 1) / kMinShareUnits;
  int64_t wk = small < p.grid ? small : p.grid;
  const int64_t bound = (total + p.max_share - 1) / p.max_share;  // sparse share cap
  wk = bound > wk ? bound : wk;
  wk = wk < 1 ? 1 : (wk > p.max_workers ? p.max_workers : wk);
  return int(wk);
}

// Work split on the device (graph-safe: lengths are read at run time), the
// same scheme as the GQA decode's: every row weighs its key tiles plus a start
// cost (plus its sink block); an exclusive scan gives each row's first unit,
// and the total is cut into `workers` equal contiguous shares, one per
// persistent workgroup (fewer for small calls; more, in rounds, when sparse
// shares must stay within the kSparsePart slot list). A workgroup walks its
// shares row by row; a row whose tiles lie in one share and that has no sinks
// writes its output directly, others write one (m, l, O) partial per share
// (and one for the sinks) into consecutive slots, combined by the merge.
// Rows without keys or sinks get their zero output here. (The former
// longest-first queue of fixed partitions left a quarter of the workgroups'
// time idle at the end of a config-5 call.) One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void mla_plan_kernel(MlaParams p) {
  __shared__ long long s_tot64[16];
  __shared__ int s_tot32[16];
  __shared__ long long s_pos;
  __shared__ int64_t s_tab[kMlaShareTab];
  __shared__ int s_slot, s_emax, s_workers;
  __shared__ int s_incl[1024];
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_pos = 0;
    s_slot = 0;
    s_emax = -1;
  }
  __syncthreads();
  // The first chunk's spans stay in registers for pass 2 (calls with more than
  // 1024 rows reload the others).
  MlaSpan first_span{0, 0, 0, 0};
  int64_t first_pos = 0;
  for (int base = 0; base < p.num_rows; base += 1024) {
    const int row = base + tid;
    long long w = 0;
    if (row < p.num_rows) {
      const int seq = mla_seq_of(p, row);
      p.row_seq[row] = seq;
      const MlaSpan sp = mla_span(p, row, seq);
      if (base == 0) first_span = sp;
      w = mla_row_weight(p, sp);
      if (w == 0) {  // no keys and no sinks: defined zero output
        uint16_t *o = p.out + int64_t(row) * p.heads * 512;
        for (int i = 0; i < p.heads * 512; i += 8) store_u32x4(o + i, u32x4{0, 0, 0, 0});
      }
    }
    long long tot;
    const long long incl = block_scan<long long, false>(w, s_tot64, &tot);
    if (row < p.num_rows) p.row_pos[row] = s_pos + incl - w;
    if (base == 0) first_pos = s_pos + incl - w;
    __syncthreads();
    if (tid == 0) s_pos += tot;
    __syncthreads();
  }
  if (tid == 0) {
    const int workers = mla_split(p, s_pos);
    s_workers = workers;
    p.plan[0] = workers;
    *reinterpret_cast<int64_t *>(p.plan + 2) = s_pos;
    mla_shares_fill(p, s_pos, workers, s_tab);
  }
  __syncthreads();
  const MlaShares<> sh{s_tab, 0, p.skew_pm};
  for (int base = 0; base < p.num_rows; base += 1024) {
    const int row = base + tid;
    int cnt = 0, e = -1;
    if (row < p.num_rows) {
      const int64_t pos = base == 0 ? first_pos : p.row_pos[row];
      const MlaRowWork rw =
          mla_row_work(p, base == 0 ? first_span : mla_span(p, row, p.row_seq[row]), pos, sh);
      cnt = rw.slots;
      // Worker of the row's last event (its last tile, or its sink block).
      if (rw.tiles > 0) e = rw.wb;
      else if (p.sink_units > 0) e = sh.worker(mla_sink_mid(p, pos));
    }
    int tot;
    const int incl = block_scan<int, false>(cnt, s_tot32, &tot);
    if (row < p.num_rows) p.row_slot[row] = make_int2(cnt > 0 ? s_slot + incl - cnt : -1, cnt);
    int emax;
    s_incl[tid] = block_scan<int, true>(e, s_tot32, &emax);
    __syncthreads();
    int prev = tid > 0 ? s_incl[tid - 1] : -1;
    prev = prev > s_emax ? prev : s_emax;
    for (int v = prev + 1; v <= e; ++v) p.start_row[v] = row;
    __syncthreads();
    if (tid == 0) {
      s_slot += tot;
      s_emax = emax > s_emax ? emax : s_emax;
    }
    __syncthreads();
  }
  for (int v = s_emax + 1 + tid; v < s_workers; v += 1024) p.start_row[v] = p.num_rows;
}

// Key-row formats of the cache.
enum MlaFmt : int {
  kFmtBf16 = 0,  // 1152-B rows: bf16[576]
  kFmtC8 = 1,    // 656-B rows: int8 latent[512], bf16 rope[64], f32 scale[4] (one per 128 dims)
  kFmtRq8 = 2,   // 576-B rows: int8[576] with one fp32 scale per row in a separate array
  kFmtRq4 = 3,   // 288-B rows: int4[576] (two's complement, low nibble first), scale as Rq8
};
// Formats whose latent dims are integer codes (scored with the biased fp16 MFMA).
constexpr bool mla_int(int F) { return F != kFmtBf16; }
// Row-quantized formats (if_cache_quantize rows): the rope dims are codes too,
// the scale lives outside the row, and dense tiles are gathered row by row.
constexpr bool mla_rq(int F) { return F == kFmtRq8 || F == kFmtRq4; }

template <int F>
struct MlaRow {
  static constexpr uint32_t BYTES = F == kFmtC8 ? 656 : (F == kFmtRq8 ? 576 : (F == kFmtRq4 ? 288 : 1152));
  static constexpr uint32_t CHUNKS = BYTES / 16;  // 72, 41, 36 or 18
  // Direct-to-LDS loads per wave per tile: 32 rows = 2304 (bf16), 1312 (C8),
  // 1152 (Rq8) or 576 (Rq4) 16-byte chunks.
  static constexpr int NI = F == kFmtC8 ? 6 : (F == kFmtRq8 ? 5 : (F == kFmtRq4 ? 3 : 9));
  static constexpr uint32_t SLOT = 4 * NI * 1024;  // LDS bytes per staged tile
  // LDS byte of 16-byte chunk j of tile row r. bf16 rows (1152 B: odd rows
  // start half a bank period in) XOR the latent chunk index with the row's low
  // 4 bits, which puts the 16 rows of one K read on 16 distinct bank groups;
  // the 8 rope chunks (j >= 64) use the low 3 bits to stay inside the row.
  // Integer rows are not swizzled.
  static __device__ __forceinline__ uint32_t key(uint32_t r, uint32_t j) {
    return j < 64 ? (r & 15) : (r & 7);
  }
  static __device__ __forceinline__ uint32_t chunk(uint32_t r, uint32_t j) {
    return F != kFmtBf16 ? r * BYTES + 16 * j : r * BYTES + 16 * (j ^ key(r, j));
  }
};
static_assert(MlaRow<kFmtBf16>::NI * 4 * 64 == 32 * 72, "bf16 tile = 2304 chunks");
static_assert(18 * 64 == 16 * 72, "bf16 loads 0..17 move exactly tile rows 0..15");
static_assert(MlaRow<kFmtC8>::NI * 4 * 64 >= 32 * 41, "C8 tile fits the slot");
static_assert(MlaRow<kFmtRq8>::NI * 4 * 64 >= 32 * 36 && MlaRow<kFmtRq4>::NI * 4 * 64 >= 32 * 18,
              "row-quantized tiles fit the slot");

// Ring depth and persistent workgroups per CU of each kernel variant. bf16
// runs one workgroup of four waves per CU with a 4-tile ring (its 36-KB tiles
// keep HBM busy while the tile math runs). C8 runs several workgroups per CU
// (two for sparse, three for dense): its 21-KB tiles arrive faster than one
// workgroup's tile math retires them, and the others overlap that math. Measured on
// 128 rows: C8 decode over log-uniform [1024, 65536] keys 582 us with one
// workgroup and 6 stages, 456 us with two and 3 stages; sparse top-2048
// 95.9 us with one workgroup and 6 stages, 75.9 us with two and 2 stages.
template <int F, bool SPARSE, bool WIDE = false>
struct MlaCfg {
  static constexpr bool C8 = mla_int(F);
  // Dense integer formats run three workgroups per CU (three waves per SIMD):
  // ring slots of exactly the 1-KiB loads a tile needs (21 for a 20992-B C8
  // tile) and one score buffer (two barriers per tile) fit three in the LDS,
  // and the tile math of one workgroup hides behind the other two (config-5
  // shapes 380-386 -> 349-356 us against two workgroups with double score
  // buffers). Sparse C8 keeps two: three (with 512-entry slot lists) measured
  // 81 against 72 us on top-2048, and two with 3-slot rings of 21-KiB slots and
  // one score buffer 74 us. Row-quantized slots end with the tile's 32 row
  // scales (256 bytes: the direct-to-LDS scale load writes a dword per lane).
  static constexpr bool TIGHT = C8 && !SPARSE;
  // Dense bf16 calls of at least 2^18 keys (WIDE) run two workgroups per CU,
  // each with a 2-slot ring and one score buffer (exactly 160 KiB): config-5
  // decode 507-510 -> 489-491 us; window 2048 over 128 rows (sinks included:
  // while one workgroup runs a sink block, the other keeps streaming)
  // 0.0735-0.0773 -> 0.0716-0.0753 ms. Smaller calls keep one workgroup with a
  // 4-slot ring and plan for themselves.
  static constexpr bool B2 = !C8 && !SPARSE && WIDE;
  // Row-quantized int8 tiles run two workgroups with 3-slot rings: their
  // gather addressing, bf16 dequantization and the rope codes' extra MFMAs
  // need more than the 168 registers of three workgroups (they spilled 17 and
  // ran 0.514-0.520 against 0.488-0.490 ms on config-5 rows). Int4 tiles (9 KB)
  // run three with 2-slot rings: 0.438-0.441 against 0.471-0.472 ms despite 8
  // spilled registers.
  static constexpr int WGS = F == kFmtRq8 ? 2 : (F == kFmtRq4 ? 3 : (C8 ? ((TIGHT && !SPARSE) ? 3 : 2) : (B2 ? 2 : 1)));
  // Waves per workgroup. Eight waves with 64-dim slices measured slower for
  // bf16 (612 against 532 us on 128 rows of log-uniform [1024, 65536] keys):
  // the score exchange then sums eight partials per tile.
  static constexpr int NW = kMlaWaves;
#ifndef IFATTN_MLA_BF16_STAGES
#define IFATTN_MLA_BF16_STAGES 4
#endif
#ifndef IFATTN_MLA_BF16_XB
#define IFATTN_MLA_BF16_XB 1
#endif
  static constexpr int STAGES = F == kFmtRq8 ? 3 : F == kFmtRq4 ? 2 : (C8 ? 2 : (SPARSE ? 3 : (B2 ? 2 : IFATTN_MLA_BF16_STAGES)));
  // 1-KiB loads per tile
  static constexpr int LOADS = TIGHT ? int((32 * MlaRow<F>::BYTES + 1023) / 1024) : 4 * MlaRow<F>::NI;
  static constexpr int SCALES = mla_rq(F) ? LOADS * 1024 : 0;  // LDS byte of the row scales
  static constexpr int SLOT = TIGHT ? LOADS * 1024 + (mla_rq(F) ? 256 : 0) : int(MlaRow<F>::SLOT);
  static constexpr int XB = (TIGHT || B2) ? 1 : (!C8 && !SPARSE ? IFATTN_MLA_BF16_XB : 2);  // score buffers
  static constexpr int RING = SLOT * STAGES;
  // (+ the self-plan arrays: two ints per planned row, except the wide variant)
  static constexpr int LDS = RING + XB * NW * 64 * 32 + (SPARSE ? 4 * kSparsePart : 0) +
                             (B2 ? 0 : 2 * 4 * 64 * kMlaWaves + 64);
  static_assert(LDS * WGS <= 160 * 1024, "LDS per CU");
  static_assert(!mla_rq(F) || !SPARSE, "row-quantized rows are attended densely");
  // Waves that issue NI loads per tile (the rest issue NI - 1; with row
  // scales, the last wave issues the scale load on top of its NI - 1).
  static constexpr int FULL_WAVES = TIGHT ? LOADS - 4 * (MlaRow<F>::NI - 1) : 4;
  static_assert(!mla_rq(F) || FULL_WAVES < 4, "the scale load goes to a wave with NI - 1 loads");
};
// Persistent workgroups per CU of the kernel variant a call runs (the grid is
// that many per CU, all resident at once).
inline int wgs_mla(int fmt, bool sparse, bool wide) {
  if (fmt == kFmtRq8) return MlaCfg<kFmtRq8, false>::WGS;
  if (fmt == kFmtRq4) return MlaCfg<kFmtRq4, false>::WGS;
  if (fmt != kFmtBf16) return sparse ? MlaCfg<kFmtC8, true>::WGS : MlaCfg<kFmtC8, false>::WGS;
  return sparse ? MlaCfg<kFmtBf16, true>::WGS
                : (wide ? MlaCfg<kFmtBf16, false, true>::WGS : MlaCfg<kFmtBf16, false>::WGS);
}
constexpr int kMlaWgsMax = 3;  // most persistent workgroups per CU of any variant
constexpr int64_t kMlaWideKeys = int64_t(1) << 18;
// Wave geometry of a workgroup of NW waves: wave w owns the latent dims
// [DPW w, DPW w + DPW) for QK^T and PV (KS k-steps of 32), waves 0 and 1 add
// 32 rope dims each; a lane holds EPL dims of each of its eight V tokens and
// the wave runs EPL PV MFMAs (16 dims each).
template <int NW>
struct MlaGeo {
  static constexpr int DPW = 512 / NW;
  static constexpr int KS = DPW / 32;
  static constexpr int EPL = DPW / 16;
};

constexpr uint32_t kNoRow = 0xFFFFFFFFu;  // sparse slot list: no key

__device__ __forceinline__ int mla_tile_token(int g, int j) {
  return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
}

// Eight int8 codes (byte i = element i) times a row scale, as bf16 values
// bf16(code * scale) rounded to nearest even, packed in element order.
__device__ __forceinline__ u32x4 i8x8_dequant_bf16(u32x2 x, float scale) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t wd = int32_t(x[i >> 1]);
    const int sh = 16 * (i & 1);
    const float a = float((wd << (24 - sh)) >> 24), b = float((wd << (16 - sh)) >> 24);
    r[i] = pack_bf16x2(a * scale, b * scale);
  }
  return r;
}
__device__ __forceinline__ uint32_t mla_i8pair(int a, int b) {
  return perm_b32(__float_as_uint(float(b)), __float_as_uint(float(a)), 0x07060302u);
}
__device__ __forceinline__ int mla_i8(uint32_t x, int b) { return (int32_t(x) << (24 - 8 * b)) >> 24; }

// Scores, online softmax and PV of one 32-key tile, from the operands already
// in registers: k = keys 16mt + c of the wave's dims (+ rope), v = keys
// tile_token(g, j) of the wave's 128 latent dims, sk = C8 tile scales of those
// keys. The four waves' partial scores are summed through xbuf (one barrier;
// every wave finished reading xbuf before the barrier that began this tile).
// Keys whose bit is clear in `live` get probability 0.
template <int EPL>
struct MlaAcc {
  f32x4 o[EPL];
  float m, l;
};

// QK^T partial scores of the wave's dims for one 32-key tile, written to xbuf
// (row w * 64 + lane); the caller publishes them with a workgroup barrier.
template <bool C8, int NW>
__device__ __forceinline__ void mla_tile_scores(const u32x4 (&k)[2][MlaGeo<NW>::KS + 1],
                                                const float *sk,
                                                const u32x4 (&qv)[MlaGeo<NW>::KS + 1],
                                                float (*xbuf)[8], int w, int lane,
                                                float k_corr = 0.0f, float q_unscale = 1.0f) {
  constexpr int KS = MlaGeo<NW>::KS;
  f32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if constexpr (C8) {
      a0 = mfma16x16x32_f16(i8x8_to_f16_biased(k[0][s][0], k[0][s][1]), qv[s], a0);
      a1 = mfma16x16x32_f16(i8x8_to_f16_biased(k[1][s][0], k[1][s][1]), qv[s], a1);
    } else {
      a0 = mfma16x16x32(k[0][s], qv[s], a0);
      a1 = mfma16x16x32(k[1][s], qv[s], a1);
    }
  }
  float part_s[8];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    part_s[r] = a0[r];
    part_s[4 + r] = a1[r];
  }
  if constexpr (C8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) part_s[j] = (part_s[j] - k_corr) * (sk[j] * q_unscale);
  }
  if (w < 2) {
    f32x4 r0 = mfma16x16x32(k[0][KS], qv[KS], f32x4{0, 0, 0, 0});
    f32x4 r1 = mfma16x16x32(k[1][KS], qv[KS], f32x4{0, 0, 0, 0});
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      part_s[r] += r0[r];
      part_s[4 + r] += r1[r];
    }
  }
  *reinterpret_cast<f32x4 *>(&xbuf[w * 64 + lane][0]) = f32x4{part_s[0], part_s[1], part_s[2], part_s[3]};
  *reinterpret_cast<f32x4 *>(&xbuf[w * 64 + lane][4]) = f32x4{part_s[4], part_s[5], part_s[6], part_s[7]};
}

// Sum of the waves' partial scores (published in xbuf), online softmax and PV
// of one 32-key tile.
template <bool C8, int NW>
__device__ __forceinline__ void mla_tile_softmax_pv(MlaAcc<MlaGeo<NW>::EPL> &acc,
                                                    const u32x4 (&v)[8], const float *sk,
                                                    const float (*xbuf)[8], uint32_t live,
                                                    float scale_log2, int lane) {
  constexpr int EPL = MlaGeo<NW>::EPL;
  const int g = lane >> 4;
  float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const f32x4 lo = *reinterpret_cast<const f32x4 *>(&xbuf[u * 64 + lane][0]);
    const f32x4 hi = *reinterpret_cast<const f32x4 *>(&xbuf[u * 64 + lane][4]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] += lo[r];
      x[4 + r] += hi[r];
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] *= scale_log2;
  if (live != 0xFFFFFFFFu) {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (live >> mla_tile_token(g, j)) & 1u ? x[j] : -INFINITY;
  }
  float tmax = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                     fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
  tmax = max_xor16(tmax);
  tmax = max_xor32(tmax);
  if (__any(tmax > acc.m + 8.0f)) {
    const float m_new = fmaxf(acc.m, tmax);
    const float alpha = fast_exp2(acc.m - m_new);
    acc.m = m_new;
    acc.l *= alpha;
#pragma unroll
    for (int i = 0; i < EPL; ++i) acc.o[i] *= alpha;
  }
  float pr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(x[j] - acc.m);
  acc.l += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
  if constexpr (C8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] *= sk[j];
  }
  const u32x4 pb = {pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                    pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7])};
#pragma unroll
  for (int b = 0; b < EPL; ++b) {
    u32x4 a;
    if constexpr (C8) {
      const int wd = b >> 2, y = b & 3;
      a = u32x4{mla_i8pair(mla_i8(v[0][wd], y), mla_i8(v[1][wd], y)),
                mla_i8pair(mla_i8(v[2][wd], y), mla_i8(v[3][wd], y)),
                mla_i8pair(mla_i8(v[4][wd], y), mla_i8(v[5][wd], y)),
                mla_i8pair(mla_i8(v[6][wd], y), mla_i8(v[7][wd], y))};
    } else {
      const int wd = b >> 1;
      if (b & 1)
        a = u32x4{pack_hi16(v[0][wd], v[1][wd]), pack_hi16(v[2][wd], v[3][wd]),
                  pack_hi16(v[4][wd], v[5][wd]), pack_hi16(v[6][wd], v[7][wd])};
      else
        a = u32x4{pack_lo16(v[0][wd], v[1][wd]), pack_lo16(v[2][wd], v[3][wd]),
                  pack_lo16(v[4][wd], v[5][wd]), pack_lo16(v[6][wd], v[7][wd])};
    }
    acc.o[b] = mfma16x16x32(a, pb, acc.o[b]);
  }
}

// Both halves with the barrier between them (sink items, one buffer).
template <bool C8, int NW>
__device__ __forceinline__ void mla_tile_math(MlaAcc<MlaGeo<NW>::EPL> &acc,
                                              const u32x4 (&k)[2][MlaGeo<NW>::KS + 1],
                                              const u32x4 (&v)[8], const float *sk,
                                              const u32x4 (&qv)[MlaGeo<NW>::KS + 1],
                                              float (*xbuf)[8], uint32_t live, float scale_log2,
                                              int w, int lane) {
  mla_tile_scores<C8, NW>(k, sk, qv, xbuf, w, lane);
  __syncthreads();
  mla_tile_softmax_pv<C8, NW>(acc, v, sk, xbuf, live, scale_log2, lane);
}

// One (row, partition) item. Tiles of the partition go HBM -> LDS once by
// direct-to-LDS loads shared by the four waves through a ring of R::STAGES
// slots; every wave reads its K operand (keys in rows) and its V operand (dims
// in rows) from the same LDS bytes.
// Tiles [j0, j1) of row `row` (span sp): output, or partial slot `slot` when
// slot >= 0.
template <int F, bool SPARSE, bool WIDE>
__device__ __forceinline__ void mla_item(const MlaParams &p, uint8_t *ring, float (*xbuf)[8],
                                         uint32_t *slot_list, int row, const MlaSpan &sp, int j0,
                                         int j1, int slot, int w, int lane) {
  constexpr bool C8 = mla_int(F);  // integer latent codes (C8 or row-quantized)
  constexpr bool RQ = mla_rq(F);
  using R = MlaRow<F>;
  using Cfg = MlaCfg<F, SPARSE, WIDE>;
  constexpr int S = Cfg::STAGES;
  constexpr int NW = Cfg::NW;
  using Geo = MlaGeo<NW>;
  constexpr int DPW = Geo::DPW, KS = Geo::KS, EPL = Geo::EPL;
  constexpr int DV = 512;
  const int c = lane & 15, g = lane >> 4;
  const bool head_live = c < p.heads;
  const bool partials = slot >= 0;

  // Q operand: latent dims DPW w + 32s + 8g (s < KS), rope dims 32w + 8g (w < 2).
  // Unconditional buffer loads (padded heads and waves without rope dims read
  // zeros from out-of-range offsets), issued together with the block ids or
  // the slot list below; the C8 conversion waits for them after that.
  u32x4 qv[KS + 1];
  {
    const auto rq = make_rsrc(p.q + int64_t(row) * p.heads * 576, uint32_t(p.heads) * 576 * 2);
    const uint32_t qh = head_live ? uint32_t(c) * 576 * 2 : 0x80000000u;
#pragma unroll
    for (int s = 0; s < KS; ++s) qv[s] = buf_load_x4(rq, qh + uint32_t(DPW * w + 32 * s + 8 * g) * 2);
    qv[KS] = buf_load_x4(rq, (w < 2 ? qh : 0x80000000u) + uint32_t(512 + 32 * w + 8 * g) * 2);
  }
  // Wave-uniform (scalar) range bounds: the tile address arithmetic below
  // then runs on the scalar unit.
  const int tile0 = uniform(sp.base + j0 * kMlaTile);
  const int t_begin = uniform(sp.lo > tile0 ? sp.lo : tile0);
  const int t_end = uniform(sp.hi < sp.base + j1 * kMlaTile ? sp.hi : sp.base + j1 * kMlaTile);
  const int n_tiles = j1 - j0;
  const int bs = p.block_size;
  const int64_t seq_table = int64_t(sp.seq) * p.table_stride;

  int lane_blocks = 0;
  if constexpr (SPARSE) {
    // Physical rows of this partition's index entries (kNoRow for padding or
    // out-of-table positions): all index loads, then all table loads, each
    // batch issued before any result is used.
    constexpr int PER = (kSparsePart + 64 * NW - 1) / (64 * NW);
    const int n = t_end - tile0;
    const auto ri = make_rsrc(p.indices + int64_t(row) * p.topk + tile0, uint32_t(n) * 4);
    const auto rb = make_rsrc(p.block_tables + seq_table, uint32_t(p.table_stride) * 4);
    int pos[PER], blk[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k)  // entries past n read as 0 and are not stored
      pos[k] = int(buf_load_x1(ri, uint32_t(threadIdx.x + k * 64 * NW) * 4));
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const bool ok = pos[k] >= 0;  // pos / bs >= table_stride reads 0 (buffer bounds)
      blk[k] = int(buf_load_x1(rb, ok ? uint32_t(pos[k] / bs) * 4 : 0x80000000u));
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int i = threadIdx.x + k * 64 * NW;
      if (i < n) {
        uint32_t slot = kNoRow;
        if (pos[k] >= 0 && pos[k] / bs < p.table_stride) {
          int b = blk[k];
          b = b < 0 ? 0 : (b >= p.num_blocks ? int(p.num_blocks - 1) : b);
          slot = uint32_t(b) * uint32_t(bs) + uint32_t(pos[k] & (bs - 1));
        }
        slot_list[i] = slot;
      }
    }
  }
  // Dense: block ids of a 64-block window from block wblk0 of the sequence,
  // one per lane; the window slides (one vector load) when a tile to be
  // issued leaves it, so a range may span any number of blocks. Entries past
  // the range end read as 0 (buffer bounds).
  const int nblk_end = (t_end - 1) / bs + 1;
  int wblk0 = tile0 / bs;
  const auto rw = make_rsrc(p.block_tables + seq_table, uint32_t(nblk_end) * 4);
  auto load_window = [&]() {
    const int b = int(buf_load_x1(rw, uint32_t(wblk0 + lane) * 4));
    lane_blocks = b < 0 ? 0 : (b >= p.num_blocks ? int(p.num_blocks - 1) : b);
  };
  if constexpr (!SPARSE) load_window();
  // C8 rows: the latent QK^T runs in fp16 on the biased codes (code +
  // kI8Bias, exact); the wave's q slice is scaled per head by a power of two
  // into fp16 range, and kI8Bias * sum(q slice) leaves each partial score.
  // (Row-quantized keys are dequantized to bf16 instead; see score().)
  float k_corr = 0.0f, q_unscale = 1.0f;
  if constexpr (C8 && !RQ) {
    float amax = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) amax = fmaxf(amax, bf16x8_absmax(qv[s]));
    amax = max_xor32(max_xor16(amax));
    const float qs = f16_range_scale(amax);
    float qsum = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) qv[s] = bf16x8_to_f16(qv[s], qs, &qsum);
    k_corr = kI8Bias * sum_xor32(sum_xor16(qsum));
    q_unscale = 1.0f / qs;
  }

  // Per-lane chunk of each direct-to-LDS load: tile row and byte within the row.
  uint32_t lrow[R::NI], lcol[R::NI];
#pragma unroll
  for (int k = 0; k < R::NI; ++k) {
    const uint32_t l = uint32_t((k * 4 + w) * 64 + lane);
    lrow[k] = l / R::CHUNKS;
    const uint32_t jj = l % R::CHUNKS;
    lcol[k] = 16 * (C8 ? jj : (jj ^ R::key(lrow[k], jj)));
  }

  if constexpr (SPARSE) __syncthreads();  // slot list complete

  const uint32_t ring_base = lds_addr(ring);
  const int bs_log2 = __builtin_ctz(uint32_t(bs));  // block_size: host-checked power of two
  // Waves 0..3 move the tiles (NI loads each); further waves only compute.
  auto issue = [&](int ti) {
    if (NW > kMlaWaves && w >= kMlaWaves) return;
    const int t0 = tile0 + ti * kMlaTile;
    const uint32_t dst = ring_base + uint32_t(ti % S) * Cfg::SLOT + uint32_t(w) * 1024;
    if constexpr (SPARSE) {
      // Gather: rows named by the slot list; offsets from the cache base.
      const u32x4 rc = raw_rsrc(p.cache, p.cache_bytes);
#pragma unroll
      for (int k = 0; k < R::NI; ++k) {
        if constexpr (Cfg::TIGHT)
          if (4 * k + w >= Cfg::LOADS) break;
        const uint32_t r = lrow[k];
        const uint32_t slot = r < 32u && t0 + int(r) < t_end ? slot_list[ti * kMlaTile + r] : kNoRow;
        const uint32_t off = slot == kNoRow ? 0xFFFFFFF0u : slot * R::BYTES + lcol[k];
        lds_dma16(rc, off, dst + uint32_t(k) * 4096);
      }
    } else if constexpr (RQ) {
      // Row-quantized rows: every lane gathers its chunk's row through the
      // block window (any page size; rows outside [t_begin, t_end) land as
      // zeros), and the last wave loads the tile's 32 row scales behind the rows.
      const int lower = t_begin > t0 ? t_begin - t0 : 0;
      const int upper = t_end - t0 < kMlaTile ? t_end - t0 : kMlaTile;
      if (((t0 + kMlaTile - 1) >> bs_log2) - wblk0 >= 64) {
        wblk0 = t0 >> bs_log2;
        load_window();
      }
      const u32x4 rc = raw_rsrc(p.cache, p.cache_bytes);
      auto row_slot = [&](int r) {  // physical row of tile row r (all lanes take part)
        const int pos = t0 + r;
        const int blk = __shfl(lane_blocks, ((pos >> bs_log2) - wblk0) & 63, 64);
        return uint32_t(blk) * uint32_t(bs) + uint32_t(pos & (bs - 1));
      };
#pragma unroll
      for (int k = 0; k < R::NI; ++k) {
        if (4 * k + w >= Cfg::LOADS) break;
        const int r = int(lrow[k]);
        const uint32_t srow = row_slot(r & 31);
        const uint32_t off = r >= lower && r < upper ? srow * R::BYTES + lcol[k] : 0xFFFFFFF0u;
        lds_dma16(rc, off, dst + uint32_t(k) * 4096);
      }
      if (w == 3) {
        const uint32_t srow = row_slot(lane & 31);
        const uint32_t off = lane < 32 && lane >= lower && lane < upper ? srow * 4u : 0xFFFFFFF0u;
        lds_dma4(raw_rsrc(p.row_scales, p.scale_bytes), off,
                 ring_base + uint32_t(ti % S) * Cfg::SLOT + uint32_t(Cfg::SCALES));
      }
    } else {
      const int lower = t_begin > t0 ? t_begin - t0 : 0;  // rows before the window start
      const int upper = t_end - t0 < kMlaTile ? t_end - t0 : kMlaTile;
      // Dense bf16 tiles stream with the nontemporal policy (config-5 decode
      // 506 against 522-528 us; C8 unchanged, sparse gathers and the GQA
      // decode's register loads measured slower with it).
      // A tile is one block, or two 16-row blocks (bf16 rows only, where load
      // n = 4k + w < 18 moves rows 0..15 and the rest rows 16..31). Each part's
      // base sits at its first live row: earlier rows wrap to offsets past the
      // extent and land as zeros, like rows past the end.
      // C8 blocks hold at least 32 rows (host-checked): one part per tile.
      const int halves = !C8 && bs < kMlaTile ? 2 : 1;
      if (((t0 + kMlaTile - 1) >> bs_log2) - wblk0 >= 64) {
        wblk0 = t0 >> bs_log2;
        load_window();
      }
      u32x4 rc[2];
      uint32_t first_row[2];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        if (hb < halves) {
          const int r0 = hb * (kMlaTile / halves), r1 = r0 + kMlaTile / halves;
          const int a = lower > r0 ? lower : r0, b = upper < r1 ? upper : r1;
          const int blk = __builtin_amdgcn_readlane(lane_blocks, (t0 >> bs_log2) - wblk0 + hb);
          const int64_t tok = int64_t(blk) * bs + (t0 & (bs - 1)) + (a - r0);
          rc[hb] = raw_rsrc(p.cache + tok * R::BYTES, b > a ? uint32_t(b - a) * R::BYTES : 0u);
          first_row[hb] = uint32_t(a);
        }
      }
#pragma unroll
      for (int k = 0; k < R::NI; ++k) {
        if constexpr (Cfg::TIGHT)
          if (4 * k + w >= Cfg::LOADS) break;
        const int hb = (halves == 2 && 4 * k + w >= 18) ? 1 : 0;
        lds_dma16<!C8>(hb ? rc[1] : rc[0], (lrow[k] - first_row[hb]) * R::BYTES + lcol[k],
                  dst + uint32_t(k) * 4096);
      }
    }
  };

  MlaAcc<EPL> acc;
#pragma unroll
  for (int i = 0; i < EPL; ++i) acc.o[i] = f32x4{0, 0, 0, 0};
  acc.m = -INFINITY;
  acc.l = 0.0f;

  // Stage 1 of a tile: operands from LDS (V kept in registers for stage 2)
  // and the wave's partial scores into xb.
  auto score = [&](const uint8_t *tile, int t0, u32x4 (&v)[8], float (&sk)[C8 ? 8 : 1],
                   uint32_t &live, float (*xb)[8]) {
    // Live rows of this tile (wave-uniform mask).
    if constexpr (SPARSE) {
      const bool ok = lane < 32 && t0 + lane < t_end && slot_list[t0 - tile0 + lane] != kNoRow;
      live = uint32_t(__ballot(ok));
    } else {
      const int lower = t_begin > t0 ? t_begin - t0 : 0;
      const int upper = t_end - t0 < kMlaTile ? t_end - t0 : kMlaTile;
      live = (upper >= 32 ? 0xFFFFFFFFu : ((1u << upper) - 1u)) & ~((1u << lower) - 1u);
    }
    // K operand: token 16mt + c, latent dims DPW w + 32s + 8g (+ rope dims 32(w&1) + 8g).
    // Row-quantized keys become the bf16 values if_cache_dequantize writes,
    // bf16(code * scale) (cache_quantization.cpp:39-57): a score depends on
    // that rounding (a large-scale row moves by up to a percent without it),
    // so the keys are scored exactly as the reference's dequantized cache.
    u32x4 k[2][KS + 1];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const uint32_t r = uint32_t(16 * mt + c);
      if constexpr (RQ) {
        const float rs = *reinterpret_cast<const float *>(tile + Cfg::SCALES + 4 * r);
        auto codes = [&](uint32_t dim) {  // 8 codes of dims dim .. dim + 7
          if constexpr (F == kFmtRq4)
            return i4x8_to_i8x8(*reinterpret_cast<const uint32_t *>(tile + r * R::BYTES + dim / 2));
          else
            return *reinterpret_cast<const u32x2 *>(tile + r * R::BYTES + dim);
        };
#pragma unroll
        for (int s = 0; s < KS; ++s) k[mt][s] = i8x8_dequant_bf16(codes(uint32_t(DPW * w + 32 * s + 8 * g)), rs);
        k[mt][KS] = w < 2 ? i8x8_dequant_bf16(codes(uint32_t(512 + 32 * (w & 1) + 8 * g)), rs)
                          : u32x4{0, 0, 0, 0};
        continue;
      }
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if constexpr (C8) {
          const u32x2 x = *reinterpret_cast<const u32x2 *>(tile + r * R::BYTES + DPW * w + 32 * s + 8 * g);
          k[mt][s] = u32x4{x[0], x[1], 0u, 0u};
        } else {
          k[mt][s] = load_u32x4(tile + R::chunk(r, uint32_t((DPW / 8) * w + 4 * s + g)));
        }
      }
      if (w < 2) {
        if constexpr (C8)
          k[mt][KS] = load_u32x4(tile + r * R::BYTES + 512 + 64 * (w & 1) + 16 * g);
        else
          k[mt][KS] = load_u32x4(tile + R::chunk(r, uint32_t(64 + 4 * (w & 1) + g)));
      } else {
        k[mt][KS] = u32x4{0, 0, 0, 0};
      }
    }
    // V operand rows: token tile_token(g, j), latent dims DPW w + EPL c .. + EPL.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t r = uint32_t(mla_tile_token(g, j));
      if constexpr (RQ) {
        static_assert(EPL == 8, "row-quantized V operands are 8 dims per lane");
        if constexpr (F == kFmtRq4) {
          const u32x2 x = i4x8_to_i8x8(
              *reinterpret_cast<const uint32_t *>(tile + r * R::BYTES + (DPW * w + 8 * c) / 2));
          v[j] = u32x4{x[0], x[1], 0u, 0u};
        } else {
          const u32x2 x = *reinterpret_cast<const u32x2 *>(tile + r * R::BYTES + DPW * w + 8 * c);
          v[j] = u32x4{x[0], x[1], 0u, 0u};
        }
        sk[j] = *reinterpret_cast<const float *>(tile + Cfg::SCALES + 4 * r);
      } else if constexpr (C8) {
        if constexpr (EPL == 8) {
          const u32x2 x = *reinterpret_cast<const u32x2 *>(tile + r * R::BYTES + DPW * w + 8 * c);
          v[j] = u32x4{x[0], x[1], 0u, 0u};
        } else {
          v[j] = u32x4{*reinterpret_cast<const uint32_t *>(tile + r * R::BYTES + DPW * w + 4 * c), 0u, 0u, 0u};
        }
        sk[j] = *reinterpret_cast<const float *>(tile + r * R::BYTES + 640 + 4 * ((DPW * w) / 128));
      } else {
        if constexpr (EPL == 8) {
          v[j] = load_u32x4(tile + R::chunk(r, uint32_t(16 * w + c)));
        } else {
          const u32x2 x = *reinterpret_cast<const u32x2 *>(
              tile + R::chunk(r, uint32_t((DPW / 8) * w + (c >> 1))) + 8 * (c & 1));
          v[j] = u32x4{x[0], x[1], 0u, 0u};
        }
      }
    }

    // Row-quantized keys were dequantized above: bf16 scores, no scale.
    mla_tile_scores<C8 && !RQ, NW>(k, sk, qv, xb, w, lane, k_corr, q_unscale);
  };

  // Ring: tile ti lives in slot ti % S; tiles 0..S-1 are issued up front. In
  // iteration ti every wave reads tile ti's operands (V stays in registers)
  // and writes its partial scores to xbuf half ti & 1; one barrier then
  // publishes those scores and tile ti+1 and retires the reads of tile ti,
  // whose slot receives tile ti+S before the softmax and PV of tile ti run.
  // One barrier per tile: the other half of xbuf is still being read by
  // slower waves while faster ones write the next tile's scores.
#pragma unroll
  for (int i = 0; i < S; ++i)
    if (i < n_tiles) issue(i);
  // Loads per wave per tile: NI, or NI - 1 for the waves past LOADS (the
  // scale load brings the last wave of a row-quantized tile back to NI).
  const bool full_loads = !Cfg::TIGHT || w < Cfg::FULL_WAVES || (RQ && w == 3);
  if (S - 1 < n_tiles) {  // tile 0; tiles 1 .. S-1 may stay in flight
    if (full_loads)
      lds_dma_wait<(S - 1) * R::NI>();
    else
      lds_dma_wait<(S - 1) * (R::NI - 1)>();
  } else {
    lds_dma_wait<0>();
  }
  __syncthreads();
  for (int ti = 0; ti < n_tiles; ++ti) {
    float (*xb)[8] = xbuf + (Cfg::XB == 2 ? (ti & 1) : 0) * NW * 64;
    u32x4 v[8];
    float sk[C8 ? 8 : 1];
    uint32_t live;
    score(ring + (ti % S) * Cfg::SLOT, tile0 + ti * kMlaTile, v, sk, live, xb);
    if (ti + S - 1 < n_tiles) {  // tile ti+1; tiles ti+2 .. ti+S-1 may stay in flight
      if (full_loads)
        lds_dma_wait<(S - 2) * R::NI>();
      else
        lds_dma_wait<(S - 2) * (R::NI - 1)>();
    } else {
      lds_dma_wait<0>();
    }
    __syncthreads();
    if (ti + S < n_tiles) issue(ti + S);
    mla_tile_softmax_pv<C8, NW>(acc, v, sk, xb, live, p.scale_log2, lane);
    if constexpr (Cfg::XB == 1) __syncthreads();  // xb is rewritten by the next tile
  }

  float l_tot = sum_xor16(acc.l);
  l_tot = sum_xor32(l_tot);
  if (!head_live) return;
  // Lane holds rows m = 4g + r of MFMA b -> dim DPW w + EPL(4g + r) + b: the
  // 4 EPL consecutive dims from DPW w + 4 EPL g.
  float ov[4 * EPL];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < EPL; ++b) ov[EPL * r + b] = acc.o[b][r];
  const int d0 = DPW * w + 4 * EPL * g;
  if (!partials) {
    const float inv = 1.0f / l_tot;
    uint16_t *op = p.out + (int64_t(row) * p.heads + c) * DV + d0;
#pragma unroll
    for (int k = 0; k < EPL / 2; ++k) {
      const float *v = ov + 8 * k;
      store_u32x4(op + 8 * k, u32x4{pack_bf16x2(v[0] * inv, v[1] * inv),
                                    pack_bf16x2(v[2] * inv, v[3] * inv),
                                    pack_bf16x2(v[4] * inv, v[5] * inv),
                                    pack_bf16x2(v[6] * inv, v[7] * inv)});
    }
  } else {
    // Partials store O / l in bf16 (half the partial traffic; the merge
    // weighs them by l), (m, l) in fp32.
    const int64_t prow = int64_t(slot) * p.heads + c;
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t *po = p.part_o + prow * DV + d0;
#pragma unroll
    for (int k = 0; k < EPL / 2; ++k) {
      const float *v = ov + 8 * k;
      store_u32x4(po + 8 * k, u32x4{pack_bf16x2(v[0] * inv, v[1] * inv),
                                    pack_bf16x2(v[2] * inv, v[3] * inv),
                                    pack_bf16x2(v[4] * inv, v[5] * inv),
                                    pack_bf16x2(v[6] * inv, v[7] * inv)});
    }
    if (w == 0 && g == 0) *reinterpret_cast<float2 *>(p.part_ml + prow * 2) = make_float2(acc.m, l_tot);
  }
}

// Learned sink rows of one query row (keys [n, 576], values [n, 512] bf16,
// shared by every row, so they are read from L2): the same tile math as the
// cache keys, four waves per row, heads in the MFMA N dimension. The (m, l, O)
// partial of the sinks alone goes to the row's first partial slot. Runs as the
// event at the start of the row's work units, in the share that holds it.
template <int NW, bool DB>
__device__ __forceinline__ void mla_sink_item(const MlaParams &p, float (*xbuf)[8], int row, int slot0,
                                              int w, int lane) {
  using Geo = MlaGeo<NW>;
  constexpr int DPW = Geo::DPW, KS = Geo::KS, EPL = Geo::EPL;
  const int c = lane & 15, g = lane >> 4, n = p.n_sinks;
  const bool head_live = c < p.heads;
  u32x4 qv[KS + 1];
  {
    const uint16_t *qp = p.q + (int64_t(row) * p.heads + (head_live ? c : 0)) * 576;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qv[s] = head_live ? load_u32x4(qp + DPW * w + 32 * s + 8 * g) : u32x4{0, 0, 0, 0};
    qv[KS] = (head_live && w < 2) ? load_u32x4(qp + 512 + 32 * w + 8 * g) : u32x4{0, 0, 0, 0};
  }
  MlaAcc<EPL> acc;
#pragma unroll
  for (int i = 0; i < EPL; ++i) acc.o[i] = f32x4{0, 0, 0, 0};
  acc.m = -INFINITY;
  acc.l = 0.0f;
  // DB (the one-workgroup-per-CU variant, which has the registers): tile
  // t + 1's rows are loaded (from L2: every row reads the same sinks) while
  // tile t is computed, two register sets alternating. The variants with
  // several workgroups per CU spilled with the second set and load one tile at
  // a time.
  auto load = [&](int t0, u32x4 (&k)[2][KS + 1], u32x4 (&v)[8]) {
    const int live_n = n - t0 < kMlaTile ? n - t0 : kMlaTile;
    // Rows past the last sink read as zero (buffer extent).
    const auto rk = make_rsrc(p.sink_k + int64_t(t0) * 576, uint32_t(live_n) * 1152u);
    const auto rv = make_rsrc(p.sink_v + int64_t(t0) * 512, uint32_t(live_n) * 1024u);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const uint32_t r = uint32_t(16 * mt + c) * 1152u;
#pragma unroll
      for (int s = 0; s < KS; ++s) k[mt][s] = buf_load_x4(rk, r + 2 * (DPW * w + 32 * s + 8 * g));
      k[mt][KS] = w < 2 ? buf_load_x4(rk, r + 1024 + 2 * (32 * (w & 1) + 8 * g)) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t off = uint32_t(mla_tile_token(g, j)) * 1024u + 2 * (DPW * w + EPL * c);
      if constexpr (EPL == 8) {
        v[j] = buf_load_x4(rv, off);
      } else {
        const u32x2 x = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0));
        v[j] = u32x4{x[0], x[1], 0u, 0u};
      }
    }
  };
  auto math = [&](int t0, const u32x4 (&k)[2][KS + 1], const u32x4 (&v)[8]) {
    const int live_n = n - t0 < kMlaTile ? n - t0 : kMlaTile;
    const uint32_t live = live_n >= 32 ? 0xFFFFFFFFu : ((1u << live_n) - 1u);
    mla_tile_math<false, NW>(acc, k, v, nullptr, qv, xbuf, live, p.scale_log2, w, lane);
    __syncthreads();  // xbuf is rewritten by the next tile
  };
  if constexpr (DB) {
    u32x4 ka[2][KS + 1], va[8], kb[2][KS + 1], vb[8];
    if (n > 0) load(0, ka, va);
    for (int t0 = 0; t0 < n; t0 += 2 * kMlaTile) {
      if (t0 + kMlaTile < n) load(t0 + kMlaTile, kb, vb);
      math(t0, ka, va);
      if (t0 + kMlaTile >= n) break;
      if (t0 + 2 * kMlaTile < n) load(t0 + 2 * kMlaTile, ka, va);
      math(t0 + kMlaTile, kb, vb);
    }
  } else {
    for (int t0 = 0; t0 < n; t0 += kMlaTile) {
      u32x4 k[2][KS + 1], v[8];
      load(t0, k, v);
      math(t0, k, v);
    }
  }
  float l_tot = sum_xor16(acc.l);
  l_tot = sum_xor32(l_tot);
  if (!head_live) return;
  const int64_t prow = int64_t(slot0) * p.heads + c;  // the row's first slot
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  uint16_t *po = p.part_o + prow * 512 + DPW * w + 4 * EPL * g;
#pragma unroll
  for (int k = 0; k < EPL; ++k) {
    const int r = (4 * k) / EPL, b = (4 * k) % EPL;  // dims EPL r + b .. + 3 of the lane's run
    *reinterpret_cast<u32x2 *>(po + 4 * k) =
        u32x2{pack_bf16x2(acc.o[b][r] * inv, acc.o[b + 1][r] * inv),
              pack_bf16x2(acc.o[b + 2][r] * inv, acc.o[b + 3][r] * inv)};
  }
  if (w == 0 && g == 0) *reinterpret_cast<float2 *>(p.part_ml + prow * 2) = make_float2(acc.m, l_tot);
}

// Rows a workgroup plans for itself (one per thread): calls of at most this
// many rows skip the plan launch.
constexpr int kMlaSelfPlanRows = 64 * kMlaWaves;
// Workgroup-wide scan over kMlaSelfPlanRows threads (sum or max, inclusive),
// wave totals through `wt`; *total gets the workgroup's total.
template <bool MAX>
__device__ __forceinline__ int wg_scan(int x, int *wt, int *total) {
  constexpr int NWV = kMlaSelfPlanRows / 64;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x = MAX ? (y > x ? y : x) : x + y;
  }
  if (lane == 63) wt[wv] = x;
  __syncthreads();
  int before = MAX ? -1 : 0, all = MAX ? -1 : 0;
#pragma unroll
  for (int u = 0; u < NWV; ++u) {
    const int t = wt[u];
    if (u < wv) before = MAX ? (t > before ? t : before) : before + t;
    all = MAX ? (t > all ? t : all) : all + t;
  }
  __syncthreads();  // wt is reused by the next scan
  *total = all;
  return MAX ? (before > x ? before : x) : before + x;
}
// The plan of a call of at most kMlaSelfPlanRows rows, computed by every
// attention workgroup for itself (the same arithmetic as mla_plan_kernel, in
// 32-bit units: the host allows it only when every prefix fits): s_pos = first
// unit of each row; s_se = (first partial slot + 1) << 16 | (running max of
// the rows' last-event workers + 1), both below 2^16 (host-checked): slot -1
// means the output is written directly, and the start row of worker v is the
// first row whose running max reaches v. Workgroup 0 also stores the rows'
// slots for the merge and zeroes the output of rows without keys and sinks.
// (Two ints per row keep three dense C8 workgroups within a CU's LDS.)
__device__ __forceinline__ int mla_se_slot(int se) { return (se >> 16) - 1; }
__device__ __forceinline__ int mla_se_e(int se) { return (se & 0xFFFF) - 1; }
__device__ __forceinline__ void mla_self_plan(const MlaParams &p, int *s_pos, int *s_se, int *s_wt,
                                              int64_t *s_tab, int &workers, int64_t &total_units) {
  const int row = threadIdx.x;
  const bool live = row < p.num_rows;
  MlaSpan sp{0, 0, 0, 0};
  int w = 0;
  if (live) {
    sp = mla_span(p, row, mla_seq_of(p, row));
    w = int(mla_row_weight(p, sp));
  }
  int total;
  const int pos = wg_scan<false>(w, s_wt, &total) - w;
  workers = mla_split(p, total);
  total_units = total;
  if (threadIdx.x == 0) mla_shares_fill(p, total, workers, s_tab);
  __syncthreads();
  const MlaShares<> sh{s_tab, 0, p.skew_pm};
  int cnt = 0, e = -1;
  if (live) {
    const MlaRowWork rw = mla_row_work(p, sp, pos, sh);
    cnt = rw.slots;
    if (rw.tiles > 0) e = rw.wb;
    else if (p.sink_units > 0) e = sh.worker(mla_sink_mid(p, pos));
  }
  int nslots;
  const int slot = wg_scan<false>(cnt, s_wt, &nslots) - cnt;
  int emax;
  const int einc = wg_scan<true>(e, s_wt, &emax);
  if (live) {
    s_pos[row] = pos;
    s_se[row] = ((cnt > 0 ? slot : -1) + 1) << 16 | (einc + 1);
    if (blockIdx.x == 0) {
      p.row_slot[row] = make_int2(cnt > 0 ? slot : -1, cnt);
      if (w == 0) {  // no keys and no sinks: defined zero output
        uint16_t *o = p.out + int64_t(row) * p.heads * 512;
        for (int i = 0; i < p.heads * 512; i += 8) store_u32x4(o + i, u32x4{0, 0, 0, 0});
      }
    }
  }
  __syncthreads();
}

// The same plan for the wide layout, whose LDS holds no per-row arrays: every
// workgroup computes it and stores each row's first unit and partial slots
// into the plan arrays the plan launch would write (row_pos, row_slot). Every
// workgroup writes the same values, and each reads them back only after its
// own stores (program order and the workgroup barrier), so whichever store a
// read returns carries this call's value. `scratch` (the score buffer, unused
// until the first tile) holds the scans' wave totals, the rows' running
// last-event workers and the start row of this workgroup's worker, which is
// returned (workers <= grid for dense calls: one worker per workgroup).
__device__ __forceinline__ int mla_self_plan_global(const MlaParams &p, int *scratch, int &workers,
                                                    int64_t &total_units) {
  int *s_wt = scratch, *s_e = scratch + 8, *s_start = scratch + 4;
  const int row = threadIdx.x;
  const bool live = row < p.num_rows;
  MlaSpan sp{0, 0, 0, 0};
  int w = 0;
  if (live) {
    sp = mla_span(p, row, mla_seq_of(p, row));
    w = int(mla_row_weight(p, sp));
  }
  if (row == 0) *s_start = p.num_rows;
  int total;
  const int pos = wg_scan<false>(w, s_wt, &total) - w;
  workers = mla_split(p, total);
  total_units = total;
  const MlaShares<false> sh{nullptr, total > 0 ? (int64_t(total) + workers - 1) / workers : 1, p.skew_pm};
  int cnt = 0, e = -1;
  if (live) {
    const MlaRowWork rw = mla_row_work(p, sp, pos, sh);
    cnt = rw.slots;
    if (rw.tiles > 0) e = rw.wb;
    else if (p.sink_units > 0) e = sh.worker(mla_sink_mid(p, pos));
  }
  int nslots;
  const int slot = wg_scan<false>(cnt, s_wt, &nslots) - cnt;
  int emax;
  const int einc = wg_scan<true>(e, s_wt, &emax);
  if (live) {
    s_e[row] = einc;
    p.row_pos[row] = pos;
    p.row_slot[row] = make_int2(cnt > 0 ? slot : -1, cnt);
    if (blockIdx.x == 0 && w == 0) {  // no keys and no sinks: defined zero output
      uint16_t *o = p.out + int64_t(row) * p.heads * 512;
      for (int i = 0; i < p.heads * 512; i += 8) store_u32x4(o + i, u32x4{0, 0, 0, 0});
    }
  }
  __syncthreads();
  // Start row of worker v = blockIdx.x: the first row whose running
  // last-event worker reaches v.
  const int v = int(blockIdx.x);
  if (live && einc >= v && (row == 0 || s_e[row - 1] < v)) *s_start = row;
  __syncthreads();
  const int start = *s_start;
  __syncthreads();  // the scratch is the score buffer from here on
  return start;
}

// STEP: the fused decode step (mla_step_kernel); the plain calls run kernels
// without its row writes and its kernel argument.
template <int F, bool SPARSE, bool WIDE, bool STEP>
__device__ __forceinline__ void mla_attention_body(const MlaParams &p, const MlaStep &st) {
  using Cfg = MlaCfg<F, SPARSE, WIDE>;
  constexpr int NW = Cfg::NW;
  __shared__ __align__(16) uint8_t ring[Cfg::RING];
  __shared__ __align__(16) float xbuf[Cfg::XB * NW * 64][8];  // score exchange
  // The sparse slot list lives in the workgroup's LDS only for sparse calls
  // (the dense C8 variant fits two workgroups per CU exactly).
  uint32_t *slot_list = nullptr;
  if constexpr (SPARSE) {
    __shared__ uint32_t sparse_slots[kSparsePart];
    slot_list = sparse_slots;
  }
  const int lane = threadIdx.x & 63;
  const int w = uniform(int(threadIdx.x >> 6));
  // Small calls: the plan in this workgroup's LDS (the wide variant has no LDS
  // to spare and serves large calls only).
  static_assert(NW * 64 == kMlaSelfPlanRows, "one planned row per thread");
  constexpr int SPR = Cfg::B2 ? 1 : kMlaSelfPlanRows;
  __shared__ int s_pos[SPR], s_se[SPR], s_wt[NW];
  __shared__ int64_t s_tab[Cfg::B2 ? 1 : kMlaShareTab];
  int workers;
  int64_t s0 = 0;
  const bool self = !Cfg::B2 && p.self_plan;
  int g_start = 0;  // wide layout planned in the kernel: this workgroup's start row
  if (self) {
    int64_t total;
    mla_self_plan(p, s_pos, s_se, s_wt, s_tab, workers, total);
  } else if (Cfg::B2 && p.self_plan) {
    int64_t total;
    g_start = mla_self_plan_global(p, reinterpret_cast<int *>(&xbuf[0][0]), workers, total);
    s0 = total > 0 ? (total + workers - 1) / workers : 1;
  } else {
    // Plan entries through scalar loads (ld_const): vector loads here each
    // waited behind the previous item's output stores.
    workers = ld_const(p.plan);
    const int64_t total = ld_const(reinterpret_cast<const int64_t *>(p.plan + 2));
    if constexpr (Cfg::B2) {
      s0 = total > 0 ? (total + workers - 1) / workers : 1;
    } else {
      if (threadIdx.x == 0) mla_shares_fill(p, total, workers, s_tab);
      __syncthreads();
    }
  }
  workers = uniform(workers);  // scalar (the self plan's scans leave it in a vector register)
  const MlaShares<!Cfg::B2> sh{s_tab, s0, p.skew_pm};
  // Plan arrays written by this kernel (the wide layout's in-kernel plan) are
  // read with ordinary loads: the scalar constant path may not see them.
  const bool gplan = Cfg::B2 && p.self_plan;
  auto start_row = [&](int v) {
    if (gplan) return g_start;
    if (!self) return int(ld_const(p.start_row + v));
    int a = 0, b = p.num_rows;  // first row whose running last-event worker reaches v
    while (a < b) {
      const int m = (a + b) >> 1;
      if (mla_se_e(s_se[m]) >= v) b = m; else a = m + 1;
    }
    return a;
  };
  // Workgroup b walks the shares b, b + grid, ... row by row: a row's sink
  // block is one event at its middle unit, its tiles j at first + 32 j.
  if constexpr (STEP) {
    static_assert(!SPARSE && !mla_rq(F), "the fused step is a dense bf16 / C8 decode");
    // Fused decode step: before any tile is loaded, the workgroup writes the
    // step's row of every sequence whose last tile (the one holding its last
    // position) lies in one of its shares; no other workgroup reads that tile.
    // One thread per sequence finds them (in parallel: a serial walk of the
    // rows put a chain of dependent loads ahead of the first tile); each wave
    // then writes the rows its lanes found, one row at a time. The decode
    // rows are one per sequence, without window or sinks, so tile 0 of row r
    // sits at unit row_pos[r] + row_cost.
    for (int base = 0; base < p.num_rows; base += NW * 64) {
      const int row = base + int(threadIdx.x);
      bool mine = false;
      int last = 0;
      if (row < p.num_rows) {
        const int64_t pos = self ? int64_t(s_pos[row]) : p.row_pos[row];
        int kv = p.kv_lens[row];
        kv = kv > p.max_context ? p.max_context : kv;
        if (kv > 0) {
          const int tiles = (kv + kMlaTile - 1) / kMlaTile;
          const int wb = sh.worker(pos + p.row_cost + int64_t(kMlaTile) * (tiles - 1));
          mine = wb < workers && wb % int(gridDim.x) == int(blockIdx.x);
          last = kv - 1;
        }
      }
      uint64_t todo = __ballot(mine);
      while (todo) {
        const int bit = __builtin_ctzll(todo);
        todo &= todo - 1;
        const int r = base + w * 64 + bit;
        const int lr = __shfl(last, bit, 64);
        int blk = ld_const(p.block_tables + int64_t(r) * p.table_stride + lr / p.block_size);
        blk = blk < 0 ? 0 : (blk >= p.num_blocks ? int(p.num_blocks - 1) : blk);
        const int64_t slot_w = int64_t(blk) * p.block_size + (lr & (p.block_size - 1));
        mla_norm_rope_row<F == kFmtC8>(st.x + int64_t(r) * 576, st.gamma, st.cos + int64_t(r) * 64,
                                       st.sin + int64_t(r) * 64, st.eps,
                                       st.cache + slot_w * MlaRow<F>::BYTES, lane);
      }
    }
    // The stores must have reached L2 before any wave loads the tile: a wait
    // on this wave's stores suffices, because only this workgroup reads the row
    // and its lines are not in the CU's L1 (tile boundaries are whole 128-B
    // lines apart, and the L1 starts the kernel invalidated). A device-scope
    // fence here wrote back the XCD's L2 and cost 50 us a call.
    lds_dma_wait<0>();
    __syncthreads();
  }
  const int sinks = p.n_sinks > 0 ? 1 : 0;
  for (int v = blockIdx.x; v < workers; v += gridDim.x) {
    const int64_t lo = uniform(sh.lo(v)), hi = uniform(sh.lo(v + 1));
    for (int row = start_row(v); row < p.num_rows; ++row) {
      const int64_t pos = self ? int64_t(s_pos[row]) : (gplan ? p.row_pos[row] : ld_const(p.row_pos + row));
      if (pos >= hi) break;
      const int slot0 =
          self ? mla_se_slot(s_se[row]) : (gplan ? p.row_slot[row].x : ld_const(&p.row_slot[row].x));
      if (sinks && mla_sink_mid(p, pos) >= lo && mla_sink_mid(p, pos) < hi) {
        mla_sink_item<NW, Cfg::WGS == 1>(p, xbuf, row, slot0, w, lane);
        __syncthreads();  // every wave is done with xbuf
      }
      const int seq = !p.cu_q ? row : (self || gplan ? mla_seq_of(p, row) : ld_const(p.row_seq + row));
      const MlaSpan sp = mla_span(p, row, seq);
      const MlaRowWork rw = mla_row_work(p, sp, pos, sh);
      if (rw.tiles == 0) continue;
      const int64_t a = lo - rw.first, b = hi - rw.first;
      const int j0 = uniform(a <= 0 ? 0 : int((a + kMlaTile - 1) / kMlaTile));
      int j1 = b <= 0 ? 0 : int((b + kMlaTile - 1) / kMlaTile);
      j1 = uniform(j1 < rw.tiles ? j1 : rw.tiles);
      if (j0 >= j1) continue;
      const int slot = uniform(slot0 >= 0 ? slot0 + sinks + (v - rw.wa) : -1);
      mla_item<F, SPARSE, WIDE>(p, ring, xbuf, slot_list, row, sp, j0, j1, slot, w, lane);
      __syncthreads();  // every wave is done with xbuf (and the ring)
    }
  }
}

template <int F, bool SPARSE, bool WIDE>
__global__ __launch_bounds__(64 * (MlaCfg<F, SPARSE, WIDE>::NW), (MlaCfg<F, SPARSE, WIDE>::WGS)) void mla_attention_kernel(MlaParams p) {
  mla_attention_body<F, SPARSE, WIDE, false>(p, MlaStep{});
}

template <int F, bool WIDE>
__global__ __launch_bounds__(64 * (MlaCfg<F, false, WIDE>::NW), (MlaCfg<F, false, WIDE>::WGS)) void mla_step_kernel(MlaParams p, MlaStep st) {
  mla_attention_body<F, false, WIDE, true>(p, st);
}

// Combine one (row, head): the row's partials (the sink partial first, when
// there are sinks, then one per share its tiles touch). Each thread owns 2
// output dims.
__global__ __launch_bounds__(256) void mla_merge_kernel(MlaParams p) {
  const int row = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int2 slots = make_int2(ld_const(&p.row_slot[row].x), ld_const(&p.row_slot[row].y));
  if (slots.x < 0) return;  // output written by the attention kernel or the plan
  const int slot0 = slots.x, total = slots.y;
  const int64_t prow0 = int64_t(slot0) * p.heads + h;
  auto part_at = [&](int k) { return prow0 + int64_t(k) * p.heads; };
  uint32_t *op = reinterpret_cast<uint32_t *>(p.out + (int64_t(row) * p.heads + h) * 512) + tid;
  constexpr int kFast = 8;
  if (total <= kFast) {
    // One round trip: every (m, l) and O word of the row's partials is loaded
    // together (indices past the last partial repeat it with weight 0) and
    // each thread takes the max itself.
    float2 m_l[kFast];
    uint32_t o[kFast];
#pragma unroll
    for (int k = 0; k < kFast; ++k) {
      const int64_t pr = part_at(k < total ? k : total - 1);
      m_l[k] = *reinterpret_cast<const float2 *>(p.part_ml + pr * 2);
      o[k] = *reinterpret_cast<const uint32_t *>(p.part_o + pr * 512 + 2 * tid);
    }
    float Mt = -INFINITY;
#pragma unroll
    for (int k = 0; k < kFast; ++k) Mt = fmaxf(Mt, m_l[k].x);
    if (Mt == -INFINITY) {  // nothing visible
      *op = 0u;
      return;
    }
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int k = 0; k < kFast; ++k) {
      const float wk = k < total ? fast_exp2(m_l[k].x - Mt) * m_l[k].y : 0.0f;  // partials hold O / l
      L += wk;
      o0 += wk * bf16_bits_to_f32(o[k] & 0xFFFFu);
      o1 += wk * bf16_bits_to_f32(o[k] >> 16);
    }
    const float inv = 1.0f / L;
    *op = pack_bf16x2(o0 * inv, o1 * inv);
    return;
  }
  // Largest partial max: threads stride over the partials, then a
  // workgroup reduction (4 waves).
  __shared__ float wmax[4];
  float mp = -INFINITY;
  for (int k = tid; k < total; k += 256) mp = fmaxf(mp, p.part_ml[part_at(k) * 2]);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mp = wave_max_xor(mp, m);
  if ((tid & 63) == 0) wmax[tid >> 6] = mp;
  __syncthreads();
  const float Mt = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  if (Mt == -INFINITY) {  // nothing visible
    *op = 0u;
    return;
  }
  float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll 8
  for (int k = 0; k < total; ++k) {
    const int64_t pr = part_at(k);
    const float2 m_l = *reinterpret_cast<const float2 *>(p.part_ml + pr * 2);
    const uint32_t o = *reinterpret_cast<const uint32_t *>(p.part_o + pr * 512 + 2 * tid);
    const float wk = fast_exp2(m_l.x - Mt) * m_l.y;  // partials hold O / l
    L += wk;
    o0 += wk * bf16_bits_to_f32(o & 0xFFFFu);
    o1 += wk * bf16_bits_to_f32(o >> 16);
  }
  const float inv = 1.0f / L;
  *op = pack_bf16x2(o0 * inv, o1 * inv);
}

namespace {

struct MlaCall {
  int fmt;  // MlaFmt
  const uint16_t *w_x = nullptr, *w_gamma = nullptr, *w_cos = nullptr, *w_sin = nullptr;
  float w_eps = 0.0f;
  const void *q, *cache;
  const float *row_scales;  // row-quantized formats
  const int32_t *block_tables;
  int32_t table_stride;
  const int32_t *cu_q, *kv_lens;
  int32_t num_seqs, num_rows;
  const int32_t *indices;
  int32_t topk, window;
  const void *sink_k, *sink_v;
  int32_t n_sinks;
  void *out;
  int32_t heads, block_size;
  int64_t num_blocks;
  int32_t max_context;
  float scale;
  void *workspace;
  uint64_t workspace_bytes;
  void *stream;
};

// Share skew (permille) of dense bf16 calls, as for the GQA decode: odd
// workers run on odd XCDs, whose tiles are slower (config-5 rows 0.4257 ->
// 0.4225 ms with 3%, 0.4165-0.4181 ms with 6% against 0.4211-0.4216 at 3% on
// one box, 4.5%: 0.4185, 8%: 0.4172-0.4191, 10%: 0.4200-0.4214; 0.4307 ms
// with the opposite skew). Only the wide variant (two workgroups per CU)
// without sinks is skewed: the one-workgroup variant of small calls runs
// tiles at the same rate on both parities (window-2048 calls: 1.497 against
// 1.507 us per tile), and the skew only unbalanced them (0.073-0.074 ms
// without, 0.078-0.079 ms with, on one box); with sinks the even workers also
// hold the sink blocks (window 2048 in the wide variant: 0.0701-0.0713 ms at
// 0 and 3%, 0.0737-0.0751 ms at 6%). C8 calls keep equal shares (3% and 6%
// measured 0.5-1.5% slower), and so do sparse calls (their shares are capped
// by the slot list). IFATTN_MLA_XCD_SKEW (0..200) overrides the default of
// dense calls.
inline int mla_skew_pm(bool c8, bool sparse, bool wide, bool sinks) {
  static const int v = [] {
    const char *e = getenv("IFATTN_MLA_XCD_SKEW");
    const int x = e ? atoi(e) : 1000;
    return (x >= 0 && x <= 200) ? x : 1000;
  }();
  return sparse ? 0 : (v != 1000 ? v : (c8 || !wide || sinks ? 0 : 60));
}
// Share weights of the dispatch slots (MlaShares), permille: the k-th
// workgroup of a CU gets a share in proportion to weight k. Dense integer
// tiles (C8, row-quantized), measured on config-5 rows against equal shares
// on the same box: C8 0.334-0.335 -> 0.320-0.326 ms at 1400/1000/600
// (1100/1000/900 and 1300/1000/700 gained less; 1500/1000/500 and
// 1600/1000/400 measured 0.334-0.343 against 0.328 ms on a later box), int4
// rows 0.435-0.439 -> 0.399-0.402 ms at 1400/1000/600, and 0.409-0.411 ->
// 0.400-0.402 ms from 1400/1000/600 to 1500/1000/500 on the later box; int8
// rows (two per CU) 0.480-0.503 -> 0.464-0.470 ms at 1300/1000, and
// 0.469-0.479 -> 0.467-0.468 ms at 1500/1000 on the later box. Sparse calls (two per CU) were 2-6% slower
// with weights and keep equal shares; the wide bf16 variant (no LDS for the
// table) always does.
// IFATTN_MLA_SLOT_WEIGHTS ("w0,w1[,w2]") overrides the weights of every
// variant but the wide one.
inline void mla_slot_weights(MlaParams &p, int wgs, int fmt, bool sparse, bool wide) {
  static const std::array<int, kMlaSlotsMax> env = [] {
    std::array<int, kMlaSlotsMax> w{0, 0, 0};
    if (const char *e = getenv("IFATTN_MLA_SLOT_WEIGHTS")) {
      for (int k = 0; k < kMlaSlotsMax && *e; ++k) {
        w[k] = atoi(e);
        while (*e && *e != ',') ++e;
        if (*e == ',') ++e;
      }
    }
    return w;
  }();
  p.slot_n = 1;
  p.slot_c = device_cus();
  for (int k = 0; k < kMlaSlotsMax; ++k) p.slot_w[k] = 1000;
  if (wgs < 2 || wgs > kMlaSlotsMax || wide) return;
  std::array<int, kMlaSlotsMax> w{1000, 1000, 1000};
  if (env[0] > 0)
    w = env;
  else if (fmt == kFmtBf16 || sparse)
    return;
  else if (fmt == kFmtC8)
    w = std::array<int, kMlaSlotsMax>{1400, 1000, 600};
  else
    w = wgs == 3 ? std::array<int, kMlaSlotsMax>{1500, 1000, 500}
                 : std::array<int, kMlaSlotsMax>{1500, 1000, 0};
  // Malformed weights: equal shares.
  int wsum = 0;
  for (int k = 0; k < wgs; ++k) wsum += w[k];
  for (int k = 0; k < wgs; ++k)
    if (w[k] < 100 || w[k] > 10000 || int64_t(w[k]) * wgs > 2 * int64_t(wsum)) return;
  p.slot_n = wgs;
  for (int k = 0; k < wgs; ++k) p.slot_w[k] = w[k];
}
// Work units charged per row start (tunable: IFATTN_MLA_ROW_COST), and the
// share cap of sparse calls: a share's tiles (at most share/32 + 1 of them)
// keep their index entries within the kSparsePart slot list.
inline int mla_row_cost() {
  static const int v = [] {
    const char *e = getenv("IFATTN_MLA_ROW_COST");
    const int x = e ? atoi(e) : -1;
    return (x >= 0 && x <= 65536) ? x : 64;
  }();
  return v;
}
constexpr int kMlaSparseShare = kSparsePart - 2 * kMlaTile;
// Units of a sink block: its tiles plus a start (the sink rows come from L2).
constexpr int kMlaSinkStart = 64;
inline int mla_sink_units(int n_sinks) {
  return n_sinks > 0 ? kMlaTile * ((n_sinks + kMlaTile - 1) / kMlaTile) + kMlaSinkStart : 0;
}
// Workers the workspace holds: the largest persistent grid, or for sparse
// calls enough capped shares for rows of topk entries.
inline uint64_t mla_max_workers(bool sparse, int rows, int topk, int n_sinks) {
  const uint64_t grid = uint64_t(device_cus()) * kMlaWgsMax;
  if (!sparse) return grid;
  const uint64_t per_row = uint64_t(mla_sink_units(n_sinks)) + mla_row_cost() +
                           uint64_t(kMlaTile) * ((uint64_t(topk) + kMlaTile - 1) / kMlaTile);
  const uint64_t need = (uint64_t(rows) * per_row + kMlaSparseShare - 1) / kMlaSparseShare;
  return need > grid ? need : grid;
}
// Workspace: plan words | row_pos | row_seq | row_slot | start_row | partial
// O | partial (m, l). Partial slots: one per row for the sinks, and at most
// two per worker for the key shares.
inline uint64_t mla_workspace(int rows, int heads, bool sparse, int topk, int n_sinks) {
  const uint64_t workers = mla_max_workers(sparse, rows, topk, n_sinks);
  const uint64_t slots = 2 * workers + (n_sinks > 0 ? uint64_t(rows) : 0);
  return kQueueBytes + 2 * align16(uint64_t(rows) * 8) + align16(uint64_t(rows) * 4) +
         align16(workers * 4) + slots * heads * (512 * sizeof(uint16_t) + 2 * sizeof(float));
}

int32_t mla_run(const MlaCall &c, const char *what) {
  const bool sparse = c.indices != nullptr;
  if (!c.q || !c.cache || !c.block_tables || !c.kv_lens || !c.out)
    return fail(IFATTN_EINVAL, what, "null pointer");
  if (c.num_seqs <= 0 || c.num_rows <= 0 || c.num_rows >= (1 << 20) || c.heads <= 0 || c.heads > 16)
    return fail(IFATTN_EINVAL, what, "1..16 heads, 1..2^20-1 rows and at least one sequence");
  if (!c.cu_q && c.num_rows != c.num_seqs)
    return fail(IFATTN_EINVAL, what, "without cu_seqlens_q every sequence has one row");
  const bool rq = c.fmt == kFmtRq8 || c.fmt == kFmtRq4;
  if (c.block_size < (c.fmt == kFmtC8 ? 32 : 16) || (c.block_size & (c.block_size - 1)))
    return fail(IFATTN_EINVAL, what,
                "block_size must be a power of two >= 16 (bf16, row-quantized) or >= 32 (C8)");
  if (c.max_context <= 0 || c.num_blocks <= 0 || c.table_stride <= 0 ||
      int64_t(c.table_stride) * c.block_size < c.max_context)
    return fail(IFATTN_EINVAL, what, "table_stride * block_size must cover max_context");
  if (!aligned16(c.q) || !aligned16(c.out) || !aligned16(c.cache))
    return fail(IFATTN_EINVAL, what, "q, out and cache must be 16-byte aligned");
  const uint64_t row_bytes = c.fmt == kFmtC8 ? 656 : (c.fmt == kFmtRq8 ? 576 : (c.fmt == kFmtRq4 ? 288 : 1152));
  if (uint64_t(c.block_size) * row_bytes > (1ull << 31))
    return fail(IFATTN_EINVAL, what, "block too large");
  const uint64_t cache_bytes = uint64_t(c.num_blocks) * c.block_size * row_bytes;
  if (sparse && (c.topk <= 0 || cache_bytes > 0xFFFFFFF0ull))
    return fail(IFATTN_EINVAL, what, "sparse attention needs topk > 0 and a cache below 4 GiB");
  if (rq && (sparse || !c.row_scales || !aligned4(c.row_scales) || cache_bytes > 0xFFFFFFF0ull))
    return fail(IFATTN_EINVAL, what,
                "row-quantized rows: dense attention, 4-byte aligned scales, a cache below 4 GiB");
  if (c.window < 0) return fail(IFATTN_EINVAL, what, "window must be >= 0");
  if (c.n_sinks < 0 || c.n_sinks > kMaxSinks || (c.n_sinks > 0 && (!c.sink_k || !c.sink_v)) ||
      (c.n_sinks > 0 && (!aligned4(c.sink_k) || !aligned4(c.sink_v))))
    return fail(IFATTN_EINVAL, what, "0..128 sink rows with 4-byte aligned keys and values");
  // Two-workgroup bf16 layout for large dense calls: at least kMlaWideKeys
  // keys possible over all rows.
  const int64_t span = (c.window > 0 && c.window < c.max_context) ? int64_t(c.window) + 31 : c.max_context;
  const bool wide = c.fmt == kFmtBf16 && !sparse && int64_t(c.num_rows) * span >= kMlaWideKeys;
  const int wgs = wgs_mla(c.fmt, sparse, wide);
  const uint64_t need = mla_workspace(c.num_rows, c.heads, sparse, c.topk, c.n_sinks);
  if (!c.workspace || c.workspace_bytes < need || !aligned16(c.workspace))
    return fail(IFATTN_EWORKSPACE, what, "workspace missing, short or misaligned");
  const uint64_t max_workers = mla_max_workers(sparse, c.num_rows, c.topk, c.n_sinks);
  if (max_workers > (uint64_t(1) << 28)) return fail(IFATTN_EINVAL, what, "too many rows for the work split");
  MlaParams p{};
  p.q = static_cast<const uint16_t *>(c.q);
  p.cache = static_cast<const uint8_t *>(c.cache);
  p.block_tables = c.block_tables;
  p.kv_lens = c.kv_lens;
  p.cu_q = c.cu_q;
  p.indices = c.indices;
  p.sink_k = static_cast<const uint16_t *>(c.sink_k);
  p.sink_v = static_cast<const uint16_t *>(c.sink_v);
  p.out = static_cast<uint16_t *>(c.out);
  p.num_blocks = c.num_blocks;
  p.cache_bytes = (sparse || rq) ? uint32_t(cache_bytes) : 0u;
  p.row_scales = rq ? c.row_scales : nullptr;
  p.scale_bytes = rq ? uint32_t(uint64_t(c.num_blocks) * c.block_size * 4) : 0u;
  p.num_seqs = c.num_seqs;
  p.num_rows = c.num_rows;
  p.heads = c.heads;
  p.table_stride = c.table_stride;
  p.block_size = c.block_size;
  p.max_context = c.max_context;
  p.topk = c.topk;
  p.window = c.window;
  p.n_sinks = c.n_sinks;
  p.scale_log2 = c.scale * kLog2e;
  const int grid = device_cus() * wgs;
  p.row_cost = mla_row_cost();
  p.sink_units = mla_sink_units(c.n_sinks);
  p.max_share = sparse ? kMlaSparseShare : 0x7FFFFFFF;
  p.skew_pm = mla_skew_pm(c.fmt != kFmtBf16, sparse, wide, c.n_sinks > 0);
  mla_slot_weights(p, wgs, c.fmt, sparse, wide);
  p.max_workers = int(max_workers);
  p.grid = grid;
  // Self-planned calls: few rows and every prefix of row units within 32
  // bits (the wide layout plans into the plan arrays instead of LDS).
  p.self_plan = c.num_rows <= kMlaSelfPlanRows &&
                int64_t(c.num_rows) * (int64_t(c.max_context) + p.row_cost + p.sink_units + kMlaTile) <
                    (int64_t(1) << 31) &&
                2 * max_workers + uint64_t(c.num_rows) < 0xFFFFu;
  uint8_t *ws = static_cast<uint8_t *>(c.workspace);
  p.plan = reinterpret_cast<int32_t *>(ws);
  ws += kQueueBytes;
  p.row_pos = reinterpret_cast<int64_t *>(ws);
  ws += align16(uint64_t(c.num_rows) * 8);
  p.row_seq = reinterpret_cast<int32_t *>(ws);
  ws += align16(uint64_t(c.num_rows) * 4);
  p.row_slot = reinterpret_cast<int2 *>(ws);
  ws += align16(uint64_t(c.num_rows) * 8);
  p.start_row = reinterpret_cast<int32_t *>(ws);
  ws += align16(max_workers * 4);
  const uint64_t slots = 2 * max_workers + (c.n_sinks > 0 ? uint64_t(c.num_rows) : 0);
  p.part_o = reinterpret_cast<uint16_t *>(ws);
  p.part_ml = reinterpret_cast<float *>(p.part_o + slots * c.heads * 512);
  hipStream_t s = static_cast<hipStream_t>(c.stream);
  if (!p.self_plan) mla_plan_kernel<<<1, 1024, 0, s>>>(p);
  constexpr int kThreads = 64 * kMlaWaves;
  const bool step = c.w_x != nullptr;
  MlaStep st{c.w_x, c.w_gamma, c.w_cos, c.w_sin,
             const_cast<uint8_t *>(static_cast<const uint8_t *>(c.cache)), c.w_eps};
  if (step && (sparse || rq || c.cu_q || c.window || c.n_sinks))
    return fail(IFATTN_EINVAL, what, "the fused step is a plain decode");
  if (c.fmt == kFmtC8) {
    if (sparse) mla_attention_kernel<kFmtC8, true, false><<<grid, kThreads, 0, s>>>(p);
    else if (step) mla_step_kernel<kFmtC8, false><<<grid, kThreads, 0, s>>>(p, st);
    else mla_attention_kernel<kFmtC8, false, false><<<grid, kThreads, 0, s>>>(p);
  } else if (c.fmt == kFmtRq8) {
    mla_attention_kernel<kFmtRq8, false, false><<<grid, kThreads, 0, s>>>(p);
  } else if (c.fmt == kFmtRq4) {
    mla_attention_kernel<kFmtRq4, false, false><<<grid, kThreads, 0, s>>>(p);
  } else {
    if (sparse) mla_attention_kernel<kFmtBf16, true, false><<<grid, kThreads, 0, s>>>(p);
    else if (wide && step) mla_step_kernel<kFmtBf16, true><<<grid, kThreads, 0, s>>>(p, st);
    else if (wide) mla_attention_kernel<kFmtBf16, false, true><<<grid, kThreads, 0, s>>>(p);
    else if (step) mla_step_kernel<kFmtBf16, false><<<grid, kThreads, 0, s>>>(p, st);
    else mla_attention_kernel<kFmtBf16, false, false><<<grid, kThreads, 0, s>>>(p);
  }
  mla_merge_kernel<<<dim3(c.num_rows, c.heads), 256, 0, s>>>(p);
  return launch_status(what);
}

MlaCall decode_call(int fmt, const void *q, const void *cache, const int32_t *block_tables,
                    int32_t table_stride, const int32_t *seq_lens, void *out, int32_t num_seqs,
                    int32_t heads, int32_t block_size, int64_t num_blocks, int32_t max_context,
                    float scale, void *workspace, uint64_t workspace_bytes, void *stream) {
  MlaCall c{};
  c.fmt = fmt;
  c.q = q;
  c.cache = cache;
  c.block_tables = block_tables;
  c.table_stride = table_stride;
  c.kv_lens = seq_lens;
  c.num_seqs = c.num_rows = num_seqs;
  c.out = out;
  c.heads = heads;
  c.block_size = block_size;
  c.num_blocks = num_blocks;
  c.max_context = max_context;
  c.scale = scale;
  c.workspace = workspace;
  c.workspace_bytes = workspace_bytes;
  c.stream = stream;
  return c;
}

}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" uint64_t ifattn_mla_decode_workspace_size(int32_t num_seqs, int32_t heads,
                                                     int32_t max_context, int32_t block_size) {
  if (num_seqs <= 0 || heads <= 0 || max_context <= 0 || block_size <= 0) return 0;
  (void)max_context;
  (void)block_size;
  return mla_workspace(num_seqs, heads, false, 0, 0);
}

extern "C" int32_t ifattn_mla_decode_bf16(const void *q, const void *cache,
                                          const int32_t *block_tables, int32_t table_stride,
                                          const int32_t *seq_lens, void *out, int32_t num_seqs,
                                          int32_t heads, int32_t block_size, int64_t num_blocks,
                                          int32_t max_context, float scale, void *workspace,
                                          uint64_t workspace_bytes, void *stream) {
  return mla_run(decode_call(kFmtBf16, q, cache, block_tables, table_stride, seq_lens, out, num_seqs,
                             heads, block_size, num_blocks, max_context, scale, workspace,
                             workspace_bytes, stream),
                 "mla decode");
}

extern "C" int32_t ifattn_mla_decode_c8(const void *q, const void *cache,
                                        const int32_t *block_tables, int32_t table_stride,
                                        const int32_t *seq_lens, void *out, int32_t num_seqs,
                                        int32_t heads, int32_t block_size, int64_t num_blocks,
                                        int32_t max_context, float scale, void *workspace,
                                        uint64_t workspace_bytes, void *stream) {
  return mla_run(decode_call(kFmtC8, q, cache, block_tables, table_stride, seq_lens, out, num_seqs,
                             heads, block_size, num_blocks, max_context, scale, workspace,
                             workspace_bytes, stream),
                 "mla decode c8");
}

extern "C" uint64_t ifattn_mla_attention_workspace_size(int32_t num_rows, int32_t heads,
                                                        int32_t max_context, int32_t window,
                                                        int32_t topk, int32_t n_sinks,
                                                        int32_t block_size) {
  if (num_rows <= 0 || heads <= 0 || max_context <= 0 || block_size <= 0) return 0;
  (void)max_context;
  (void)window;
  (void)block_size;
  return mla_workspace(num_rows, heads, topk > 0, topk, n_sinks);
}

extern "C" int32_t ifattn_mla_window_attention_bf16(
    const void *q, const void *cache, const int32_t *block_tables, int32_t table_stride,
    const int32_t *cu_seqlens_q, const int32_t *kv_lens, int32_t num_seqs, int32_t num_rows,
    int32_t window, const void *sink_keys, const void *sink_values, int32_t n_sinks, void *out,
    int32_t heads, int32_t block_size, int64_t num_blocks, int32_t max_context, float scale,
    void *workspace, uint64_t workspace_bytes, void *stream) {
  MlaCall c = decode_call(kFmtBf16, q, cache, block_tables, table_stride, kv_lens, out, num_seqs,
                          heads, block_size, num_blocks, max_context, scale, workspace,
                          workspace_bytes, stream);
  c.cu_q = cu_seqlens_q;
  c.num_rows = num_rows;
  c.window = window;
  c.sink_k = sink_keys;
  c.sink_v = sink_values;
  c.n_sinks = n_sinks;
  return mla_run(c, "mla window attention");
}

extern "C" int32_t ifattn_mla_sparse_attention_c8(
    const void *q, const void *cache, const int32_t *indices, int32_t topk,
    const int32_t *block_tables, int32_t table_stride, const int32_t *cu_seqlens_q,
    const int32_t *kv_lens, int32_t num_seqs, int32_t num_rows, const void *sink_keys,
    const void *sink_values, int32_t n_sinks, void *out, int32_t heads, int32_t block_size,
    int64_t num_blocks, int32_t max_context, float scale, void *workspace,
    uint64_t workspace_bytes, void *stream) {
  if (!indices) return fail(IFATTN_EINVAL, "mla sparse attention: null indices");
  MlaCall c = decode_call(kFmtC8, q, cache, block_tables, table_stride, kv_lens, out, num_seqs,
                          heads, block_size, num_blocks, max_context, scale, workspace,
                          workspace_bytes, stream);
  c.cu_q = cu_seqlens_q;
  c.num_rows = num_rows;
  c.indices = indices;
  c.topk = topk;
  c.sink_k = sink_keys;
  c.sink_v = sink_values;
  c.n_sinks = n_sinks;
  return mla_run(c, "mla sparse attention");
}

extern "C" int32_t ifattn_mla_window_attention_rowq(
    const void *q, const void *cache, const float *row_scales, int32_t bits,
    const int32_t *block_tables, int32_t table_stride, const int32_t *cu_seqlens_q,
    const int32_t *kv_lens, int32_t num_seqs, int32_t num_rows, int32_t window,
    const void *sink_keys, const void *sink_values, int32_t n_sinks, void *out, int32_t heads,
    int32_t block_size, int64_t num_blocks, int32_t max_context, float scale, void *workspace,
    uint64_t workspace_bytes, void *stream) {
  if (bits != 8 && bits != 4) return fail(IFATTN_EINVAL, "mla row-quantized attention: bits 8 or 4");
  MlaCall c = decode_call(bits == 8 ? kFmtRq8 : kFmtRq4, q, cache, block_tables, table_stride,
                          kv_lens, out, num_seqs, heads, block_size, num_blocks, max_context,
                          scale, workspace, workspace_bytes, stream);
  c.row_scales = row_scales;
  c.cu_q = cu_seqlens_q;
  c.num_rows = num_rows;
  c.window = window;
  c.sink_k = sink_keys;
  c.sink_v = sink_values;
  c.n_sinks = n_sinks;
  return mla_run(c, "mla row-quantized attention");
}

extern "C" int32_t ifattn_mla_decode_step(const void *q, const void *x_new, const void *gamma,
                                          const void *cos, const void *sin, float eps, void *cache,
                                          int32_t packed, const int32_t *block_tables,
                                          int32_t table_stride, const int32_t *seq_lens, void *out,
                                          int32_t num_seqs, int32_t heads, int32_t block_size,
                                          int64_t num_blocks, int32_t max_context, float scale,
                                          void *workspace, uint64_t workspace_bytes, void *stream) {
  if (!x_new || !gamma || !cos || !sin)
    return fail(IFATTN_EINVAL, "mla decode step: null writer input");
  if (!aligned16(x_new) || !aligned16(gamma) || !aligned4(cos) || !aligned4(sin))
    return fail(IFATTN_EINVAL, "mla decode step: misaligned writer input");
  if (!(eps >= 0.0f)) return fail(IFATTN_EINVAL, "mla decode step: eps must be >= 0");
  MlaCall c = decode_call(packed ? kFmtC8 : kFmtBf16, q, cache, block_tables, table_stride, seq_lens,
                          out, num_seqs, heads, block_size, num_blocks, max_context, scale, workspace,
                          workspace_bytes, stream);
  c.w_x = static_cast<const uint16_t *>(x_new);
  c.w_gamma = static_cast<const uint16_t *>(gamma);
  c.w_cos = static_cast<const uint16_t *>(cos);
  c.w_sin = static_cast<const uint16_t *>(sin);
  c.w_eps = eps;
  return mla_run(c, "mla decode step");
}
