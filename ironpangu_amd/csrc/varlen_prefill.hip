// Packed varlen chunked-prefill attention over paged bf16 caches (gfx950).
//
// Sequence s owns query rows [cu[s], cu[s+1]) (count rows) and kv_len cached
// keys, this chunk's rows already written (writes precede queries,
// native/include/sliding_window_layout.h:7). Row t of the chunk sees keys
// [0, kv_len - count + t] — the causal rule of
// native/src/openpangu_attention_metadata.h:20-22 — with GQA grouping
// kh = h / (q_heads/kv_heads). fp32 accumulation, bf16 in/out. This replaces the
// TND attention call of native/src/token_executor.h:863-906 (without window
// or sinks).
//
// Work split:
//  * single-row sequences (decode rows of a mixed batch) go to the split-K
//    paged decode kernels through a q-row indirection;
//  * longer chunks are cut into query tiles of 256/G rows (G = q heads per kv
//    head); a workgroup (8 waves, two per SIMD) owns one (sequence, query
//    tile, kv head), and the kv heads of a query tile are adjacent
//    workgroups. The MFMA N dimension packs (query row, grouped head)
//    columns, so all G heads of a kv head reuse every K/V tile. Each wave owns
//    2 column blocks of 16 (1 for head_dim 256).
//  * K/V 32-token tiles are copied HBM -> LDS with direct-to-LDS buffer loads
//    into a ring of steps of four tiles (16-B chunks XOR-swizzled by a row
//    key; two steps at head_dim 128, one in flight); a loop step waits,
//    synchronises and runs the softmax bookkeeping once per 128 keys. QK^T runs transposed (tokens in M,
//    columns in N) so the score tile is already the B operand of the PV MFMA;
//    V^T operands come from transposing LDS reads. The two waves of a SIMD
//    overlap one's MFMAs with the other's softmax.
//  * tiles wholly above the diagonal are never visited; only tiles crossing a
//    column's limit apply the causal mask.
//  * query tiles are scheduled longest-first by a device plan kernel.
#include <cstdlib>

#include "common.h"
#include "ifattn_internal.h"
#include "split_k.h"

namespace ifattn {

struct PrefillParams {
  const uint16_t *q;
  const uint8_t *k_cache;
  const uint8_t *v_cache;
  const int32_t *block_tables;
  const int32_t *cu;
  const int32_t *kv_lens;
  uint16_t *out;
  uint32_t *items;   // (seq << 12 | query tile), longest first
  int32_t *n_items;
  int64_t num_blocks;
  int num_seqs, q_heads, kv_heads, group, table_stride, block_size, max_kv, q_tile;
  int max_q_len;   // rows per sequence beyond this are not scheduled (cu_seqlens is device data)
  int max_items;   // capacity of `items`
  float scale_log2;
};

#ifndef IFATTN_PREFILL_WAVES
#define IFATTN_PREFILL_WAVES 8
#endif
// Eight waves (two per SIMD) with two column blocks each: one wave's softmax
// VALU work overlaps the other's MFMAs.
constexpr int kPrefillWaves = IFATTN_PREFILL_WAVES;
constexpr int kPrefillTile = 32;
constexpr int prefill_nb(int d) {  // column blocks per wave
  return kPrefillWaves == 8 ? (d > 128 ? 1 : 2) : (d > 128 ? 2 : 4);
}
constexpr int prefill_q_tile(int d, int g) { return kPrefillWaves * prefill_nb(d) * 16 / g; }

// Work list for the multi-row sequences, sorted by the number of key tokens
// the query tile visits (descending, 256-token buckets).
__global__ __launch_bounds__(1024) void prefill_plan_kernel(PrefillParams p) {
  constexpr int kBuckets = 1025;
  __shared__ int bucket[kBuckets];
  __shared__ int s_count[1024], s_kv[1024];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int QT = p.q_tile;
  const int nbk = (p.max_kv + 255) / 256 + 1;  // <= kBuckets (host-checked)
  for (int b = tid; b < kBuckets; b += 1024) bucket[b] = 0;
  // Bucket of query tile qt: the key tokens it visits, most work first.
  auto cost_bucket = [&](int kv, int qt, int count) {
    const int rows_end = (qt + 1) * QT < count ? (qt + 1) * QT : count;
    int reach = kv - count + rows_end;
    reach = reach < 0 ? 0 : (reach > p.max_kv ? p.max_kv : reach);
    return nbk - 1 - reach / 256;
  };
  // Sequences are staged 1024 at a time (one parallel load each); the query
  // tiles of a sequence are then spread over the lanes of one wave, so a long
  // chunk costs one LDS atomic per lane instead of a serial loop in one thread.
  auto for_each_tile = [&](auto &&fn) {
    for (int base = 0; base < p.num_seqs; base += 1024) {
      __syncthreads();  // the previous chunk's staged values are no longer read
      if (base + tid < p.num_seqs) {
        const int seq = base + tid;
        const int count = p.cu[seq + 1] - p.cu[seq];
        s_count[tid] = count > p.max_q_len ? p.max_q_len : count;
        const int kv = p.kv_lens[seq];
        s_kv[tid] = kv > p.max_kv ? p.max_kv : kv;
      }
      __syncthreads();
      const int n = p.num_seqs - base < 1024 ? p.num_seqs - base : 1024;
      for (int i = wave; i < n; i += 16) {
        const int count = s_count[i];
        if (count <= 1) continue;
        for (int qt = lane; qt * QT < count; qt += 64) fn(base + i, qt, cost_bucket(s_kv[i], qt, count));
      }
    }
  };
  for_each_tile([&](int, int, int b) { atomicAdd(&bucket[b], 1); });
  __syncthreads();
  {
    static_assert(kBuckets <= 64 * 17, "bucket_prefix covers 17 buckets per lane");
    const int run = bucket_prefix<17>(bucket, nbk - 1, 0, tid);
    if (tid == 0) *p.n_items = run < p.max_items ? run : p.max_items;
  }
  for_each_tile([&](int seq, int qt, int b) {
    const int slot = atomicAdd(&bucket[b], 1);
    if (slot < p.max_items) p.items[slot] = (uint32_t(seq) << 12) | uint32_t(qt);
  });
}

__device__ __forceinline__ int pf_tile_token(int g, int j) {
  return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
}

// K/V tile staging: a ring of kPrefillStages slots, each holding a 32-token
// K tile and V tile (rows of D bf16, no padding). The 16-byte chunks of a row
// are XOR-swizzled by a key derived from the row index so that K operand reads
// and transposing V reads are free of bank conflicts (SQ_LDS_BANK_CONFLICT
// reads 0).
#ifndef IFATTN_PF_STAGES
#define IFATTN_PF_STAGES 3
#endif
// 32-key tiles per loop step: the per-step costs (wait, barrier, row max,
// rescale check) are paid once per 128 keys. At head_dim 128 the ring then
// holds two steps (one being read, one in flight, 128 KiB): config-3 chunks
// 0.2951-0.2989 -> 0.2839-0.2890 ms against two tiles per step in three
// steps (three tiles in two steps: 0.2871-0.2880 ms).
#ifndef IFATTN_PF_KT
#define IFATTN_PF_KT 4
#endif
constexpr int prefill_kt(int d) { return d <= 128 ? IFATTN_PF_KT : 1; }
// Ring depth in steps: up to 128 KiB of staged tiles (16 KiB per tile at
// head_dim 128), at most three steps (one being read, two in flight).
constexpr int prefill_stages(int d) {
  return IFATTN_PF_STAGES * prefill_kt(d) * 4 * 32 * d <= 131072
             ? IFATTN_PF_STAGES
             : 131072 / (prefill_kt(d) * 4 * 32 * d);
}
template <int D>
struct PrefillRing {
  static constexpr int CH = D / 8;                  // 16-byte chunks per row
  static constexpr int SW = CH < 16 ? CH - 1 : 15;  // swizzle mask
  static constexpr int TILE = kPrefillTile * D * 2;  // bytes of one K (or V) tile
  static constexpr int SLOT = 2 * TILE;
  static constexpr int NIW = CH / kPrefillWaves;    // direct-to-LDS loads per wave per tile
  static_assert(CH % kPrefillWaves == 0, "every wave moves the same number of chunks");
  static constexpr int SWB = SW == 15 ? 4 : (SW == 7 ? 3 : (SW == 3 ? 2 : 1));  // mask bits
  // XOR key: the row rotated left by one bit within the mask. The 16 rows of
  // a K operand read get 16 distinct keys, and so do the eight consecutive
  // rows of two 16-lane groups of a transposing V read, whose lanes touch
  // chunk pairs {2b, 2b+1}: keys that differ only in bit 0 (rows r, r^1 under
  // a plain row key) would map both rows' pairs to the same banks. Only row
  // bits below SWB (at most 4) enter the key, so rows r and r + 16 share it.
  static_assert(SWB <= 4, "rows 16 apart share a swizzle key");
  static __device__ __forceinline__ int swz(int row) {
    return ((row << 1) | ((row >> (SWB - 1)) & 1)) & SW;
  }
  static __device__ __forceinline__ uint32_t at(int row, int chunk) {
    return uint32_t(row) * (D * 2) + 16u * uint32_t(chunk ^ swz(row));
  }
};

// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left at their
// maxima (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4], lgkmcnt[11:8]).
constexpr unsigned kVmcntZero = 0x0F70u;

template <int D, int G>
__global__ __launch_bounds__(64 * kPrefillWaves) void varlen_prefill_kernel(PrefillParams p) {
  constexpr int NB = prefill_nb(D);
  constexpr int QT = prefill_q_tile(D, G);
  constexpr int VPL = D / 16;                        // V dims per lane
  using RG = PrefillRing<D>;
  constexpr int S = prefill_stages(D);
  constexpr int KT = prefill_kt(D);
  constexpr int STEP = KT * RG::SLOT;  // LDS bytes of one step's tiles
  __shared__ __align__(16) uint8_t ring[S * STEP];

  // The kv heads of one query tile are adjacent workgroups, so the halves of
  // every cache row are fetched at about the same time (DRAM page hits).
  const int it = int(blockIdx.x) / p.kv_heads;
  const int kvh = int(blockIdx.x) - it * p.kv_heads;
  if (it >= *p.n_items) return;
  const uint32_t e = p.items[it];
  const int seq = int(e >> 12), qt = int(e & 0xfffu);
  const int tid = threadIdx.x, lane = tid & 63, w = uniform(int(tid >> 6));
  const int c = lane & 15, g = lane >> 4;
  const int q0 = p.cu[seq];
  const int count = p.cu[seq + 1] - q0;
  int kv_len = p.kv_lens[seq];
  kv_len = kv_len > p.max_kv ? p.max_kv : kv_len;
  const int row0 = qt * QT;
  const int rows_here = count - row0 < QT ? count - row0 : QT;
  const int base_lim = kv_len - count;  // row t sees keys [0, base_lim + t]
  int range_end = base_lim + row0 + rows_here;
  range_end = range_end < 0 ? 0 : range_end;

  // Columns of this lane: block nb -> (row, head).
  int lim[NB];
  int64_t qrow[NB];
  int head[NB];
  bool live[NB];
  u32x4 qv[NB][D / 32];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = (w * NB + nb) * 16 + c;
    const int r = col / G;
    live[nb] = r < rows_here;
    const int t = row0 + (live[nb] ? r : rows_here - 1);
    lim[nb] = base_lim + t;
    qrow[nb] = int64_t(q0) + t;
    head[nb] = kvh * G + col % G;
    const uint16_t *qp = p.q + (qrow[nb] * p.q_heads + head[nb]) * D + (D / 4) * g;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) qv[nb][s] = live[nb] ? load_u32x4(qp + 8 * s) : u32x4{0, 0, 0, 0};
  }

  const int32_t *table_row = p.block_tables + int64_t(seq) * p.table_stride;
  const uint32_t row_bytes = uint32_t(p.kv_heads) * D * 2;
  // Per-lane source offset (within a tile) of each direct-to-LDS load: load
  // n = (waves)k + w moves chunks 64n .. 64n+63 of the K tile (n < CH/2) or of the
  // V tile (n >= CH/2), in LDS order.
  uint32_t src[RG::NIW];
#pragma unroll
  for (int k = 0; k < RG::NIW; ++k) {
    const int n = kPrefillWaves * k + w;
    const int l = (n % (RG::CH / 2)) * 64 + lane;
    const int row = l / RG::CH, pos = l % RG::CH;
    src[k] = uint32_t(row) * row_bytes + 16u * uint32_t(pos ^ RG::swz(row));
  }
  // Block ids of a 64-block window, one per lane, read with v_readlane: a
  // dependent scalar table load in front of every tile's loads would stall the
  // wave for a memory round trip per tile. The window moves (one vector load)
  // when a tile leaves it.
  const int n_blocks = range_end > 0 ? (range_end - 1) / p.block_size + 1 : 0;
  int win0 = 0;
  int lane_blk = lane < n_blocks ? table_row[lane] : 0;
  const uint32_t ring_base = lds_addr(ring);
  // Tile ti goes to ring slot ti % (S * KT). Tiles past the range (the second
  // tile of a last, half-used step) move no bytes and land as zeros.
  auto issue = [&](int ti) {
    const int t0 = ti * kPrefillTile;
    if (t0 >= range_end) {
      const u32x4 rz = raw_rsrc(p.k_cache, 0u);
      const uint32_t slot = ring_base + uint32_t(ti % (S * KT)) * RG::SLOT;
#pragma unroll
      for (int k = 0; k < RG::NIW; ++k) {
        const int n = kPrefillWaves * k + w;
        const bool is_v = n >= RG::CH / 2;
        lds_dma16(rz, src[k], slot + (is_v ? uint32_t(RG::TILE) : 0u) + uint32_t(n % (RG::CH / 2)) * 1024u);
      }
      return;
    }
    const int bi = t0 / p.block_size;
    if (bi >= win0 + 64) {
      win0 = bi;
      lane_blk = win0 + lane < n_blocks ? table_row[win0 + lane] : 0;
      // Wait here, once per 64 blocks, with a wait the compiler accounts for:
      // otherwise it cannot prove the id load complete at the readlane below
      // and drains every in-flight tile load (vmcnt(0)) on every tile.
      __builtin_amdgcn_s_waitcnt(kVmcntZero);
    }
    int blk = __builtin_amdgcn_readlane(lane_blk, bi - win0);
    blk = blk < 0 ? 0 : (blk >= p.num_blocks ? int(p.num_blocks - 1) : blk);
    const int64_t tok0 = int64_t(blk) * p.block_size + (t0 & (p.block_size - 1));
    const int n_live = range_end - t0 < kPrefillTile ? range_end - t0 : kPrefillTile;
    const uint32_t extent = uint32_t(n_live - 1) * row_bytes + D * 2;  // later rows read as zero
    const int64_t first = (tok0 * p.kv_heads + kvh) * D * 2;
    const u32x4 rk = raw_rsrc(p.k_cache + first, extent);
    const u32x4 rv = raw_rsrc(p.v_cache + first, extent);
    const uint32_t slot = ring_base + uint32_t(ti % (S * KT)) * RG::SLOT;
#pragma unroll
    for (int k = 0; k < RG::NIW; ++k) {
      const int n = kPrefillWaves * k + w;
      const bool is_v = n >= RG::CH / 2;
      lds_dma16(is_v ? rv : rk, src[k],
                slot + (is_v ? uint32_t(RG::TILE) : 0u) + uint32_t(n % (RG::CH / 2)) * 1024u);
    }
  };

  f32x4 oacc[NB][VPL];
  // Softmax denominators: an extra PV MFMA with an all-ones A operand sums
  // the bf16 probabilities of each column over every key (all four rows of
  // lacc hold the same sum), instead of per-lane VALU adds and a cross-lane
  // reduction; the sum is of exactly the values the numerator used.
  f32x4 lacc[NB];
  float m_run[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m_run[nb] = -INFINITY;
    lacc[nb] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < VPL; ++b) oacc[nb][b] = f32x4{0, 0, 0, 0};
  }
  const int lim_min = base_lim + row0;  // smallest limit among this tile's rows

  // QK^T of one step's KT tiles (raw scores per tile, column block and
  // 16-token half).
  auto qk = [&](const uint8_t *step, f32x4 (&sc)[KT][NB][2]) {
#pragma unroll
    for (int h = 0; h < KT; ++h) {
      const uint8_t *kt = step + h * RG::SLOT;
      // One 16-token half at a time keeps 16 operand registers live. Rows r
      // and r + 16 share a swizzle key, so the second half is an immediate
      // offset from the first (one set of per-lane addresses, not two).
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        u32x4 ka[D / 32];
#pragma unroll
        for (int s = 0; s < D / 32; ++s)
          ka[s] = load_u32x4(kt + mt * 16 * D * 2 + RG::at(c, (D / 32) * g + s));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          f32x4 acc = {0, 0, 0, 0};
#pragma unroll
          for (int s = 0; s < D / 32; ++s) acc = mfma16x16x32(ka[s], qv[nb][s], acc);
          sc[h][nb][mt] = acc;
        }
      }
    }
  };
  // Mask, online softmax and PV of one step from its scores.
  auto finish = [&](const uint8_t *step, int t0, const f32x4 (&sc)[KT][NB][2]) {
    u32x4 pb[KT][NB];
    const bool masked = t0 + KT * kPrefillTile - 1 > lim_min;  // step crosses some column's limit
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      // Raw scores; the softmax scale (> 0) is applied inside the exponent's
      // fused multiply-add, and the max is taken before scaling.
      float x[KT * 8];
#pragma unroll
      for (int h = 0; h < KT; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[8 * h + r] = sc[h][nb][0][r];
          x[8 * h + 4 + r] = sc[h][nb][1][r];
        }
      if (masked) {
#pragma unroll
        for (int h = 0; h < KT; ++h)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            x[8 * h + j] = t0 + kPrefillTile * h + pf_tile_token(g, j) <= lim[nb] ? x[8 * h + j] : -INFINITY;
      }
      float tmax = x[0];
#pragma unroll
      for (int j = 1; j < KT * 8; ++j) tmax = fmaxf(tmax, x[j]);
      tmax = max_xor16(tmax);
      tmax = max_xor32(tmax) * p.scale_log2;
      if (__any(tmax > m_run[nb] + 8.0f)) {
        const float m_new = fmaxf(m_run[nb], tmax);
        const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run[nb] - m_new);
        m_run[nb] = m_new;
        lacc[nb] *= alpha;
#pragma unroll
        for (int b = 0; b < VPL; ++b) oacc[nb][b] *= alpha;
      }
      const float m_use = m_run[nb] == -INFINITY ? 0.0f : m_run[nb];
#pragma unroll
      for (int h = 0; h < KT; ++h) {
        float pr[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(__builtin_fmaf(x[8 * h + j], p.scale_log2, -m_use));
        pb[h][nb] = u32x4{pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                          pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7])};
      }
    }
    // V^T operand of PV MFMA b (rows = dims 16b .. 16b+15, k = the eight
    // tokens tile_token(g, 0..7) of the lane's P column) straight from LDS with
    // two transposing reads (ds_read_b64_tr_b16): in each 16-lane group, lane i
    // names 4 consecutive dims 16b + 4(i&3) of token tile_token(g, i>>2) (then
    // of tile_token(g, 4 + (i>>2))), and lane c receives dim 16b + c of those
    // four tokens.
    const int tr_dim = 4 * (c & 3);
    const int tr_row0 = pf_tile_token(g, c >> 2);  // pf_tile_token(g, 4 + (c >> 2)) = tr_row0 + 16
#pragma unroll
    for (int h = 0; h < KT; ++h) {
      const __attribute__((address_space(3))) char *vt_lds =
          (const __attribute__((address_space(3))) char *)(step + h * RG::SLOT + RG::TILE);
#pragma unroll
      for (int b = 0; b < VPL; ++b) {
        const int d = 16 * b + tr_dim;
        const uint32_t o0 = RG::at(tr_row0, d >> 3) + 2 * (d & 7);
        const uint32_t o1 = o0 + 16 * D * 2;  // row tr_row0 + 16: same swizzle key
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(vt_lds + o0));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(vt_lds + o1));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 a = u32x4{l2[0], l2[1], h2[0], h2[1]};
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) oacc[nb][b] = mfma16x16x32(a, pb[h][nb], oacc[nb][b]);
      }
      const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) lacc[nb] = mfma16x16x32(ones, pb[h][nb], lacc[nb]);
    }
  };

  // Ring: step si (tiles KT*si .. KT*si+KT-1) lives in step slot si % S, and
  // S-1 steps ahead are issued (every step issues KT*NIW loads per wave, dead
  // tiles included, so the wait counts are exact). The top of iteration si
  // waits for step si, and the barrier both publishes it and retires every
  // wave's reads of step si-1, whose slot then receives step si+S-1. The two
  // waves of a SIMD overlap one's MFMAs with the other's softmax. The loop is
  // unrolled by S so every slot offset is a compile-time constant (LDS
  // immediate offsets instead of per-step address arithmetic).
  static_assert(S >= 2, "one step resident, one in flight");
  constexpr int PER_STEP = KT * RG::NIW;  // direct-to-LDS loads per wave per step
  const int n_tiles = (range_end + kPrefillTile - 1) / kPrefillTile;
  const int n_steps = (n_tiles + KT - 1) / KT;
  auto issue_step = [&](int si) {
#pragma unroll
    for (int h = 0; h < KT; ++h) issue(si * KT + h);
  };
  if (n_steps > 0) {
#pragma unroll
    for (int i = 0; i < S - 1; ++i)
      if (i < n_steps) issue_step(i);
    f32x4 sc[KT][NB][2];
    for (int t = 0; t < n_steps; t += S) {
#pragma unroll
      for (int u = 0; u < S; ++u) {
        const int si = t + u;
        if (si < n_steps) {
          if (si + S - 2 < n_steps)  // steps si+1 .. si+S-2 may stay in flight
            lds_dma_wait<(S - 2) * PER_STEP>();
          else
            lds_dma_wait<0>();
          __syncthreads();
          if (si + S - 1 < n_steps) issue_step(si + S - 1);
          qk(ring + u * STEP, sc);
          finish(ring + u * STEP, si * KT * kPrefillTile, sc);
        }
      }
    }
  }

#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float l_tot = lacc[nb][0];
    if (!live[nb]) continue;
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t *op = p.out + (qrow[nb] * p.q_heads + head[nb]) * D + 4 * g;
    // PV MFMA b row 4g + r -> dim 16b + 4g + r
#pragma unroll
    for (int b = 0; b < VPL; ++b) {
      const f32x4 v = oacc[nb][b];
      *reinterpret_cast<u32x2 *>(op + 16 * b) =
          u32x2{pack_bf16x2(v[0] * inv, v[1] * inv), pack_bf16x2(v[2] * inv, v[3] * inv)};
    }
  }
}

namespace {

template <int D>
void launch_prefill(const PrefillParams &p, int grid, hipStream_t s) {
  const dim3 g(grid * p.kv_heads);
  switch (p.group) {
    case 1: varlen_prefill_kernel<D, 1><<<g, 64 * kPrefillWaves, 0, s>>>(p); break;
    case 2: varlen_prefill_kernel<D, 2><<<g, 64 * kPrefillWaves, 0, s>>>(p); break;
    case 4: varlen_prefill_kernel<D, 4><<<g, 64 * kPrefillWaves, 0, s>>>(p); break;
    case 8: varlen_prefill_kernel<D, 8><<<g, 64 * kPrefillWaves, 0, s>>>(p); break;
    default: varlen_prefill_kernel<D, 16><<<g, 64 * kPrefillWaves, 0, s>>>(p); break;
  }
}

uint64_t prefill_items_bound(int num_seqs, int total_q, int q_tile) {
  return uint64_t(total_q) / q_tile + uint64_t(num_seqs) + 1;
}

}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" uint64_t ifattn_varlen_prefill_workspace_size(int32_t num_seqs, int32_t total_q,
                                                         int32_t q_heads, int32_t head_dim,
                                                         int32_t max_kv_len) {
  if (num_seqs <= 0 || total_q <= 0 || q_heads <= 0 || head_dim <= 0 || max_kv_len <= 0) return 0;
  const uint64_t dec = split_k_workspace_bytes(num_seqs, q_heads, head_dim, max_kv_len);
  return align16(dec) + 16 + 4 * prefill_items_bound(num_seqs, total_q, 1);
}

extern "C" int32_t ifattn_varlen_prefill_bf16(const void *q, const void *k_cache, const void *v_cache,
                                              const int32_t *block_tables, int32_t table_stride,
                                              const int32_t *cu_seqlens_q, const int32_t *kv_lens,
                                              void *out, int32_t num_seqs, int32_t total_q,
                                              int32_t max_q_len, int32_t max_kv_len,
                                              int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                              int32_t block_size, int64_t num_blocks, float scale,
                                              void *workspace, uint64_t workspace_bytes,
                                              void *stream) {
  if (!q || !k_cache || !v_cache || !block_tables || !cu_seqlens_q || !kv_lens || !out)
    return fail(IFATTN_EINVAL, "varlen prefill: null pointer");
  if (num_seqs <= 0 || total_q <= 0 || max_q_len <= 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads)
    return fail(IFATTN_EINVAL, "varlen prefill: bad sequence or head counts");
  // Work items pack (sequence << 12 | query tile) into 32 bits.
  if (num_seqs >= (1 << 20))
    return fail(IFATTN_EINVAL, "varlen prefill: num_seqs must be below 2^20");
  const int group = q_heads / kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8 && group != 16)
    return fail(IFATTN_EINVAL, "varlen prefill: q_heads / kv_heads must be 1, 2, 4, 8 or 16");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IFATTN_EINVAL, "varlen prefill: head_dim must be 64, 128 or 256");
  if (block_size < 32 || (block_size & (block_size - 1)))
    return fail(IFATTN_EINVAL, "varlen prefill: block_size must be a power of two >= 32");
  if (max_kv_len <= 0 || max_kv_len > 262144 || num_blocks <= 0 || table_stride <= 0 ||
      int64_t(table_stride) * block_size < max_kv_len)
    return fail(IFATTN_EINVAL, "varlen prefill: max_kv_len in [1, 262144] covered by the tables");
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(IFATTN_EINVAL, "varlen prefill: q, out and caches must be 16-byte aligned");
  const uint64_t need = ifattn_varlen_prefill_workspace_size(num_seqs, total_q, q_heads, head_dim,
                                                             max_kv_len);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(IFATTN_EWORKSPACE, "varlen prefill: workspace missing, short or misaligned");
  hipStream_t s = static_cast<hipStream_t>(stream);

  // Decode rows: split-K decode kernels with the q-row indirection.
  DecodeParams d{};
  d.q = (const uint16_t *)q;
  d.k_cache = (const uint8_t *)k_cache;
  d.v_cache = (const uint8_t *)v_cache;
  d.block_tables = block_tables;
  d.seq_lens = kv_lens;
  d.out = (uint16_t *)out;
  d.cu_seqlens = cu_seqlens_q;
  d.num_blocks = num_blocks;
  d.num_seqs = num_seqs;
  d.q_heads = q_heads;
  d.kv_heads = kv_heads;
  d.group = group;
  d.table_stride = table_stride;
  d.block_size = block_size;
  d.max_context = max_kv_len;
  d.scale_log2 = scale * kLog2e;
  split_k_bind_workspace(d, workspace, q_heads, head_dim);

  PrefillParams p{};
  p.q = d.q;
  p.k_cache = d.k_cache;
  p.v_cache = d.v_cache;
  p.block_tables = block_tables;
  p.cu = cu_seqlens_q;
  p.kv_lens = kv_lens;
  p.out = d.out;
  {
    uint8_t *w = static_cast<uint8_t *>(workspace) +
                 align16(split_k_workspace_bytes(num_seqs, q_heads, head_dim, max_kv_len));
    p.n_items = reinterpret_cast<int32_t *>(w);
    p.items = reinterpret_cast<uint32_t *>(w + 16);
  }
  p.num_blocks = num_blocks;
  p.num_seqs = num_seqs;
  p.q_heads = q_heads;
  p.kv_heads = kv_heads;
  p.group = group;
  p.table_stride = table_stride;
  p.block_size = block_size;
  p.max_kv = max_kv_len;
  p.q_tile = prefill_q_tile(head_dim, group);
  p.scale_log2 = d.scale_log2;
  if (int64_t(max_q_len) > int64_t(4096) * p.q_tile)
    return fail(IFATTN_EINVAL, "varlen prefill: max_q_len above 4096 query tiles per sequence");
  p.max_q_len = max_q_len;
  const int grid = int(prefill_items_bound(num_seqs, total_q, p.q_tile));
  p.max_items = grid;

  launch_varlen_decode_rows(d, head_dim, s);
  prefill_plan_kernel<<<1, 1024, 0, s>>>(p);
  if (head_dim == 64) launch_prefill<64>(p, grid, s);
  else if (head_dim == 128) launch_prefill<128>(p, grid, s);
  else launch_prefill<256>(p, grid, s);
  return launch_status("varlen prefill");
}
