// Gated paged attention over per-token physical indices (the Qwen-shape decode
// operation of the reference session ABI, inferfabric_acl_paged_attention_prepare:
// native/include/inferfabric_acl.h:103-113, body native/src/inferfabric_acl.cpp:1343-1430).
//
// Per request b (batch <= 64), q head h (8 heads over 2 kv heads, kh = h / 4),
// head_dim 256, scale 1/16:
//   keys[append[b]] = k[b], values[append[b]] = v[b]           (the step's row)
//   s_j  = scale * q[b,h] . keys[table[b,j], kh] + mask[b,j]    j < context
//   out  = (sum_j softmax(s)_j values[table[b,j], kh]) * gate[b,h]
// The table holds one physical token row per context position (int64), the
// mask is fp32 and additive, and the gate buffer holds the gate the preceding
// operation produced (its sigmoid, inferfabric_acl.cpp:1335-1340), applied as a
// product. Accumulation is fp32 (scores, softmax, PV); the reference rounds
// scores and probabilities to bf16 between its ACLNN calls.
//
// Launches (one stream): plan (four workgroups per request, each over a
// quarter of its partitions of 64/128/256 positions, list the partitions
// holding a position whose mask is not -inf; the first also appends the step's
// rows); decode (persistent waves, eight per CU, take the live (partition, kv
// head) items round-robin); merge (per request and head, the live partitions'
// (m, l, O), normalised and gated). A one-partition context
// runs an append launch in place of the plan, and no merge.
//
// Decode item: the wave loads the partition's (mask, index) pairs and compacts
// the positions that can contribute (mask not -inf, index in range) into an
// LDS list by ballot. Live rows are processed 16 at a time, the next tile's
// rows loaded while this tile is computed: QK^T as MFMA 16x16x32 bf16 (A = the
// 16 rows' K straight from HBM, moved into the operand layout with ds_bpermute;
// B = the group's four q heads), the score tile feeding PV directly as the B
// operand of MFMA 16x16x16 (A = V rows), online softmax in the exp2 domain with
// lazy rescale.
#include "common.h"
#include "ifattn_internal.h"
#include "split_k.h"

namespace ifattn {
namespace {

constexpr int kD = 256;           // head_dim
constexpr int kGroup = 4;         // q heads per kv head
constexpr int kKvHeads = 2;
constexpr int kHeads = kGroup * kKvHeads;
constexpr int kRowBytes = kKvHeads * kD * 2;  // 1024 B per cache row
constexpr int kPart = 256;        // largest partition (context positions)
constexpr int kMinPart = 64;      // smallest partition
constexpr float kScale = 0.0625f; // 1/sqrt(256), inferfabric_acl.cpp:1400
// Cache-policy bits of the V row loads (2: nontemporal; rows are read once).
constexpr int kPolicy = 2;
// K reads half lines per instruction (the other half in the next one), which
// the nontemporal policy would fetch twice: default policy (measured 194
// against 227 us per operator).
constexpr int kKPolicy = 0;
// Growth of a head's running max (log2 units) tolerated before rescaling.
constexpr float kRescaleSlack = 8.0f;
// Decode waves per CU in the grid. At the kernel's 267 registers one wave per
// SIMD is resident, so four run at a time and the others start as they end;
// a grid of four per CU (all resident) measured the same (0.1355 ms per call
// at 64 requests over 32768 positions): the decode streams at about 6.6 TB/s
// either way.
constexpr int kWavesPerCu = 8;

struct GatedParams {
  const uint16_t *q, *gate;
  const uint8_t *keys, *values;
  const int64_t *table;
  const float *mask;
  uint16_t *out;
  uint16_t *part_o;  // [batch, parts, heads, D] bf16 O / l
  float *part_ml;  // [batch, parts, heads, 2]
  int32_t *live_parts;  // [batch, parts]: each request's partitions with a live position
  int32_t *live_count;  // [batch, kPlanSplit] (per chunk of partitions); both null for a one-partition context
  // The step's rows (appended by the plan kernel when there is one).
  const uint8_t *k_new, *v_new;
  const int64_t *append;
  uint8_t *keys_out, *values_out;
  int64_t slots;
  int context, parts, batch;
  int part, part_shift;  // partition length (64, 128 or 256) and its log2
};

// Lane c of a 16-lane row gets the value of lane (c + 8) % 16 (DPP row_ror:8).
__device__ __forceinline__ u32x4 row_ror8(u32x4 v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __builtin_amdgcn_update_dpp(0u, v[i], 0x128, 0xF, 0xF, false);
  return r;
}

// One (request b, kv head kvh, partition part) item, whose partials go to row
// `slot` of the request's partials (the partition's place in the request's
// live list); s_row / s_mask hold the wave's list of live positions.
__device__ __forceinline__ void gated_item(const GatedParams &p, int part, int slot, int kvh, int b,
                                           uint32_t *s_row, float *s_mask) {
  const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;
  const bool head_live = c < kGroup;
  const int head = kvh * kGroup + c;
  // Whole caches as buffers: rows are < 2^20, so byte offsets fit 32 bits.
  const auto rk = make_rsrc(p.keys + kvh * kD * 2, uint32_t(p.slots) * kRowBytes);
  const auto rv = make_rsrc(p.values + kvh * kD * 2, uint32_t(p.slots) * kRowBytes);
  const float sl2 = kScale * kLog2e;

  f32x4 oacc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) oacc[i] = f32x4{0, 0, 0, 0};
  float m_run = -INFINITY, l_run = 0.0f;

  const int t_begin = part * p.part;
  const int t_end = t_begin + p.part < p.context ? t_begin + p.part : p.context;
  const int64_t meta = int64_t(b) * p.context;
  // The partition's live positions (mask not -inf, row in range), in order, as
  // an LDS list: every lane's (mask, row) pairs (four at the largest partition)
  // are loaded before the first ballot.
  float mk[kPart / 64];
  int64_t rw[kPart / 64];
#pragma unroll
  for (int j = 0; j < kPart / 64; ++j) {
    const int t = t_begin + 64 * j + lane;
    mk[j] = t < t_end ? p.mask[meta + t] : -INFINITY;
    rw[j] = t < t_end ? p.table[meta + t] : 0;
  }
  int n_live = 0;
#pragma unroll
  for (int j = 0; j < kPart / 64; ++j) {
    const bool live = mk[j] != -INFINITY && rw[j] >= 0 && rw[j] < p.slots;
    const uint64_t ballot = __ballot(live);
    if (live) {
      const int at = n_live + __builtin_amdgcn_mbcnt_hi(uint32_t(ballot >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(uint32_t(ballot), 0u));
      s_row[at] = uint32_t(rw[j]);
      s_mask[at] = mk[j] * kLog2e;
    }
    n_live += __popcll(ballot);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");

  // q as the B operand of QK^T: k-step s, lane group g holds dims 32s + 8g .. +7.
  u32x4 qv[kD / 32];
  {
    const uint16_t *qr = p.q + (int64_t(b) * kHeads + (head_live ? head : 0)) * kD;
#pragma unroll
    for (int s = 0; s < kD / 32; ++s)
      qv[s] = head_live && n_live > 0 ? load_u32x4(qr + 32 * s + 8 * g) : u32x4{0, 0, 0, 0};
  }
  // Tile loads. V: lane (c, g) reads rows k0 + 4g + j, dims 8c .. 8c + 7 and
  // 128 + 8c .. 128 + 8c + 7, so 16 lanes read 256 contiguous bytes (whole
  // lines) of a row. Padded rows read past the buffer (zeros), so no stale
  // value (NaN or inf) can reach the scores or the accumulator, and a tile past
  // the list issues no memory traffic.
  auto row_off = [&](int e) { return e < n_live ? s_row[e] * uint32_t(kRowBytes) : 0xFFFFFC00u; };
  u32x4 kv[kD / 32];
  u32x4 vw[4][2];
  // K: instruction s reads dims 32s .. 32s + 31 (64 B) of the tile's 16 rows,
  // lane l taking 16-B chunk (l & 3) of row k0 + (l >> 2), so each quad of
  // lanes reads one contiguous 64-B piece; ds_bpermute then hands lane (c, g)
  // row c's chunk g, the MFMA A operand.
  const int k_src = 4 * (4 * c + g);  // byte address of the source lane
  auto load_k = [&](int k0) {
    const uint32_t krow = row_off(k0 + (lane >> 2)) + 16 * (lane & 3);
#pragma unroll
    for (int s = 0; s < kD / 32; ++s) kv[s] = buf_load_x4<kKPolicy>(rk, krow + 64 * s);
  };
  auto load_v = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t vrow = row_off(k0 + 4 * g + j);
      vw[j][0] = buf_load_x4<kPolicy>(rv, vrow + 16 * c);
      vw[j][1] = buf_load_x4<kPolicy>(rv, vrow + 256 + 16 * c);
    }
  };
  // Rolling prefetch: the next tile's K is issued as soon as QK^T has consumed
  // this tile's K, and its V once PV has consumed this tile's V, so a tile's
  // worth of rows stays in flight without a second set of registers.
  if (n_live > 0) {
    load_k(0);
    load_v(0);
  }
  for (int k0 = 0; k0 < n_live; k0 += 16) {
    f32x4 sacc = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < kD / 32; ++s) {
      u32x4 op;
#pragma unroll
      for (int i = 0; i < 4; ++i) op[i] = uint32_t(__builtin_amdgcn_ds_bpermute(k_src, int(kv[s][i])));
      sacc = mfma16x16x32(op, qv[s], sacc);
    }
    load_k(k0 + 16);
    // Lane (c, g) holds the scores of rows k0 + 4g + r for head c.
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = k0 + 4 * g + r;
      x[r] = sacc[r] * sl2 + (e < n_live ? s_mask[e] : -INFINITY);
    }
    float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    tmax = max_xor16(tmax);
    tmax = max_xor32(tmax);
    // Lazy rescale: the accumulators (held in AGPRs) are rescaled only when a
    // head's max grows by more than 2^8, so probabilities stay below 2^8
    // (exact enough for bf16 P) and most tiles skip the 64 multiplies.
    if (__any(tmax > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.0f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[i] *= alpha;
    }
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = m_run == -INFINITY ? 0.0f : fast_exp2(x[r] - m_run);
    l_run += (pr[0] + pr[1]) + (pr[2] + pr[3]);
    const u32x2 pb = u32x2{pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3])};
    // PV: MFMA d gives O^T row m <-> dim 8m + d (d < 8) or 128 + 8m + d - 8.
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      const int w = (d >> 1) & 3, h = d >> 3;
      const u32x2 a = (d & 1) ? u32x2{pack_hi16(vw[0][h][w], vw[1][h][w]), pack_hi16(vw[2][h][w], vw[3][h][w])}
                              : u32x2{pack_lo16(vw[0][h][w], vw[1][h][w]), pack_lo16(vw[2][h][w], vw[3][h][w])};
      oacc[d] = mfma16x16x16(a, pb, oacc[d]);
    }
    load_v(k0 + 16);
  }
  float l_tot = sum_xor16(l_run);
  l_tot = sum_xor32(l_tot);
  if (!head_live) return;
  // Lane (c, g) holds two 32-dim runs of head c: dims 128u + 32g + e (e < 32)
  // in oacc[8u + (e & 7)][e >> 3].
  auto elem = [&](int u, int e) { return oacc[8 * u + (e & 7)][e >> 3]; };
  if (p.parts == 1) {
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const int64_t o = (int64_t(b) * kHeads + head) * kD + 32 * g;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint16_t *gp = p.gate + o + 128 * u;
      uint16_t *op = p.out + o + 128 * u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // 8 dims per 16-byte store
        const u32x4 gw = load_u32x4(gp + 8 * k);
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e0 = 8 * k + 2 * i;
          w[i] = pack_bf16x2(elem(u, e0) * inv * bf16_bits_to_f32(gw[i] & 0xffffu),
                             elem(u, e0 + 1) * inv * bf16_bits_to_f32(gw[i] >> 16));
        }
        store_u32x4(op + 8 * k, w);
      }
    }
  } else {
    const int64_t prow = (int64_t(b) * p.parts + slot) * kHeads + head;
    if (g == 0) *reinterpret_cast<float2 *>(p.part_ml + prow * 2) = make_float2(m_run, l_tot);
    // O / l in bf16 (half the partial bytes; the merge weighs it by l).
    // Written even without a live row (zeros, m = -inf): the merge loads every
    // listed partition's O alongside its (m, l).
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t *po = p.part_o + prow * kD + 32 * g;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = pack_bf16x2(elem(u, 8 * k + 2 * i) * inv, elem(u, 8 * k + 2 * i + 1) * inv);
        store_u32x4(po + 128 * u + 8 * k, w);
      }
  }
}

// Live partitions of each request, in kPlanSplit chunks of pc = ceil(parts /
// kPlanSplit) partitions: workgroup (b, c) scans chunk c of mask row b
// (kPlanThreads threads, up to 32 positions each in flight) and lists, in
// order, the chunk's partitions with at least one position whose mask is not
// -inf at live_parts[b][c pc ..], their number at live_count[b][c]. Request
// b's list is the concatenation of its chunks' lists. One workgroup per
// request read its 128 KiB of mask at a CU's bandwidth: 6.7 us per call at 64
// requests over 32768 positions.
#ifndef IFATTN_GATED_PLAN_SPLIT
#define IFATTN_GATED_PLAN_SPLIT 4
#endif
constexpr int kPlanSplit = IFATTN_GATED_PLAN_SPLIT;
constexpr int kPlanThreads = 1024 / kPlanSplit;
constexpr int kMaxParts = 262144 / kMinPart;
__host__ __device__ __forceinline__ int plan_chunk(int parts) {
  return (parts + kPlanSplit - 1) / kPlanSplit;
}
__global__ __launch_bounds__(kPlanThreads) void gated_plan_kernel(GatedParams p) {
  constexpr int NW = kPlanThreads / 64;
  __shared__ uint32_t s_flag[kMaxParts / kPlanSplit + 1];
  __shared__ int s_wave[NW];
  const int b = blockIdx.x / kPlanSplit, c = blockIdx.x % kPlanSplit;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // Append request b's step row (K as 16-B pieces 0-63, V as 64-127) before
  // the decode launch reads the caches.
  for (int i = tid; c == 0 && i < 2 * (kRowBytes / 16); i += kPlanThreads) {
    const int64_t slot = p.append[b];
    const bool val = i >= kRowBytes / 16;
    const int cc = val ? i - kRowBytes / 16 : i;
    if (slot >= 0 && slot < p.slots)
      store_u32x4((val ? p.values_out : p.keys_out) + (slot * (kRowBytes / 16) + cc) * 16,
                  load_u32x4((val ? p.v_new : p.k_new) + (int64_t(b) * (kRowBytes / 16) + cc) * 16));
  }
  const int pc = plan_chunk(p.parts);
  const int p0 = c * pc;
  const int np = p.parts - p0 < pc ? (p.parts - p0 > 0 ? p.parts - p0 : 0) : pc;
  const int t_beg = p0 * p.part;
  const int t_len = np == 0 ? 0 : (p.context - t_beg < np * p.part ? p.context - t_beg : np * p.part);
  for (int i = tid; i < np; i += kPlanThreads) s_flag[i] = 0u;
  __syncthreads();
  // Unconditional 16-byte buffer loads, four positions a lane (zeros past the
  // chunk; the position test comes after the load), so all U loads of a
  // thread are in flight together: a quarter of the load instructions of one
  // position a lane.
  const auto rm = make_rsrc(p.mask + int64_t(b) * p.context + t_beg, uint32_t(t_len) * 4u);
  constexpr int U = 8;
  constexpr int kRound = kPlanThreads * 4;  // positions per load row
  const int lanes_per_part = p.part >> 2;  // 16, 32 or 64 lanes cover a partition
  for (int t0 = 0; t0 < t_len; t0 += U * kRound) {
    u32x4 x[U];
#pragma unroll
    for (int e = 0; e < U; ++e) x[e] = buf_load_x4(rm, uint32_t(t0 + e * kRound + tid * 4) * 4u);
    // A wave's 256 positions hold 256 / part whole partitions (chunks and
    // partitions are 64-aligned multiples of 64): lane 0 stores their flags
    // from the ballot, not one store per lane (same-address LDS stores from
    // many lanes serialise).
#pragma unroll
    for (int e = 0; e < U; ++e) {
      const int tb = t0 + e * kRound + tid * 4;
      bool live = false;
#pragma unroll
      for (int j = 0; j < 4; ++j) live |= tb + j < t_len && __uint_as_float(x[e][j]) != -INFINITY;
      const uint64_t bal = __ballot(live);
      if (lane == 0 && bal != 0) {
        const int wbase = t0 + e * kRound + w * 256;
        for (int q = 0; q < 64; q += lanes_per_part) {
          const uint64_t m = lanes_per_part == 64 ? ~uint64_t(0) : ((uint64_t(1) << lanes_per_part) - 1) << q;
          if (bal & m) s_flag[(wbase + 4 * q) >> p.part_shift] = 1u;
        }
      }
    }
  }
  __syncthreads();
  // Compaction in partition order: wave w owns chunk partitions 64w + kPlanThreads r + lane.
  int base = 0;
  int32_t *list = p.live_parts + int64_t(b) * p.parts + p0;
  for (int r0 = 0; r0 < np; r0 += kPlanThreads) {
    const int i = r0 + tid;
    const bool live = i < np && s_flag[i] != 0u;
    const uint64_t ballot = __ballot(live);
    if (lane == 0) s_wave[w] = __popcll(ballot);
    __syncthreads();
    int before = base;
    for (int u = 0; u < w; ++u) before += s_wave[u];
    if (live)
      list[before + __builtin_amdgcn_mbcnt_hi(uint32_t(ballot >> 32),
                                              __builtin_amdgcn_mbcnt_lo(uint32_t(ballot), 0u))] = p0 + i;
    for (int u = 0; u < NW; ++u) base += s_wave[u];
    __syncthreads();
  }
  if (tid == 0) p.live_count[b * kPlanSplit + c] = base;
}

// Position in request b's list row of its k-th live partition, given its
// chunks' counts n[0 .. kPlanSplit).
__device__ __forceinline__ int live_slot(int k, const int *n, int pc) {
  int c = 0;
#pragma unroll
  for (int u = 0; u < kPlanSplit - 1; ++u) {
    if (k >= n[u] && c == u) {
      k -= n[u];
      c = u + 1;
    }
  }
  return c * pc + k;
}

// Persistent waves (kWavesPerCu per CU) over the live items: item k is kv head
// k % 2 of the (k / 2)-th live partition in (request, partition) order, and
// wave w takes items w, w + grid, ... Items are whole partitions and nearly
// equal, so the static split is balanced, and the two kv heads of a partition
// (the halves of the same 1024-B rows) are read by neighbouring waves at about
// the same time. With one workgroup per (request, kv head, partition), most of
// them without a live position on ragged batches, the dispatcher kept a third
// of the wave slots busy and live items started up to 150 us late.
// A one-partition context (no plan) runs one wave per (request, kv head).
__global__ __launch_bounds__(64) void gated_decode_kernel(GatedParams p) {
  __shared__ uint32_t s_row[kPart];
  __shared__ float s_mask[kPart];
  if (!p.live_parts) {
    gated_item(p, 0, 0, int(blockIdx.x) % kKvHeads, int(blockIdx.x) / kKvHeads, s_row, s_mask);
    return;
  }
  const int lane = threadIdx.x;
  // Inclusive prefix of the live counts over requests (lane b = request b,
  // holding its chunks' counts).
  int nc[kPlanSplit];
#pragma unroll
  for (int u = 0; u < kPlanSplit; ++u) nc[u] = lane < p.batch ? p.live_count[lane * kPlanSplit + u] : 0;
  int cnt = 0;
#pragma unroll
  for (int u = 0; u < kPlanSplit; ++u) cnt += nc[u];
  const int pc = plan_chunk(p.parts);
  int incl = cnt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  const int total = kKvHeads * __builtin_amdgcn_readlane(incl, 63);
  for (int k = blockIdx.x; k < total; k += gridDim.x) {
    const int idx = k / kKvHeads;  // live partition index over all requests
    const int b = __popcll(__ballot(incl <= idx));
    const int j = idx - (__builtin_amdgcn_readlane(incl, b) - __builtin_amdgcn_readlane(cnt, b));
    int nb[kPlanSplit];
#pragma unroll
    for (int u = 0; u < kPlanSplit; ++u) nb[u] = __builtin_amdgcn_readlane(nc[u], b);
    const int part = p.live_parts[int64_t(b) * p.parts + live_slot(j, nb, pc)];
    gated_item(p, part, j, k % kKvHeads, b, s_row, s_mask);
    // The next item rewrites the list this one read.
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  }
}

// One workgroup of kMergeWaves waves per (request, head): combine the live
// partitions' (m, l, O) in one online pass, normalise, apply the gate. Wave w
// takes partial rows w, w + kMergeWaves, ... (the decode wrote the request's
// live partitions' partials to rows 0 .. n-1 in partition order), so each
// round of eight partials ((m, l) with O, lane l owning dims 4l .. 4l + 3)
// costs one memory round trip, after the one that loads the chunk counts and
// the gate. A partition whose rows were all out of range has m = -inf, weight
// 0 and zero O. The waves' (m, l, O) meet in LDS. Eight waves per
// workgroup (7.2 us per call) launched faster than sixteen (8.4 us) and four
// (8.1 us) on the benchmark's 512 (request, head) pairs.
constexpr int kMergeWaves = 8;
__global__ __launch_bounds__(64 * kMergeWaves) void gated_merge_kernel(GatedParams p) {
  __shared__ float s_m[kMergeWaves], s_l[kMergeWaves];
  __shared__ f32x4 s_o[kMergeWaves][64];
  const int b = blockIdx.x, h = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t o_out = (int64_t(b) * kHeads + h) * kD + 4 * lane;
  const u32x2 gw = *reinterpret_cast<const u32x2 *>(p.gate + o_out);
  int n = 0;
#pragma unroll
  for (int u = 0; u < kPlanSplit; ++u) n += p.live_count[b * kPlanSplit + u];
  const int64_t base = int64_t(b) * p.parts * kHeads + h;
  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 acc = f32x4{0, 0, 0, 0};
  constexpr int U = 8;
  for (int k0 = w; k0 < n; k0 += kMergeWaves * 64) {
    const int cnt = (n - k0 + kMergeWaves - 1) / kMergeWaves < 64 ? (n - k0 + kMergeWaves - 1) / kMergeWaves : 64;
    for (int u0 = 0; u0 < cnt; u0 += U) {
      float2 ml[U];
      f32x4 o[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = u0 + u;
        const int row = i < cnt ? k0 + kMergeWaves * i : 0;
        const int64_t r = base + int64_t(row) * kHeads;
        ml[u] = *reinterpret_cast<const float2 *>(p.part_ml + r * 2);
        const u32x2 ob = *reinterpret_cast<const u32x2 *>(p.part_o + r * kD + 4 * lane);
        o[u] = f32x4{bf16_bits_to_f32(ob[0] & 0xffffu), bf16_bits_to_f32(ob[0] >> 16),
                     bf16_bits_to_f32(ob[1] & 0xffffu), bf16_bits_to_f32(ob[1] >> 16)};
        if (i >= cnt) {
          ml[u] = make_float2(-INFINITY, 0.0f);
          o[u] = f32x4{0, 0, 0, 0};
        }
      }
      float mx = m_run;
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, ml[u].x);
      if (mx == -INFINITY) continue;
      const float sc = m_run == -INFINITY ? 0.0f : fast_exp2(m_run - mx);
      m_run = mx;
      l_run *= sc;
      acc *= sc;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float wt = ml[u].x == -INFINITY ? 0.0f : fast_exp2(ml[u].x - mx);
        l_run += wt * ml[u].y;
        acc += (wt * ml[u].y) * o[u];
      }
    }
  }
  s_o[w][lane] = acc;
  if (lane == 0) {
    s_m[w] = m_run;
    s_l[w] = l_run;
  }
  __syncthreads();
  if (w != 0) return;
  float mmax = s_m[0];
#pragma unroll
  for (int u = 1; u < kMergeWaves; ++u) mmax = fmaxf(mmax, s_m[u]);
  acc = f32x4{0, 0, 0, 0};
  float lsum = 0.0f;
  if (mmax != -INFINITY) {
#pragma unroll
    for (int u = 0; u < kMergeWaves; ++u) {
      const float wt = s_m[u] == -INFINITY ? 0.0f : fast_exp2(s_m[u] - mmax);
      acc += wt * s_o[u][lane];
      lsum += wt * s_l[u];
    }
  }
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  *reinterpret_cast<u32x2 *>(p.out + o_out) =
      u32x2{pack_bf16x2(acc[0] * inv * bf16_bits_to_f32(gw[0] & 0xffffu),
                        acc[1] * inv * bf16_bits_to_f32(gw[0] >> 16)),
            pack_bf16x2(acc[2] * inv * bf16_bits_to_f32(gw[1] & 0xffffu),
                        acc[3] * inv * bf16_bits_to_f32(gw[1] >> 16))};
}

// The step's K/V rows: keys[append[b]] = k[b] (1024 B), the same for values.
__global__ __launch_bounds__(256) void gated_append_kernel(const uint8_t *k, const uint8_t *v,
                                                           uint8_t *keys, uint8_t *values,
                                                           const int64_t *append, int batch,
                                                           int64_t slots) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte vector
  constexpr int kVecs = kRowBytes / 16;
  if (i >= batch * kVecs * 2) return;
  const bool val = i >= batch * kVecs;
  const int j = val ? i - batch * kVecs : i;
  const int r = j / kVecs, c = j % kVecs;
  const int64_t slot = append[r];
  if (slot < 0 || slot >= slots) return;
  store_u32x4((val ? values : keys) + (slot * kVecs + c) * 16,
              load_u32x4((val ? v : k) + (int64_t(r) * kVecs + c) * 16));
}

// Partition length: 256 positions when the batch's partitions give at least
// two items per wave slot of a full MI355X (256 CUs x kWavesPerCu), else 128,
// else 64, so that small batches over long contexts still spread over the chip
// (a wave's items run one after another, one tile latency at a time). A
// function of (batch, context) only, so the workspace size follows it.
int part_len(int64_t batch, int64_t context) {
  constexpr int64_t kTarget = 2 * 256 * kWavesPerCu;
  for (int len = kPart; len > kMinPart; len /= 2)
    if (batch * ((context + len - 1) / len) * kKvHeads >= kTarget) return len;
  return kMinPart;
}
int parts_for(int64_t batch, int64_t context) {
  const int len = part_len(batch, context);
  return int((context + len - 1) / len);
}

}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" uint64_t ifattn_gated_paged_attention_workspace_size(int64_t batch, int64_t context) {
  if (batch <= 0 || context <= 0) return 0;
  const uint64_t parts = uint64_t(parts_for(batch, context));
  if (parts == 1) return 16;
  // Partials (bf16 O / l, then fp32 (m, l)), the live partition lists and their counts.
  return uint64_t(batch) * parts * (kHeads * (kD * sizeof(uint16_t) + 2 * sizeof(float)) + sizeof(int32_t)) +
         align16(uint64_t(batch) * kPlanSplit * sizeof(int32_t));
}

extern "C" int32_t ifattn_gated_paged_attention_bf16(
    const void *q, const void *k, const void *v, const void *gate, void *keys, void *values,
    const int64_t *append, const int64_t *table, const float *mask, void *out, int64_t batch,
    int64_t slots, int64_t context, void *workspace, uint64_t workspace_bytes, void *stream) {
  if (batch <= 0 || batch > 64 || slots <= 0 || slots > 1048576 || context <= 0 ||
      context > 262144)
    return fail(IFATTN_EINVAL, "gated paged attention: batch 1..64, slots 1..2^20, context 1..262144");
  if (!q || !k || !v || !gate || !keys || !values || !append || !table || !mask || !out)
    return fail(IFATTN_EINVAL, "gated paged attention: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(gate) || !aligned16(keys) ||
      !aligned16(values) || !aligned16(out) || !aligned8(append) || !aligned8(table) ||
      !aligned4(mask))
    return fail(IFATTN_EINVAL, "gated paged attention: misaligned tensor");
  const uint64_t need = ifattn_gated_paged_attention_workspace_size(batch, context);
  GatedParams p{};
  p.q = static_cast<const uint16_t *>(q);
  p.gate = static_cast<const uint16_t *>(gate);
  p.keys = static_cast<const uint8_t *>(keys);
  p.values = static_cast<const uint8_t *>(values);
  p.table = table;
  p.mask = mask;
  p.out = static_cast<uint16_t *>(out);
  p.slots = slots;
  p.context = int(context);
  p.parts = parts_for(batch, context);
  p.part = part_len(batch, context);
  p.part_shift = __builtin_ctz(unsigned(p.part));
  if (p.parts > 1) {
    if (!workspace || workspace_bytes < need || !aligned16(workspace))
      return fail(IFATTN_EWORKSPACE, "gated paged attention: workspace missing, short or misaligned");
    p.part_o = static_cast<uint16_t *>(workspace);
    p.part_ml = reinterpret_cast<float *>(p.part_o + uint64_t(batch) * p.parts * kHeads * kD);
    p.live_parts = reinterpret_cast<int32_t *>(p.part_ml + uint64_t(batch) * p.parts * kHeads * 2);
    p.live_count = p.live_parts + uint64_t(batch) * p.parts;  // [batch, kPlanSplit]
  }
  p.batch = int(batch);
  hipStream_t s = static_cast<hipStream_t>(stream);
  p.k_new = static_cast<const uint8_t *>(k);
  p.v_new = static_cast<const uint8_t *>(v);
  p.append = append;
  p.keys_out = static_cast<uint8_t *>(keys);
  p.values_out = static_cast<uint8_t *>(values);
  const int items = p.parts * kKvHeads * int(batch);
  const int waves = device_cus() * kWavesPerCu;
  if (p.live_parts) {
    gated_plan_kernel<<<unsigned(batch) * kPlanSplit, kPlanThreads, 0, s>>>(p);  // appends the step's rows too
  } else {
    const int vecs = int(batch) * (kRowBytes / 16) * 2;
    gated_append_kernel<<<(vecs + 255) / 256, 256, 0, s>>>(p.k_new, p.v_new, p.keys_out,
                                                            p.values_out, append, int(batch), slots);
  }
  gated_decode_kernel<<<p.live_parts ? (items < waves ? items : waves) : items, 64, 0, s>>>(p);
  if (p.parts > 1) gated_merge_kernel<<<dim3(unsigned(batch), kHeads), 64 * kMergeWaves, 0, s>>>(p);
  return launch_status("gated paged attention");
}
