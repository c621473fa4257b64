// Packed-MLA latent-cache decode for gfx950 (bf16 rows and packed C8 rows).
//
// Per sequence b and head h (all heads share one cache row per token):
//   s_j = scale * q[b,h,0:576] . row_j[0:576]
//   out[b,h] = sum_j softmax(s)_j * row_j[0:512]
// fp32 accumulation. This is the latent attention of the reference's MLA
// decoder (native/src/token_executor.h:841-906) whose CPU oracles are
// native/probes/packed_cache_probe.cpp:47-66 (C8) and
// native/probes/sliding_window_probe.cpp:144-163 (bf16), here without learned
// sinks or a window. C8 rows are {int8 latent[512], bf16 rope[64], f32 scale[4]}
// (docs/packed-mla-cache.md:27-43); latent d dequantizes as int8 * scale[d/128]
// (packed_cache_probe.cpp:57).
//
// Decomposition: a workgroup of four waves owns a (sequence, partition) item
// from the shared split-K queue. Wave w owns latent dims [128w, 128w+128) for
// both QK^T and PV (K and V are the same bytes), waves 0 and 1 also take one
// 32-dim step of the rope part. Partial 32-token score tiles are summed across
// the waves through LDS (double-buffered, one barrier per tile); every wave then
// runs the same online softmax. With C8 the wave's 128 dims are exactly one
// scale tile, so the per-token tile scale multiplies the wave's partial score
// and is folded into its probabilities for PV — dequantization stays in
// registers. MFMA 16x16x32 bf16 with all 16 heads in the N dimension.
#include "common.h"
#include "ifattn_internal.h"
#include "split_k.h"

namespace ifattn {

constexpr int kMlaWaves = 4;
constexpr int kMlaTile = 32;

template <bool C8>
struct MlaRow {
  static constexpr uint32_t BYTES = C8 ? 656 : 1152;
  // Direct-to-LDS loads per wave per tile: 32 rows = 2304 (bf16) / 1312 (C8) 16-byte chunks.
  static constexpr int NI = C8 ? 6 : 9;
  static constexpr uint32_t SLOT = 4 * NI * 1024;  // LDS bytes per staged tile
#ifndef IFATTN_MLA_C8_STAGES
#define IFATTN_MLA_C8_STAGES 6
#endif
#ifndef IFATTN_MLA_WGS
#define IFATTN_MLA_WGS 1
#endif
#ifndef IFATTN_MLA_BF16_STAGES
#define IFATTN_MLA_BF16_STAGES 4
#endif
  static constexpr int STAGES = C8 ? IFATTN_MLA_C8_STAGES : IFATTN_MLA_BF16_STAGES;
  // LDS byte of 16-byte chunk j of tile row r. bf16 rows (1152 B, a multiple of
  // 128) XOR the chunk index with the row's low 3 bits so the 16 rows that one
  // K read touches spread over the banks; C8 rows (656 B) are not swizzled.
  static __device__ __forceinline__ uint32_t chunk(uint32_t r, uint32_t j) {
    return C8 ? r * BYTES + 16 * j : r * BYTES + 16 * (j ^ (r & 7));
  }
};
static_assert(MlaRow<false>::SLOT * MlaRow<false>::STAGES + 4 * 64 * 32 <= 160 * 1024, "LDS");
static_assert(MlaRow<true>::SLOT * MlaRow<true>::STAGES + 4 * 64 * 32 <= 160 * 1024, "LDS");
static_assert(MlaRow<false>::NI * 4 * 64 == 32 * 72, "bf16 tile = 2304 chunks");
static_assert(MlaRow<true>::NI * 4 * 64 >= 32 * 41, "C8 tile fits the slot");

constexpr int kMlaLds =
    MlaRow<false>::SLOT * MlaRow<false>::STAGES > MlaRow<true>::SLOT * MlaRow<true>::STAGES
        ? MlaRow<false>::SLOT * MlaRow<false>::STAGES
        : MlaRow<true>::SLOT * MlaRow<true>::STAGES;

__device__ __forceinline__ int mla_tile_token(int g, int j) {
  return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
}

__device__ __forceinline__ uint32_t mla_i8pair(int a, int b) {
  return perm_b32(__float_as_uint(float(b)), __float_as_uint(float(a)), 0x07060302u);
}
__device__ __forceinline__ int mla_i8(uint32_t x, int b) { return (int32_t(x) << (24 - 8 * b)) >> 24; }
__device__ __forceinline__ u32x4 mla_i8x8(uint32_t lo, uint32_t hi) {
  return u32x4{mla_i8pair(mla_i8(lo, 0), mla_i8(lo, 1)), mla_i8pair(mla_i8(lo, 2), mla_i8(lo, 3)),
               mla_i8pair(mla_i8(hi, 0), mla_i8(hi, 1)), mla_i8pair(mla_i8(hi, 2), mla_i8(hi, 3))};
}

// One (sequence, partition) item. The partition's 32-token tiles are copied
// HBM -> LDS once by direct-to-LDS loads shared by the four waves (each tile is
// 32 consecutive rows of one block) through a ring of R::STAGES slots; every
// wave then reads its K operand (tokens in rows) and its V operand (dims in
// rows) from the same LDS bytes.
template <bool C8>
__device__ __forceinline__ void mla_item(const DecodeParams &p, const uint8_t *cache,
                                         uint8_t *ring, float (*xbuf)[8], int seq, int part,
                                         int w, int lane) {
  using R = MlaRow<C8>;
  constexpr int S = R::STAGES;
  const int len = clamp_len(p, seq);
  const int PT = p.part_tokens;
  const int nparts = parts_of(len, PT);
  const int c = lane & 15, g = lane >> 4;
  const bool head_live = c < p.q_heads;
  constexpr int DV = 512;

  if (len <= 0) {
    if (head_live) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        store_u32x4(p.out + (int64_t(seq) * p.q_heads + c) * DV + 128 * w + 32 * g + 8 * k,
                    u32x4{0, 0, 0, 0});
    }
    return;
  }

  // Q operand: latent dims 128w + 32s + 8g (s < 4), rope dims 32w + 8g (w < 2).
  u32x4 qv[5];
  {
    const uint16_t *qp = p.q + (int64_t(seq) * p.q_heads + (head_live ? c : 0)) * 576;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qv[s] = head_live ? load_u32x4(qp + 128 * w + 32 * s + 8 * g) : u32x4{0, 0, 0, 0};
    qv[4] = (head_live && w < 2) ? load_u32x4(qp + 512 + 32 * w + 8 * g) : u32x4{0, 0, 0, 0};
  }

  const int t_begin = part * PT;
  const int t_end = t_begin + PT < len ? t_begin + PT : len;
  const int n_tiles = (t_end - t_begin + kMlaTile - 1) / kMlaTile;
  int lane_blocks;
  {
    const int first = t_begin / p.block_size;
    const int nblk = (t_end - 1) / p.block_size - first + 1;
    int b = lane < nblk ? p.block_tables[int64_t(seq) * p.table_stride + first + lane] : 0;
    lane_blocks = b < 0 ? 0 : (b >= p.num_blocks ? int(p.num_blocks - 1) : b);
  }
  // Source offset (within a tile) of the 16-byte chunk each lane moves per load.
  uint32_t src[R::NI];
#pragma unroll
  for (int k = 0; k < R::NI; ++k) {
    const uint32_t l = uint32_t((k * 4 + w) * 64 + lane);
    if constexpr (C8) {
      src[k] = 16 * l;  // chunks past the 32 rows fall outside the tile's extent
    } else {
      const uint32_t r = l / 72, jj = l % 72;
      src[k] = r * R::BYTES + 16 * (jj ^ (r & 7));
    }
  }
  const uint32_t ring_base = lds_addr(ring);
  auto issue = [&](int ti) {
    const int t0 = t_begin + ti * kMlaTile;
    const int bs = p.block_size;
    const int blk = __builtin_amdgcn_readlane(lane_blocks, (t0 - (t_begin & ~(bs - 1))) / bs);
    const int64_t tok0 = int64_t(blk) * bs + (t0 & (bs - 1));
    const int n_live = t_end - t0 < kMlaTile ? t_end - t0 : kMlaTile;
    const u32x4 rc = raw_rsrc(cache + tok0 * R::BYTES, uint32_t(n_live) * R::BYTES);
    const uint32_t dst = ring_base + uint32_t(ti % S) * R::SLOT + uint32_t(w) * 1024;
#pragma unroll
    for (int k = 0; k < R::NI; ++k) lds_dma16(rc, src[k], dst + uint32_t(k) * 4096);
  };

  f32x4 oacc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) oacc[i] = f32x4{0, 0, 0, 0};
  float m_run = -INFINITY, l_run = 0.0f;

  auto compute = [&](const uint8_t *tile, int t0) {
    // K operand: token 16mt + c, latent dims 128w + 32s + 8g (+ rope dims 32(w&1) + 8g).
    u32x4 k[2][5];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const uint32_t r = uint32_t(16 * mt + c);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if constexpr (C8) {
          const u32x2 x = *reinterpret_cast<const u32x2 *>(tile + r * R::BYTES + 128 * w + 32 * s + 8 * g);
          k[mt][s] = u32x4{x[0], x[1], 0u, 0u};
        } else {
          k[mt][s] = load_u32x4(tile + R::chunk(r, uint32_t(16 * w + 4 * s + g)));
        }
      }
      if (w < 2) {
        if constexpr (C8)
          k[mt][4] = load_u32x4(tile + r * R::BYTES + 512 + 64 * (w & 1) + 16 * g);
        else
          k[mt][4] = load_u32x4(tile + R::chunk(r, uint32_t(64 + 4 * (w & 1) + g)));
      } else {
        k[mt][4] = u32x4{0, 0, 0, 0};
      }
    }
    // V operand rows: token tile_token(g, j), latent dims 128w + 8c .. +8.
    u32x4 v[8];
    float sk[C8 ? 8 : 1];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t r = uint32_t(mla_tile_token(g, j));
      if constexpr (C8) {
        const u32x2 x = *reinterpret_cast<const u32x2 *>(tile + r * R::BYTES + 128 * w + 8 * c);
        v[j] = u32x4{x[0], x[1], 0u, 0u};
        sk[j] = *reinterpret_cast<const float *>(tile + r * R::BYTES + 640 + 4 * w);
      } else {
        v[j] = load_u32x4(tile + R::chunk(r, uint32_t(16 * w + c)));
      }
    }

    f32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if constexpr (C8) {
        a0 = mfma16x16x32(mla_i8x8(k[0][s][0], k[0][s][1]), qv[s], a0);
        a1 = mfma16x16x32(mla_i8x8(k[1][s][0], k[1][s][1]), qv[s], a1);
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
      for (int j = 0; j < 8; ++j) part_s[j] *= sk[j];
    }
    if (w < 2) {
      f32x4 r0 = mfma16x16x32(k[0][4], qv[4], f32x4{0, 0, 0, 0});
      f32x4 r1 = mfma16x16x32(k[1][4], qv[4], f32x4{0, 0, 0, 0});
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        part_s[r] += r0[r];
        part_s[4 + r] += r1[r];
      }
    }
    // Sum the four waves' partial scores. The buffer is free again: every wave
    // finished reading it before the barrier that starts this tile.
    *reinterpret_cast<f32x4 *>(&xbuf[w * 64 + lane][0]) = f32x4{part_s[0], part_s[1], part_s[2], part_s[3]};
    *reinterpret_cast<f32x4 *>(&xbuf[w * 64 + lane][4]) = f32x4{part_s[4], part_s[5], part_s[6], part_s[7]};
    __syncthreads();
    float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < kMlaWaves; ++u) {
      const f32x4 lo = *reinterpret_cast<const f32x4 *>(&xbuf[u * 64 + lane][0]);
      const f32x4 hi = *reinterpret_cast<const f32x4 *>(&xbuf[u * 64 + lane][4]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] += lo[r];
        x[4 + r] += hi[r];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] *= p.scale_log2;
    if (t_end - t0 < kMlaTile) {
      const int n_live = t_end - t0;
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = mla_tile_token(g, j) < n_live ? x[j] : -INFINITY;
    }
    float tmax = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                       fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    tmax = wave_max_xor(tmax, 16);
    tmax = wave_max_xor(tmax, 32);
    if (__any(tmax > m_run + 8.0f)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) oacc[i] *= alpha;
    }
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(x[j] - m_run);
    l_run += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
    if constexpr (C8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) pr[j] *= sk[j];
    }
    const u32x4 pb = {pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                      pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7])};
#pragma unroll
    for (int b = 0; b < 8; ++b) {
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
      oacc[b] = mfma16x16x32(a, pb, oacc[b]);
    }
  };

  // Ring: tile ti lives in slot ti % S. Tiles 0..S-2 are issued up front; the
  // top of iteration ti waits for tile ti (S-2 newer tiles may stay in flight,
  // fewer near the end), then a barrier both publishes it and retires every
  // wave's reads of tile ti-1, whose slot receives tile ti+S-1.
#pragma unroll
  for (int i = 0; i < S - 1; ++i)
    if (i < n_tiles) issue(i);
  for (int ti = 0; ti < n_tiles; ++ti) {
    if (ti + S - 2 < n_tiles)
      lds_dma_wait<(S - 2) * R::NI>();
    else
      lds_dma_wait<0>();
#ifndef IFATTN_EXP_NOBARRIER
    __syncthreads();
#endif
    if (ti + S - 1 < n_tiles) issue(ti + S - 1);
#ifndef IFATTN_EXP_NOCOMPUTE
    compute(ring + (ti % S) * R::SLOT, t_begin + ti * kMlaTile);
#endif
  }

  float l_tot = wave_sum_xor(l_run, 16);
  l_tot = wave_sum_xor(l_tot, 32);
  if (!head_live) return;
  // Lane holds rows m = 4g + r of MFMA b -> dim 128w + 8(4g + r) + b.
  float ov[32];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < 8; ++b) ov[8 * r + b] = oacc[b][r];
  const int d0 = 128 * w + 32 * g;
  if (nparts == 1) {
    const float inv = 1.0f / l_tot;
    uint16_t *op = p.out + (int64_t(seq) * p.q_heads + c) * DV + d0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float *v = ov + 8 * k;
      store_u32x4(op + 8 * k, u32x4{pack_bf16x2(v[0] * inv, v[1] * inv),
                                    pack_bf16x2(v[2] * inv, v[3] * inv),
                                    pack_bf16x2(v[4] * inv, v[5] * inv),
                                    pack_bf16x2(v[6] * inv, v[7] * inv)});
    }
  } else {
    const int64_t prow = (int64_t(seq) * p.max_parts + part) * p.q_heads + c;
    float *po = p.part_o + prow * DV + d0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      *reinterpret_cast<f32x4 *>(po + 4 * k) = f32x4{ov[4 * k], ov[4 * k + 1], ov[4 * k + 2], ov[4 * k + 3]};
    if (w == 0 && g == 0) *reinterpret_cast<float2 *>(p.part_ml + prow * 2) = make_float2(m_run, l_tot);
  }
}

template <bool C8>
__global__ __launch_bounds__(64 * kMlaWaves, IFATTN_MLA_WGS) void mla_decode_kernel(DecodeParams p) {
  __shared__ __align__(16) uint8_t ring[kMlaLds];
  __shared__ __align__(16) float xbuf[kMlaWaves * 64][8];
  // The item index travels through the score buffer, idle between items.
  int *item_slot = reinterpret_cast<int *>(&xbuf[0][0]);
  const int lane = threadIdx.x & 63;
  const int w = uniform(int(threadIdx.x >> 6));
  const uint8_t *cache = p.k_cache;
  while (true) {
    __syncthreads();
    if (threadIdx.x == 0) *item_slot = atomicAdd(p.queue, 1);
    __syncthreads();
    const int it = uniform(*item_slot);
    __syncthreads();
    if (it >= p.queue[1]) break;
    const uint32_t e = uniform(p.items[it]);
    const int seq = int(e >> 12);
    mla_item<C8>(p, cache, ring, xbuf, seq, int(e & 0xfffu), w, lane);
  }
}

namespace {

int32_t mla_common(bool c8, const void *q, const void *cache, const int32_t *block_tables,
                   int32_t table_stride, const int32_t *seq_lens, void *out, int32_t num_seqs,
                   int32_t heads, int32_t block_size, int64_t num_blocks, int32_t max_context,
                   float scale, void *workspace, uint64_t workspace_bytes, void *stream) {
  if (!q || !cache || !block_tables || !seq_lens || !out)
    return fail(IFATTN_EINVAL, "mla decode: null pointer");
  if (num_seqs <= 0 || heads <= 0 || heads > 16)
    return fail(IFATTN_EINVAL, "mla decode: 1..16 heads per call");
  if (block_size < 32 || (block_size & (block_size - 1)))
    return fail(IFATTN_EINVAL, "mla decode: block_size must be a power of two >= 32");
  if (max_context <= 0 || num_blocks <= 0 || table_stride <= 0 ||
      int64_t(table_stride) * block_size < max_context)
    return fail(IFATTN_EINVAL, "mla decode: table_stride * block_size must cover max_context");
  if (!aligned16(q) || !aligned16(out) || !aligned16(cache))
    return fail(IFATTN_EINVAL, "mla decode: q, out and cache must be 16-byte aligned");
  if (uint64_t(block_size) * (c8 ? 656 : 1152) * 1 > (1ull << 31))
    return fail(IFATTN_EINVAL, "mla decode: block too large");
  DecodeParams p{};
  p.q = (const uint16_t *)q;
  p.k_cache = (const uint8_t *)cache;
  p.block_tables = block_tables;
  p.seq_lens = seq_lens;
  p.out = (uint16_t *)out;
  p.num_blocks = num_blocks;
  p.num_seqs = num_seqs;
  p.q_heads = heads;
  p.kv_heads = 1;
  p.group = heads;
  p.table_stride = table_stride;
  p.block_size = block_size;
  p.max_context = max_context;
  p.part_tokens = part_tokens();
  p.max_parts = max_parts_for(max_context);
  p.scale_log2 = scale * kLog2e;
  if (p.max_parts > 4096) return fail(IFATTN_EINVAL, "mla decode: max_context above 1M tokens");
  if (p.part_tokens > 64 * block_size)
    return fail(IFATTN_EINVAL, "mla decode: partition spans more than 64 blocks");
  const uint64_t need = ifattn_mla_decode_workspace_size(num_seqs, heads, max_context);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(IFATTN_EWORKSPACE, "mla decode: workspace missing, short or misaligned");
  split_k_bind_workspace(p, workspace, heads, 512);
  hipStream_t s = static_cast<hipStream_t>(stream);
  launch_prologue(p, RowWrite{}, s);
  if (c8)
    mla_decode_kernel<true><<<device_cus() * IFATTN_MLA_WGS, 64 * kMlaWaves, 0, s>>>(p);
  else
    mla_decode_kernel<false><<<device_cus() * IFATTN_MLA_WGS, 64 * kMlaWaves, 0, s>>>(p);
  launch_merge<512>(p, s);
  return launch_status("mla decode");
}

}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" uint64_t ifattn_mla_decode_workspace_size(int32_t num_seqs, int32_t heads,
                                                     int32_t max_context) {
  if (num_seqs <= 0 || heads <= 0 || max_context <= 0) return 0;
  return split_k_workspace_bytes(num_seqs, heads, 512, max_context);
}

extern "C" int32_t ifattn_mla_decode_bf16(const void *q, const void *cache,
                                          const int32_t *block_tables, int32_t table_stride,
                                          const int32_t *seq_lens, void *out, int32_t num_seqs,
                                          int32_t heads, int32_t block_size, int64_t num_blocks,
                                          int32_t max_context, float scale, void *workspace,
                                          uint64_t workspace_bytes, void *stream) {
  return mla_common(false, q, cache, block_tables, table_stride, seq_lens, out, num_seqs, heads,
                    block_size, num_blocks, max_context, scale, workspace, workspace_bytes, stream);
}

extern "C" int32_t ifattn_mla_decode_c8(const void *q, const void *cache,
                                        const int32_t *block_tables, int32_t table_stride,
                                        const int32_t *seq_lens, void *out, int32_t num_seqs,
                                        int32_t heads, int32_t block_size, int64_t num_blocks,
                                        int32_t max_context, float scale, void *workspace,
                                        uint64_t workspace_bytes, void *stream) {
  return mla_common(true, q, cache, block_tables, table_stride, seq_lens, out, num_seqs, heads,
                    block_size, num_blocks, max_context, scale, workspace, workspace_bytes, stream);
}
