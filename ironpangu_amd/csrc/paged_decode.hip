// Ragged paged GQA decode for gfx950 (bf16 and C8 int8 caches).
//
// Computes, per sequence b, q head h, kv head kh = h / group:
//   s_j = scale * q[b,h] . K[slot(b,j), kh],  j < len_b
//   out[b,h] = sum_j softmax(s)_j * V[slot(b,j), kh]
// with fp32 accumulation: the paged GQA operator of
// native/src/inferfabric_acl.cpp:1377-1428 (Embedding gather, matmul, fp32
// softmax, matmul) whose CPU oracle is crates/inferfabric-cli/src/npu_probe/attention.rs:221-253
// (grouping kh = h / (q_heads/kv_heads) at :226). slot(b,j) = table[b][j/bs]*bs + j%bs
// (native/src/page_binding.h:56-59).
//
// Work decomposition (one launch, grid = seqs x partitions x kv-head groups):
//  * a workgroup owns a `part_tokens` slice of one sequence; each of its waves
//    owns one kv head, so the two waves of a 2-kv-head model stream the two
//    halves of the same 512-byte cache rows at the same time;
//  * a wave walks 32-token tiles. QK^T is one MFMA 16x16x32 bf16 per (16 tokens,
//    32 dims): A = K rows straight from HBM (16 B per lane), B = the group's q
//    heads (n = head, zero-padded to 16). The score tile lands with lane
//    (c = lane%16, g = lane/16) holding tokens 4g..4g+3 and 16+4g..16+4g+3 of
//    head c, so P never leaves registers: it is exactly the B operand of the
//    PV MFMA once those eight tokens are declared the lane's k-slots;
//  * PV is O^T = V^T P^T: the A operand needs eight tokens of one dimension,
//    fetched as dword gathers (two adjacent dims) and split into even/odd dims
//    with v_perm, so V is never staged or transposed through LDS;
//  * online softmax in the exp2 domain; max/sum across the four lane groups by
//    two xor shuffles per tile;
//  * sequences longer than one partition write (m, l, unnormalised O) partials
//    and a second kernel merges them (split-K); single-partition sequences
//    write bf16 output directly.
//  * the next tile's loads are issued before the current tile's math (register
//    double buffering), keeping ~16 KiB in flight per wave.
// C8: K/V int8 with an fp32 scale per (token, kv head). int8 -> bf16 is exact,
// so QK^T runs on the integer codes and the K scale multiplies the score; the
// V scale is folded into the probability before the PV MFMA.
#include "common.h"
#include "ifattn_internal.h"

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
  float *part_o;   // [num_seqs, max_parts, q_heads, D]
  float *part_ml;  // [num_seqs, max_parts, q_heads, 2]
  int64_t num_blocks;
  int num_seqs, q_heads, kv_heads, group, table_stride, block_size, max_context, max_parts,
      part_tokens;
  float scale_log2;  // softmax scale * log2(e)
};

constexpr int kDecodeWaves = 2;
constexpr int kTile = 32;

// Token of k-slot j (0..7) for lane group g within a 32-token tile.
__device__ __forceinline__ int tile_token(int g, int j) {
  return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
}

template <int D, bool C8>
struct TileRegs {
  // K A-operands: [mt][kstep] (bf16: 16 B each; C8: 8 B each stored in .xy)
  u32x4 k[2][D / 32];
  // V dwords: [slice][token j]; bf16: dims 32*sl+2c..+1; C8: dims 64*sl+4c..+3
  uint32_t v[C8 ? D / 64 : D / 32][8];
  float ks[8], vs[8];  // C8 scales for the lane's 8 tokens
};

template <int D, bool C8>
__device__ __forceinline__ void load_tile(TileRegs<D, C8> &t, const DecodeParams &p, int seq,
                                          int kvh, int t0, int t_end, int c, int g) {
  const int bs = p.block_size;
  int blk = p.block_tables[int64_t(seq) * p.table_stride + t0 / bs];
  blk = blk < 0 ? 0 : (blk >= p.num_blocks ? int(p.num_blocks - 1) : blk);
  const int64_t base = int64_t(blk) * bs + (t0 & (bs - 1));
  constexpr int EB = C8 ? 1 : 2;  // element bytes
  const int64_t row_bytes = int64_t(p.kv_heads) * D * EB;
  const uint8_t *krow0 = p.k_cache + (base * p.kv_heads + kvh) * D * EB;
  const uint8_t *vrow0 = p.v_cache + (base * p.kv_heads + kvh) * D * EB;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const uint8_t *kr = krow0 + int64_t(16 * mt + c) * row_bytes + (D / 4) * g * EB;
    if constexpr (!C8) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) t.k[mt][s] = load_u32x4(kr + 16 * s);
    } else {
#pragma unroll
      for (int s = 0; s < D / 32; s += 2) {
        u32x4 w = load_u32x4(kr + 8 * s);
        t.k[mt][s] = u32x4{w[0], w[1], 0u, 0u};
        t.k[mt][s + 1] = u32x4{w[2], w[3], 0u, 0u};
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int x = tile_token(g, j);
    const bool live = t0 + x < t_end;
    const uint8_t *vr = vrow0 + int64_t(x) * row_bytes;
    if constexpr (!C8) {
#pragma unroll
      for (int sl = 0; sl < D / 32; ++sl) {
        uint32_t w = *reinterpret_cast<const uint32_t *>(vr + (32 * sl + 2 * c) * 2);
        t.v[sl][j] = live ? w : 0u;
      }
    } else {
#pragma unroll
      for (int sl = 0; sl < D / 64; ++sl) {
        uint32_t w = *reinterpret_cast<const uint32_t *>(vr + 64 * sl + 4 * c);
        t.v[sl][j] = live ? w : 0u;
      }
      const int64_t srow = (base + x) * p.kv_heads + kvh;
      t.ks[j] = p.k_scale[srow];
      t.vs[j] = live ? p.v_scale[srow] : 0.0f;
    }
  }
}

// int8 codes (4 per dword) -> exact bf16 values, 8 codes -> 4 packed dwords.
__device__ __forceinline__ uint32_t i8pair_to_bf16x2(int a, int b) {
  // Small integers are exact in fp32 and in bf16 (|x| <= 128 < 2^8), so the
  // high half of the fp32 pattern is the bf16 value.
  return perm_b32(__float_as_uint(float(b)), __float_as_uint(float(a)), 0x07060302u);
}
__device__ __forceinline__ u32x4 i8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  const int32_t l = int32_t(lo), h = int32_t(hi);
  return u32x4{i8pair_to_bf16x2((l << 24) >> 24, (l << 16) >> 24),
               i8pair_to_bf16x2((l << 8) >> 24, l >> 24),
               i8pair_to_bf16x2((h << 24) >> 24, (h << 16) >> 24),
               i8pair_to_bf16x2((h << 8) >> 24, h >> 24)};
}
__device__ __forceinline__ int i8_at(uint32_t w, int b) {
  return (int32_t(w) << (24 - 8 * b)) >> 24;
}

template <int D, bool C8>
__global__ __launch_bounds__(64 * kDecodeWaves) void paged_decode_kernel(DecodeParams p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kvh = blockIdx.z * kDecodeWaves + wave;
  if (kvh >= p.kv_heads) return;
  const int seq = blockIdx.x, part = blockIdx.y;
  int len = p.seq_lens[seq];
  len = len > p.max_context ? p.max_context : len;
  const int PT = p.part_tokens;
  const int nparts = len > 0 ? (len + PT - 1) / PT : 1;
  if (part >= nparts) return;
  const int c = lane & 15, g = lane >> 4;
  const int head = kvh * p.group + c;
  const bool head_live = c < p.group;

  if (len <= 0) {  // no visible key: defined zero output
    if (head_live) {
#pragma unroll
      for (int d0 = 8 * g; d0 < D; d0 += 32)
        store_u32x4(p.out + (int64_t(seq) * p.q_heads + head) * D + d0, u32x4{0, 0, 0, 0});
    }
    return;
  }

  // B operand of QK^T: q[head][(D/4)*g + 8*s + e], zero for padded heads.
  u32x4 qv[D / 32];
  {
    const uint16_t *qp = p.q + (int64_t(seq) * p.q_heads + (head_live ? head : 0)) * D + (D / 4) * g;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) qv[s] = head_live ? load_u32x4(qp + 8 * s) : u32x4{0, 0, 0, 0};
  }

  constexpr int NV = D / 16;  // PV MFMAs per tile (each yields 16 dims x 16 heads)
  f32x4 oacc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) oacc[i] = f32x4{0, 0, 0, 0};
  float m_run = -INFINITY, l_run = 0.0f;

  const int t_begin = part * PT;
  const int t_end = t_begin + PT < len ? t_begin + PT : len;

  auto compute = [&](const TileRegs<D, C8> &t, int t0) {
    f32x4 s0 = {0, 0, 0, 0}, s1 = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      u32x4 a0, a1;
      if constexpr (!C8) {
        a0 = t.k[0][s];
        a1 = t.k[1][s];
      } else {
        a0 = i8x8_to_bf16x8(t.k[0][s][0], t.k[0][s][1]);
        a1 = i8x8_to_bf16x8(t.k[1][s][0], t.k[1][s][1]);
      }
      s0 = mfma16x16x32(a0, qv[s], s0);
      s1 = mfma16x16x32(a1, qv[s], s1);
    }
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s0[r];
      x[4 + r] = s1[r];
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = x[j] * p.scale_log2;
      if constexpr (C8) v *= t.ks[j];
      v = (t0 + tile_token(g, j) < t_end) ? v : -INFINITY;
      x[j] = v;
      tmax = fmaxf(tmax, v);
    }
    tmax = wave_max_xor(tmax, 16);
    tmax = wave_max_xor(tmax, 32);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float pr[8];
    float psum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pr[j] = exp2f(x[j] - m_new);
    }
    u32x4 pb;
    if constexpr (!C8) {
      // The MFMA consumes bf16 probabilities; normalise by the same rounded values.
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pr[j] = bf16_bits_to_f32(f32_to_bf16_bits(pr[j]));
        psum += pr[j];
      }
      pb = u32x4{pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                 pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7])};
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) psum += pr[j];
      pb = u32x4{pack_bf16x2(pr[0] * t.vs[0], pr[1] * t.vs[1]),
                 pack_bf16x2(pr[2] * t.vs[2], pr[3] * t.vs[3]),
                 pack_bf16x2(pr[4] * t.vs[4], pr[5] * t.vs[5]),
                 pack_bf16x2(pr[6] * t.vs[6], pr[7] * t.vs[7])};
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < NV; ++i) oacc[i] *= alpha;
    if constexpr (!C8) {
#pragma unroll
      for (int sl = 0; sl < D / 32; ++sl) {
        const uint32_t *w = t.v[sl];
        u32x4 ev = {pack_lo16(w[0], w[1]), pack_lo16(w[2], w[3]), pack_lo16(w[4], w[5]),
                    pack_lo16(w[6], w[7])};
        u32x4 od = {pack_hi16(w[0], w[1]), pack_hi16(w[2], w[3]), pack_hi16(w[4], w[5]),
                    pack_hi16(w[6], w[7])};
        oacc[2 * sl] = mfma16x16x32(ev, pb, oacc[2 * sl]);
        oacc[2 * sl + 1] = mfma16x16x32(od, pb, oacc[2 * sl + 1]);
      }
    } else {
#pragma unroll
      for (int sl = 0; sl < D / 64; ++sl) {
        const uint32_t *w = t.v[sl];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          u32x4 a = {i8pair_to_bf16x2(i8_at(w[0], b), i8_at(w[1], b)),
                     i8pair_to_bf16x2(i8_at(w[2], b), i8_at(w[3], b)),
                     i8pair_to_bf16x2(i8_at(w[4], b), i8_at(w[5], b)),
                     i8pair_to_bf16x2(i8_at(w[6], b), i8_at(w[7], b))};
          oacc[4 * sl + b] = mfma16x16x32(a, pb, oacc[4 * sl + b]);
        }
      }
    }
  };

  TileRegs<D, C8> ta, tb;
  int t0 = t_begin;
  load_tile<D, C8>(ta, p, seq, kvh, t0, t_end, c, g);
  while (true) {
    int tn = t0 + kTile < t_end ? t0 + kTile : t0;
    load_tile<D, C8>(tb, p, seq, kvh, tn, t_end, c, g);
    compute(ta, t0);
    t0 += kTile;
    if (t0 >= t_end) break;
    tn = t0 + kTile < t_end ? t0 + kTile : t0;
    load_tile<D, C8>(ta, p, seq, kvh, tn, t_end, c, g);
    compute(tb, t0);
    t0 += kTile;
    if (t0 >= t_end) break;
  }

  float l_tot = wave_sum_xor(l_run, 16);
  l_tot = wave_sum_xor(l_tot, 32);
  if (!head_live) return;

  // Lane owns dims d0..d0+7 of head c for each 32-dim slice (bf16 layout) or
  // dims 64*sl + 4*(4g+r) + b (C8 layout).
  float o[D / 4];
  if constexpr (!C8) {
#pragma unroll
    for (int sl = 0; sl < D / 32; ++sl)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o[8 * sl + 2 * r] = oacc[2 * sl][r];
        o[8 * sl + 2 * r + 1] = oacc[2 * sl + 1][r];
      }
  } else {
    // slice sl (64 dims): lane holds rows m = 4g + r of MFMA b -> dim 64sl + 4(4g+r) + b,
    // i.e. 16 contiguous dims 64sl + 16g .. +16.
#pragma unroll
    for (int sl = 0; sl < D / 64; ++sl)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int b = 0; b < 4; ++b) o[16 * sl + 4 * r + b] = oacc[4 * sl + b][r];
  }
  // Chunk k of 8 values starts at dim: bf16 32*k + 8g; C8 64*(k/2) + 16g + 8*(k%2).
  auto chunk_dim = [&](int k) { return C8 ? 64 * (k >> 1) + 16 * g + 8 * (k & 1) : 32 * k + 8 * g; };
  if (nparts == 1) {
    const float inv = 1.0f / l_tot;
    uint16_t *op = p.out + (int64_t(seq) * p.q_heads + head) * D;
#pragma unroll
    for (int k = 0; k < D / 32; ++k) {
      const float *v = o + 8 * k;
      store_u32x4(op + chunk_dim(k), u32x4{pack_bf16x2(v[0] * inv, v[1] * inv),
                                           pack_bf16x2(v[2] * inv, v[3] * inv),
                                           pack_bf16x2(v[4] * inv, v[5] * inv),
                                           pack_bf16x2(v[6] * inv, v[7] * inv)});
    }
  } else {
    const int64_t prow = (int64_t(seq) * p.max_parts + part) * p.q_heads + head;
    float *po = p.part_o + prow * D;
#pragma unroll
    for (int k = 0; k < D / 32; ++k) {
      const float *v = o + 8 * k;
      *reinterpret_cast<f32x4 *>(po + chunk_dim(k)) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4 *>(po + chunk_dim(k) + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
    if (g == 0) *reinterpret_cast<float2 *>(p.part_ml + prow * 2) = make_float2(m_run, l_tot);
  }
}

// Merge split-K partials: one workgroup per sequence, 4 output dims per thread.
template <int D>
__global__ __launch_bounds__(256) void paged_decode_reduce_kernel(DecodeParams p) {
  const int seq = blockIdx.x;
  int len = p.seq_lens[seq];
  len = len > p.max_context ? p.max_context : len;
  const int nparts = len > 0 ? (len + p.part_tokens - 1) / p.part_tokens : 1;
  if (nparts <= 1) return;
  const int per_head = D / 4;
  for (int idx = threadIdx.x; idx < p.q_heads * per_head; idx += blockDim.x) {
    const int h = idx / per_head, d = (idx - h * per_head) * 4;
    const int64_t row0 = int64_t(seq) * p.max_parts * p.q_heads + h;
    float mmax = -INFINITY;
    for (int k = 0; k < nparts; ++k) mmax = fmaxf(mmax, p.part_ml[(row0 + int64_t(k) * p.q_heads) * 2]);
    float lsum = 0.0f;
    f32x4 acc = {0, 0, 0, 0};
    for (int k = 0; k < nparts; ++k) {
      const int64_t row = row0 + int64_t(k) * p.q_heads;
      const float2 ml = *reinterpret_cast<const float2 *>(p.part_ml + row * 2);
      const float w = exp2f(ml.x - mmax);
      lsum += w * ml.y;
      acc += w * *reinterpret_cast<const f32x4 *>(p.part_o + row * D + d);
    }
    const float inv = 1.0f / lsum;
    uint16_t *op = p.out + (int64_t(seq) * p.q_heads + h) * D + d;
    *reinterpret_cast<u32x2 *>(op) =
        u32x2{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
  }
}

namespace {
constexpr int kPartTokens = 256;

int max_parts_for(int max_context) { return (max_context + kPartTokens - 1) / kPartTokens; }

template <int D, bool C8>
void launch_decode(const DecodeParams &p, hipStream_t s) {
  dim3 grid(p.num_seqs, p.max_parts, (p.kv_heads + kDecodeWaves - 1) / kDecodeWaves);
  paged_decode_kernel<D, C8><<<grid, 64 * kDecodeWaves, 0, s>>>(p);
  if (p.max_parts > 1) paged_decode_reduce_kernel<D><<<p.num_seqs, 256, 0, s>>>(p);
}

int32_t decode_common(bool c8, const void *q, const void *k_cache, const void *v_cache,
                      const void *k_scale, const void *v_scale, const int32_t *block_tables,
                      int32_t table_stride, const int32_t *seq_lens, void *out, int32_t num_seqs,
                      int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t block_size,
                      int64_t num_blocks, int32_t max_context, float scale, void *workspace,
                      uint64_t workspace_bytes, void *stream) {
  if (!q || !k_cache || !v_cache || !block_tables || !seq_lens || !out ||
      (c8 && (!k_scale || !v_scale)))
    return fail(IFATTN_EINVAL, "paged decode: null pointer");
  if (num_seqs <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads ||
      q_heads / kv_heads > 16)
    return fail(IFATTN_EINVAL, "paged decode: need q_heads = group * kv_heads with group <= 16");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IFATTN_EINVAL, "paged decode: head_dim must be 64, 128 or 256");
  if (block_size < 32 || (block_size & (block_size - 1)))
    return fail(IFATTN_EINVAL, "paged decode: block_size must be a power of two >= 32");
  if (max_context <= 0 || num_blocks <= 0 || table_stride <= 0 ||
      int64_t(table_stride) * block_size < max_context)
    return fail(IFATTN_EINVAL, "paged decode: table_stride * block_size must cover max_context");
  if (num_seqs > 65535 * 64)
    return fail(IFATTN_EINVAL, "paged decode: too many sequences");
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(IFATTN_EINVAL, "paged decode: q, out and caches must be 16-byte aligned");
  DecodeParams p{};
  p.q = (const uint16_t *)q;
  p.k_cache = (const uint8_t *)k_cache;
  p.v_cache = (const uint8_t *)v_cache;
  p.k_scale = (const float *)k_scale;
  p.v_scale = (const float *)v_scale;
  p.block_tables = block_tables;
  p.seq_lens = seq_lens;
  p.out = (uint16_t *)out;
  p.num_blocks = num_blocks;
  p.num_seqs = num_seqs;
  p.q_heads = q_heads;
  p.kv_heads = kv_heads;
  p.group = q_heads / kv_heads;
  p.table_stride = table_stride;
  p.block_size = block_size;
  p.max_context = max_context;
  p.part_tokens = kPartTokens;
  p.max_parts = max_parts_for(max_context);
  p.scale_log2 = scale * kLog2e;
  if (p.max_parts > 65535) return fail(IFATTN_EINVAL, "paged decode: max_context too large");
  if (p.max_parts > 1) {
    const uint64_t need = ifattn_paged_decode_workspace_size(num_seqs, q_heads, head_dim, max_context);
    if (!workspace || workspace_bytes < need || !aligned16(workspace))
      return fail(IFATTN_EWORKSPACE, "paged decode: workspace missing, short or misaligned");
    p.part_o = (float *)workspace;
    p.part_ml = p.part_o + int64_t(num_seqs) * p.max_parts * q_heads * head_dim;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (c8) {
    if (head_dim == 64) launch_decode<64, true>(p, s);
    else if (head_dim == 128) launch_decode<128, true>(p, s);
    else launch_decode<256, true>(p, s);
  } else {
    if (head_dim == 64) launch_decode<64, false>(p, s);
    else if (head_dim == 128) launch_decode<128, false>(p, s);
    else launch_decode<256, false>(p, s);
  }
  return launch_status("paged decode");
}
}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" uint64_t ifattn_paged_decode_workspace_size(int32_t num_seqs, int32_t q_heads,
                                                       int32_t head_dim, int32_t max_context) {
  if (num_seqs <= 0 || q_heads <= 0 || head_dim <= 0 || max_context <= 0) return 0;
  const uint64_t parts = uint64_t(max_parts_for(max_context));
  if (parts <= 1) return 0;
  return uint64_t(num_seqs) * parts * q_heads * (uint64_t(head_dim) + 2) * sizeof(float);
}

extern "C" int32_t ifattn_paged_decode_bf16(const void *q, const void *k_cache, const void *v_cache,
                                            const int32_t *block_tables, int32_t table_stride,
                                            const int32_t *seq_lens, void *out, int32_t num_seqs,
                                            int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                            int32_t block_size, int64_t num_blocks,
                                            int32_t max_context, float scale, void *workspace,
                                            uint64_t workspace_bytes, void *stream) {
  return decode_common(false, q, k_cache, v_cache, nullptr, nullptr, block_tables, table_stride,
                       seq_lens, out, num_seqs, q_heads, kv_heads, head_dim, block_size, num_blocks,
                       max_context, scale, workspace, workspace_bytes, stream);
}

extern "C" int32_t ifattn_paged_decode_c8(const void *q, const void *k_cache, const void *v_cache,
                                          const void *k_scale, const void *v_scale,
                                          const int32_t *block_tables, int32_t table_stride,
                                          const int32_t *seq_lens, void *out, int32_t num_seqs,
                                          int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                          int32_t block_size, int64_t num_blocks,
                                          int32_t max_context, float scale, void *workspace,
                                          uint64_t workspace_bytes, void *stream) {
  return decode_common(true, q, k_cache, v_cache, k_scale, v_scale, block_tables, table_stride,
                       seq_lens, out, num_seqs, q_heads, kv_heads, head_dim, block_size, num_blocks,
                       max_context, scale, workspace, workspace_bytes, stream);
}
