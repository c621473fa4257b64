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
// Work decomposition: a prologue kernel cuts the call's tokens (plus a start
// cost per sequence) into equal contiguous shares, one per worker; a
// persistent grid (two workgroups per CU) walks them:
//  * a workgroup owns the tile range of one share within one sequence at a
//    time; each of its waves owns one kv head, so the two waves of a
//    2-kv-head model stream the two halves of the same 512-byte cache rows at
//    the same time;
//  * a wave walks 32-token tiles (16-token tiles at head_dim 256). QK^T is one
//    MFMA 16x16x32 bf16 per (16 tokens, 32 dims): A = K rows straight from HBM
//    (16 B per lane; bf16 loads cover whole 128-B lines and one DPP lane
//    rotation puts each chunk at its token's lane), B = the group's q heads
//    (n = head, zero-padded to 16). K and V loads stream nontemporally.
//    The score tile lands with lane (c = lane%16, g = lane/16) holding tokens
//    4g..4g+3 (and 16+4g..16+4g+3) of head c, so P never leaves registers: it
//    is exactly the B operand of the PV MFMA once those tokens are declared
//    the lane's k-slots;
//  * PV is O^T = V^T P^T: the A operand needs the lane's tokens of one
//    dimension, fetched as 16-byte token loads and split into even/odd dims
//    with v_perm, so V is never staged or transposed through LDS;
//  * online softmax in the exp2 domain with lazy rescaling; max/sum across
//    the four lane groups by permlane swaps;
//  * sequences spread over several shares write (m, l, unnormalised O)
//    partials and a second kernel merges them (split-K); a sequence inside one
//    share writes bf16 output directly.
//  * a register ring of decode_stages() tiles keeps the next tiles' loads in
//    flight while the current tile is reduced.
// C8: K/V int8 with an fp32 scale per (token, kv head). QK^T runs on the
// integer codes as fp16 (biased by kI8Bias, exact; q scaled into fp16 range
// and kI8Bias * sum(q) subtracted from each score) and the K scale multiplies
// the score; V codes become exact bf16 and the V scale is folded into the
// probability before the PV MFMA.
#include <cstdlib>
#include <mutex>

#include "common.h"
#include "ifattn_internal.h"
#include "split_k.h"

namespace ifattn {

// Waves per workgroup = min(kv_heads, max_decode_waves(D)), one kv head each;
// a workgroup never needs more than one wave per SIMD, so each wave may use
// the whole register file (deep prefetch ring).
constexpr int max_decode_waves(int) { return 4; }
// Tokens per tile: 32, or 16 at head_dim 256, where a 32-token tile takes 128
// registers and only two would fit; 16-token tiles keep four in the ring.
constexpr int decode_tile(int d) { return d > 128 ? 16 : 32; }
#ifndef IFATTN_DECODE_STAGES
#define IFATTN_DECODE_STAGES 3
#endif
// V loads stream with the nontemporal cache policy: each V load instruction
// covers whole 128-B lines (16 lanes x 16 B of one row), which no other load
// touches again (config-2 decode 5.58 -> 5.95 TB/s, C8 5.2 -> 5.5). With
// half-line K loads (one instruction reading half of each line of 16 rows, the
// next the other half) the nontemporal policy measured 16% slower, because the
// second half is then fetched again; bf16 K therefore uses the whole-line
// scheme below and streams nontemporally too (kKPolicy), while C8 K keeps
// half-line loads with the default policy.
constexpr int kVPolicy = 2;
// K loads cover whole lines too: instruction (h, L) of a 16-token row block
// reads line L (128 B) of the kv head's slice of rows 8h .. 8h+7, lane (c, g)
// taking 16-B chunk g + 4(c >> 3) of row (c & 7) + 8h, and streams
// nontemporally. The MFMA operand (lane (c, g) = token c) of chunk column
// g (+4) is then the lane's own value or that of lane c ^ 8 (DPP row_ror:8), so
// a k-step's dims are a fixed permutation of the head dims, matched in q
// (config-2 decode 5.95 -> 6.06 TB/s). bf16 caches with head_dim >= 64 (a kv
// head's slice of a row is then whole lines); C8 caches keep the
// half-line loads (the same scheme measured 3% slower on config 4).
template <int D, bool C8>
constexpr bool k_lines() { return !C8 && D * 2 >= 128; }
constexpr int kKPolicy = 2;
// Lane c of a 16-lane row gets the value of lane (c + 8) % 16 (DPP row_ror:8).
__device__ __forceinline__ u32x4 row_ror8(u32x4 v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __builtin_amdgcn_update_dpp(0u, v[i], 0x128, 0xF, 0xF, false);
  return r;
}
// Tile buffers per wave (stages-1 tiles prefetched).
template <int D>
constexpr int decode_stages() { return D > 128 ? 4 : IFATTN_DECODE_STAGES; }

// Token of k-slot j (0..7) for lane group g within a 32-token tile (j < 4 in a
// 16-token tile).
__device__ __forceinline__ int tile_token(int g, int j) {
  return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
}

// V row slice held by one lane: dims [c*VPL, (c+1)*VPL) of each of its eight
// tokens (VPL = D/16 values), fetched with 16-byte loads.
template <int D, bool C8>
struct VSlice {
  static constexpr int VPL = D / 16;                  // values per lane per token
  static constexpr int BYTES = VPL * (C8 ? 1 : 2);    // 4..32 bytes
  static constexpr int DW = BYTES / 4;                // dwords per token
};

template <int D, bool C8>
struct TileRegs {
  static constexpr int TT = decode_tile(D);  // tokens per tile
  static constexpr int MT = TT / 16;         // 16-token row blocks of QK^T
  static constexpr int TPL = TT / 4;         // V tokens per lane
  // K A-operands: [mt][kstep] (bf16: 16 B each; C8: 8 B each stored in .xy)
  u32x4 k[MT][D / 32];
  // V: [token j][dword]: dims c*VPL .. c*VPL+VPL-1 of token tile_token(g, j)
  uint32_t v[TPL][VSlice<D, C8>::DW];
  float ks[C8 ? TPL : 1], vs[C8 ? TPL : 1];  // C8 scales for the lane's tokens
};

// Per-lane byte offsets inside a tile; identical for every tile, so
// they are computed once per range and the per-tile cost is one scalar
// buffer descriptor per cache.
struct LaneOffsets {
  uint32_t k[2];  // K loads of row block mt (see k_lines)
  uint32_t v[8];  // row tile_token(g, j), dims c*D/16 ..
  uint32_t sc[8]; // C8 scale of row tile_token(g, j)
};

// The partition's block ids are fetched once per item, one per lane
// (`lane_blocks`; a second register holds ids 64..127 with 16-token pages); a
// tile reads its id with v_readlane instead of a dependent scalar load in front
// of every tile's loads.
struct LaneBlocks {
  int lo, hi;
};
template <bool SP>
__device__ __forceinline__ int block_at(const LaneBlocks &lb, int i) {  // i wave-uniform
  if constexpr (SP) return i < 64 ? __builtin_amdgcn_readlane(lb.lo, i) : __builtin_amdgcn_readlane(lb.hi, i - 64);
  return __builtin_amdgcn_readlane(lb.lo, i);
}

// SP (16-token pages): a 32-token tile spans two pages, so its rows 0..15 and
// 16..31 come through one buffer descriptor each; the lane offsets of the
// second half are then relative to the second page (see decode_item).
template <int D, bool C8, bool SP>
__device__ __forceinline__ void load_tile(TileRegs<D, C8> &t, const DecodeParams &p,
                                          const LaneBlocks &lane_blocks, int win0, int kvh,
                                          int t0, int t_end, const LaneOffsets &o) {
  constexpr int EB = C8 ? 1 : 2;  // element bytes
  constexpr int TT = TileRegs<D, C8>::TT;
  constexpr bool SPLIT = SP && TT == 32;
  const int bs = p.block_size;
  const int idx = t0 / bs - win0;  // lane of the tile's block id in the window
  const int blk = block_at<SP>(lane_blocks, idx);
  const int64_t tok0 = int64_t(blk) * bs + (t0 & (bs - 1));
  const int n_live = t_end - t0 < TT ? t_end - t0 : TT;
  const uint32_t row_bytes = uint32_t(p.kv_heads) * D * EB;
  // Rows past the live tokens read as zero (buffer range check), which masks
  // V of a partial tile without any per-lane selects.
  const int n0 = SPLIT && n_live > 16 ? 16 : n_live;
  const uint32_t extent = uint32_t(n0 - 1) * row_bytes + D * EB;
  const int64_t first = (tok0 * p.kv_heads + kvh) * D * EB;
  const auto rk0 = make_rsrc(p.k_cache + first, extent);
  const auto rv0 = make_rsrc(p.v_cache + first, extent);
  // Second page of a split tile (an empty range when no row of it is live).
  auto rk1 = rk0, rv1 = rv0;
  int64_t tok1 = tok0;
  uint32_t extent1 = 0;
  if constexpr (SPLIT) {
    tok1 = int64_t(block_at<SP>(lane_blocks, idx + 1)) * bs;
    extent1 = n_live > 16 ? uint32_t(n_live - 17) * row_bytes + D * EB : 0u;
    const int64_t first1 = (tok1 * p.kv_heads + kvh) * D * EB;
    rk1 = make_rsrc(p.k_cache + first1, extent1);
    rv1 = make_rsrc(p.v_cache + first1, extent1);
  }
#pragma unroll
  for (int mt = 0; mt < TileRegs<D, C8>::MT; ++mt) {
    const auto &rk = SPLIT && mt == 1 ? rk1 : rk0;
    if constexpr (!C8) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) {
        if constexpr (k_lines<D, C8>())  // t.k[mt][2L + h] = instruction (h, L)
          t.k[mt][s] = buf_load_x4<kKPolicy>(rk, o.k[mt] + (s & 1) * 8 * row_bytes + 128 * (s >> 1));
        else
          t.k[mt][s] = buf_load_x4(rk, o.k[mt] + 16 * s);
      }
    } else {
#pragma unroll
      for (int s = 0; s < D / 32; s += 2) {
        u32x4 w = buf_load_x4(rk, o.k[mt] + 8 * s);
        t.k[mt][s] = u32x4{w[0], w[1], 0u, 0u};
        t.k[mt][s + 1] = u32x4{w[2], w[3], 0u, 0u};
      }
    }
  }
  constexpr int DW = VSlice<D, C8>::DW;
#pragma unroll
  for (int j = 0; j < TileRegs<D, C8>::TPL; ++j) {
    const auto &rv = SPLIT && j >= 4 ? rv1 : rv0;
    if constexpr (DW == 1) {
      t.v[j][0] = buf_load_x1(rv, o.v[j]);
    } else if constexpr (DW == 2) {
      const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, o.v[j], 0, kVPolicy));
      t.v[j][0] = w[0];
      t.v[j][1] = w[1];
    } else {
#pragma unroll
      for (int q = 0; q < DW; q += 4) {
        const u32x4 w = buf_load_x4<kVPolicy>(rv, o.v[j] + 4 * q);
        t.v[j][q] = w[0];
        t.v[j][q + 1] = w[1];
        t.v[j][q + 2] = w[2];
        t.v[j][q + 3] = w[3];
      }
    }
  }
  if constexpr (C8) {
    const int64_t s0 = tok0 * p.kv_heads + kvh;
    const uint32_t sext = (uint32_t(n0 - 1) * p.kv_heads + 1) * 4;
    const auto rks0 = make_rsrc(p.k_scale + s0, sext);
    const auto rvs0 = make_rsrc(p.v_scale + s0, sext);
    auto rks1 = rks0, rvs1 = rvs0;
    if constexpr (SPLIT) {
      const int64_t s1 = tok1 * p.kv_heads + kvh;
      const uint32_t sext1 = n_live > 16 ? (uint32_t(n_live - 17) * p.kv_heads + 1) * 4 : 0u;
      rks1 = make_rsrc(p.k_scale + s1, sext1);
      rvs1 = make_rsrc(p.v_scale + s1, sext1);
    }
#pragma unroll
    for (int j = 0; j < TileRegs<D, C8>::TPL; ++j) {
      t.ks[j] = buf_load_f32(SPLIT && j >= 4 ? rks1 : rks0, o.sc[j]);
      t.vs[j] = buf_load_f32(SPLIT && j >= 4 ? rvs1 : rvs0, o.sc[j]);
    }
  }
}

// int8 codes (4 per dword) -> exact bf16 values, 8 codes -> 4 packed dwords.
__device__ __forceinline__ uint32_t i8pair_to_bf16x2(int a, int b) {
  // Small integers are exact in fp32 and in bf16 (|x| <= 128 < 2^8), so the
  // high half of the fp32 pattern is the bf16 value.
  return perm_b32(__float_as_uint(float(b)), __float_as_uint(float(a)), 0x07060302u);
}
__device__ __forceinline__ int i8_at(uint32_t w, int b) {
  return (int32_t(w) << (24 - 8 * b)) >> 24;
}

// Growth of the running max (log2 units) tolerated before the accumulators
// are rescaled; probabilities then stay below 2^8, exact enough for bf16 P.
constexpr float kRescaleSlack = 8.0f;

// Tokens [t_begin, t_end) of sequence seq (t_begin a multiple of 32) for kv
// head kvh; writes the output
// (slot < 0: the range is the whole sequence) or partial slot `slot`.
template <int D, bool C8, bool SP>
__device__ __forceinline__ void decode_item(const DecodeParams &p, int seq, int t_begin, int t_end,
                                            int slot, int kvh, int lane) {
  const int c = lane & 15, g = lane >> 4;
  const int head = kvh * p.group + c;
  const bool head_live = c < p.group;

  // B operand of QK^T: q[head][d0(s, g) + e], zero for padded heads. Buffer
  // loads with an out-of-range offset for padded heads: unconditional loads
  // issue together (loads behind a branch each got their own full wait).
  u32x4 qv[D / 32];
  {
    const auto rq = make_rsrc(p.q + q_row_of(p, seq) * p.q_heads * D, uint32_t(p.q_heads) * D * 2);
    const uint32_t qoff = head_live ? uint32_t(head) * D * 2 : 0x80000000u;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      // Dims of k-step s, lane group g (matching the K operand).
      const int d0 = k_lines<D, C8>() ? 32 * s + 8 * g : (D / 4) * g + 8 * s;
      qv[s] = buf_load_x4(rq, qoff + uint32_t(d0) * 2);
    }
  }
  // C8 keys: QK^T runs in fp16 on the codes biased by kI8Bias (exact, three
  // VALU ops per four codes against a convert per code), q scaled per head by
  // a power of two into fp16 range; kI8Bias * sum(q) leaves each score.
  float k_corr = 0.0f, sl2 = p.scale_log2;
  if constexpr (C8) {
    float amax = 0.0f;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) amax = fmaxf(amax, bf16x8_absmax(qv[s]));
    amax = max_xor32(max_xor16(amax));
    const float qs = f16_range_scale(amax);
    float qsum = 0.0f;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) qv[s] = bf16x8_to_f16(qv[s], qs, &qsum);
    sl2 = p.scale_log2 / qs;
    k_corr = kI8Bias * sum_xor32(sum_xor16(qsum)) * sl2;
  }

  LaneOffsets o;
  {
    constexpr int EB = C8 ? 1 : 2;
    const uint32_t row_bytes = uint32_t(p.kv_heads) * D * EB;
    // Split tiles (16-token pages) address rows 16..31 from their own page.
    constexpr int kHalf = SP && decode_tile(D) == 32 ? 16 : 0;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int r0 = 16 * mt - (mt ? kHalf : 0);
      if (k_lines<D, C8>())
        o.k[mt] = uint32_t(r0 + (c & 7)) * row_bytes + 16 * (g + 4 * (c >> 3));
      else
        o.k[mt] = uint32_t(r0 + c) * row_bytes + (D / 4) * g * EB;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = tile_token(g, j) - (j >= 4 ? kHalf : 0);
      o.v[j] = uint32_t(row) * row_bytes + c * VSlice<D, C8>::BYTES;
      o.sc[j] = uint32_t(row) * p.kv_heads * 4;
    }
  }
  // Block ids of a window of 64 blocks (128 with 16-token pages) from block
  // win0 of the sequence, one per lane; the window slides (one vector load)
  // when a tile to be issued leaves it, so a range may span any number of
  // blocks.
  LaneBlocks lane_blocks{0, 0};
  constexpr int kWin = SP ? 128 : 64;
  const int32_t *table_row = p.block_tables + int64_t(seq) * p.table_stride;
  const int nblk_end = (t_end - 1) / p.block_size + 1;  // blocks up to the range end
  int win0 = t_begin / p.block_size;
  // Entries past the range end read as 0 (buffer bounds), without a branch.
  const auto rt = make_rsrc(table_row, uint32_t(nblk_end) * 4);
  auto load_window = [&]() {
    auto clamp = [&](int b) { return b < 0 ? 0 : (b >= p.num_blocks ? int(p.num_blocks - 1) : b); };
    lane_blocks.lo = clamp(int(buf_load_x1(rt, uint32_t(win0 + lane) * 4)));
    if constexpr (SP) lane_blocks.hi = clamp(int(buf_load_x1(rt, uint32_t(win0 + lane + 64) * 4)));
  };
  load_window();

  constexpr int NV = D / 16;  // PV MFMAs per tile (each yields 16 dims x 16 heads)
  f32x4 oacc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) oacc[i] = f32x4{0, 0, 0, 0};
  float m_run = -INFINITY, l_run = 0.0f;

  using TR = TileRegs<D, C8>;
  constexpr int TT = TR::TT, TPL = TR::TPL;
  auto qk = [&](const TR &t, f32x4 (&sacc)[TR::MT]) {
    // Scores: row block mt gives tokens 16 mt + 4g + r of head c.
#pragma unroll
    for (int mt = 0; mt < TR::MT; ++mt) sacc[mt] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
#pragma unroll
      for (int mt = 0; mt < TR::MT; ++mt) {
        u32x4 a;
        if constexpr (k_lines<D, C8>()) {
          // k-step s: chunk column g (s even) or g + 4 (s odd) of line s >> 1,
          // from instructions (0, s >> 1) and (1, s >> 1).
          const u32x4 A = t.k[mt][s & ~1], B = t.k[mt][s | 1];
          const bool lo = c < 8;
          if ((s & 1) == 0) {
            const u32x4 r = row_ror8(B);
            a = u32x4{lo ? A[0] : r[0], lo ? A[1] : r[1], lo ? A[2] : r[2], lo ? A[3] : r[3]};
          } else {
            const u32x4 r = row_ror8(A);
            a = u32x4{lo ? r[0] : B[0], lo ? r[1] : B[1], lo ? r[2] : B[2], lo ? r[3] : B[3]};
          }
        } else if constexpr (!C8)
          a = t.k[mt][s];
        else
          a = i8x8_to_f16_biased(t.k[mt][s][0], t.k[mt][s][1]);
        sacc[mt] = C8 ? mfma16x16x32_f16(a, qv[s], sacc[mt]) : mfma16x16x32(a, qv[s], sacc[mt]);
      }
    }
  };
  auto finish = [&](const TR &t, int t0, const f32x4 (&sacc)[TR::MT]) {
    float x[TPL];
#pragma unroll
    for (int mt = 0; mt < TR::MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        x[4 * mt + r] = C8 ? __builtin_fmaf(sacc[mt][r], sl2, -k_corr) : sacc[mt][r] * sl2;
    if constexpr (C8) {
#pragma unroll
      for (int j = 0; j < TPL; ++j) x[j] *= t.ks[j];
    }
    if (t_end - t0 < TT) {  // partial last tile (wave-uniform branch)
      const int n_live = t_end - t0;
#pragma unroll
      for (int j = 0; j < TPL; ++j) x[j] = tile_token(g, j) < n_live ? x[j] : -INFINITY;
    }
    float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    if constexpr (TPL == 8) tmax = fmaxf(tmax, fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    tmax = max_xor16(tmax);
    tmax = max_xor32(tmax);
    if (__any(tmax > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < NV; ++i) oacc[i] *= alpha;
    }
    float pr[TPL];
#pragma unroll
    for (int j = 0; j < TPL; ++j) pr[j] = fast_exp2(x[j] - m_run);
    float psum = (pr[0] + pr[1]) + (pr[2] + pr[3]);
    if constexpr (TPL == 8) psum += (pr[4] + pr[5]) + (pr[6] + pr[7]);
    l_run += psum;
    if constexpr (C8) {
#pragma unroll
      for (int j = 0; j < TPL; ++j) pr[j] *= t.vs[j];
    }
    uint32_t pb[TPL / 2];
#pragma unroll
    for (int i = 0; i < TPL / 2; ++i) pb[i] = pack_bf16x2(pr[2 * i], pr[2 * i + 1]);
    // PV: MFMA b produces O^T rows m = c <-> dim c*VPL + b; its A operand is
    // element b of the lane's tokens, paired into bf16x2 words (16x16x32 for
    // 32-token tiles, 16x16x16 for 16-token tiles).
    constexpr int VPL = VSlice<D, C8>::VPL;
#pragma unroll
    for (int b = 0; b < VPL; ++b) {
      uint32_t a[TPL / 2];
#pragma unroll
      for (int i = 0; i < TPL / 2; ++i) {
        if constexpr (!C8) {
          const int w = b >> 1;
          a[i] = (b & 1) ? pack_hi16(t.v[2 * i][w], t.v[2 * i + 1][w])
                         : pack_lo16(t.v[2 * i][w], t.v[2 * i + 1][w]);
        } else {
          const int w = b >> 2, y = b & 3;
          a[i] = i8pair_to_bf16x2(i8_at(t.v[2 * i][w], y), i8_at(t.v[2 * i + 1][w], y));
        }
      }
      if constexpr (TPL == 8)
        oacc[b] = mfma16x16x32(u32x4{a[0], a[1], a[2], a[3]}, u32x4{pb[0], pb[1], pb[2], pb[3]}, oacc[b]);
      else
        oacc[b] = mfma16x16x16(u32x2{a[0], a[1]}, u32x2{pb[0], pb[1]}, oacc[b]);
    }
  };

  // Ring of kStages tile buffers: tiles t+1 .. t+kStages-1 are in flight while
  // tile t is reduced. Tiles past the range end reload the last tile (a cache
  // hit) so every iteration has the same shape. Tiles are issued in order, so
  // the block-id window only moves forward.
  constexpr int kStages = decode_stages<D>();
  TileRegs<D, C8> tr[kStages];
  auto clamp_tile = [&](int t) { return t < t_end ? t : t_end - 1 - ((t_end - 1 - t_begin) & (TT - 1)); };
  auto issue = [&](TileRegs<D, C8> &t, int t0) {
    if ((t0 + TT - 1) / p.block_size - win0 >= kWin) {
      win0 = t0 / p.block_size;
      load_window();
    }
    load_tile<D, C8, SP>(t, p, lane_blocks, win0, kvh, t0, t_end, o);
  };
#pragma unroll
  for (int i = 0; i < kStages - 1; ++i) issue(tr[i], clamp_tile(t_begin + i * TT));
  int t0 = t_begin;
  // C8 tiles: the next tile's QK^T MFMAs are issued before this tile's
  // softmax and PV, so the MFMAs run under that VALU work (one wave per SIMD
  // leaves no other wave to hide them; config 4 0.2031-0.2059 -> 0.2020-0.2024
  // ms). bf16 tiles keep the plain order (head_dim 256 measured 1% slower
  // pipelined, head_dim 128 unchanged).
  if constexpr (C8) {
    f32x4 sc[TR::MT];
    qk(tr[0], sc);
    while (true) {
#pragma unroll
      for (int i = 0; i < kStages; ++i) {
        issue(tr[(i + kStages - 1) % kStages], clamp_tile(t0 + (kStages - 1) * TT));
        __builtin_amdgcn_sched_barrier(0);
        f32x4 sn[TR::MT];
        qk(tr[(i + 1) % kStages], sn);
        finish(tr[i], t0, sc);
#pragma unroll
        for (int mt = 0; mt < TR::MT; ++mt) sc[mt] = sn[mt];
        t0 += TT;
        if (t0 >= t_end) break;
      }
      if (t0 >= t_end) break;
    }
  } else {
    while (true) {
#pragma unroll
      for (int i = 0; i < kStages; ++i) {
        issue(tr[(i + kStages - 1) % kStages], clamp_tile(t0 + (kStages - 1) * TT));
        // Keep the prefetch issued ahead of this tile's math (the scheduler would
        // otherwise sink it below the QK^T MFMAs and shrink the loads in flight).
        __builtin_amdgcn_sched_barrier(0);
        f32x4 sc[TR::MT];
        qk(tr[i], sc);
        finish(tr[i], t0, sc);
        t0 += TT;
        if (t0 >= t_end) break;
      }
      if (t0 >= t_end) break;
    }
  }

  float l_tot = sum_xor16(l_run);
  l_tot = sum_xor32(l_tot);
  if (!head_live) return;

  // Lane holds O^T rows m = 4g + r of MFMA b -> dim (4g + r)*VPL + b: the
  // contiguous dims [4g*VPL, 4g*VPL + D/4) of head c.
  constexpr int VPL = VSlice<D, C8>::VPL;
  float ov[D / 4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int b = 0; b < VPL; ++b) ov[r * VPL + b] = oacc[b][r];
  auto chunk_dim = [&](int k) { return 4 * g * VPL + 8 * k; };
  if (slot < 0) {
    const float inv = 1.0f / l_tot;
    uint16_t *op = p.out + (q_row_of(p, seq) * p.q_heads + head) * D;
#pragma unroll
    for (int k = 0; k < D / 32; ++k) {
      const float *v = ov + 8 * k;
      store_u32x4(op + chunk_dim(k), u32x4{pack_bf16x2(v[0] * inv, v[1] * inv),
                                           pack_bf16x2(v[2] * inv, v[3] * inv),
                                           pack_bf16x2(v[4] * inv, v[5] * inv),
                                           pack_bf16x2(v[6] * inv, v[7] * inv)});
    }
  } else {
    const int64_t prow = int64_t(slot) * p.q_heads + head;
    float *po = p.part_o + prow * D;
#pragma unroll
    for (int k = 0; k < D / 32; ++k) {
      const float *v = ov + 8 * k;
      *reinterpret_cast<f32x4 *>(po + chunk_dim(k)) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4 *>(po + chunk_dim(k) + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
    if (g == 0) *reinterpret_cast<float2 *>(p.part_ml + prow * 2) = make_float2(m_run, l_tot);
  }
}

// Persistent decode: workgroup b takes workers b, b + grid, ...; worker v owns
// the work units [lo(v), lo(v + 1)) of Shares (share units each, skewed
// between odd and even workers for bf16), i.e. the 32-token tiles j of
// sequence s with seq_pos[s] + seq_cost + 32 j in that range, walked from
// start_seq[v] in sequence order. The waves of a workgroup take the kv heads of
// one range, so the halves of every cache row are fetched by sibling waves at
// the same time (whole rows stay DRAM-page friendly; measured ~40% more
// bandwidth than independent waves). Every workgroup gets the same work; the
// former longest-first work queue left half of them idle for the last third of
// a config-2 step (a full 2048-token item at its end) and serialised 512
// same-address atomics at the start.
// Workgroup-wide exclusive scan (sum, or max with identity -1) over the
// workgroup's waves (at most four), wave totals through `wt`; *total gets the
// workgroup's total.
template <bool MAX>
__device__ __forceinline__ int decode_wg_scan(int x, int *wt, int *total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  constexpr int kId = MAX ? -1 : 0;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x = MAX ? (y > x ? y : x) : x + y;
  }
  int excl = __shfl_up(x, 1, 64);
  excl = lane == 0 ? kId : excl;
  if (lane == 63) wt[wv] = x;
  __syncthreads();
  int before = kId, all = kId;
  for (int u = 0; u < nw; ++u) {
    const int t = wt[u];
    if (u < wv) before = MAX ? (t > before ? t : before) : before + t;
    all = MAX ? (t > all ? t : all) : all + t;
  }
  __syncthreads();  // wt is reused by the next scan
  *total = all;
  return MAX ? (before > excl ? before : excl) : before + excl;
}

// The decode plan of a call of at most kSelfPlanPerThread sequences per
// thread, computed by every decode workgroup for itself (the prologue's
// arithmetic in 32-bit units, which the host allows only when every prefix
// fits): s_pos = first unit of each sequence; s_se = (first partial slot + 1)
// << 16 | (running max of the sequences' last-tile workers + 1), so the first
// sequence of worker v is the first whose running max reaches v. Thread t
// takes sequences K t .. K t + K - 1 (in unit order). Workgroup 0 also stores
// the sequences' slots for the merge and zeroes the output of sequences
// without a visible key.
__device__ __forceinline__ void decode_self_plan_wg(const DecodeParams &p, int *s_pos, int *s_se,
                                                    int *s_wt, int &workers, int64_t &share) {
  constexpr int K = kSelfPlanPerThread;
  const int s0 = threadIdx.x * K;
  int len[K], sum = 0;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int seq = s0 + k;
    const bool dec = seq < p.num_seqs && decode_seq(p, seq);
    len[k] = dec ? clamp_len(p, seq) : 0;
    if (blockIdx.x == 0 && dec && len[k] <= 0) {  // no visible key: defined zero output
      uint16_t *o = p.out + q_row_of(p, seq) * p.q_heads * p.head_dim;
      for (int i = 0; i < p.q_heads * p.head_dim; i += 8) store_u32x4(o + i, u32x4{0, 0, 0, 0});
    }
    sum += len[k] > 0 ? len[k] + p.seq_cost : 0;
  }
  int total;
  const int pos0 = decode_wg_scan<false>(sum, s_wt, &total);
  {
    const int64_t small = (int64_t(total) + kMinShareUnits - 1) / kMinShareUnits;
    workers = int(small < p.grid ? small : p.grid);
    workers = workers < 1 ? 1 : workers;
    share = total > 0 ? (int64_t(total) + workers - 1) / workers : 1;
  }
  int cnt[K], last[K], csum = 0, emine = -1;
  int pos = pos0;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    cnt[k] = 0;
    last[k] = -1;
    if (len[k] > 0) {
      int wa, wb;
      seq_workers(int64_t(pos) + p.seq_cost, len[k], make_shares(p, share), wa, wb);
      cnt[k] = wb > wa ? wb - wa + 1 : 0;
      last[k] = wb;
      emine = wb;  // nondecreasing along the thread's sequences
      pos += len[k] + p.seq_cost;
    }
    csum += cnt[k];
  }
  int nslots, emax;
  int slot = decode_wg_scan<false>(csum, s_wt, &nslots);
  int erun = decode_wg_scan<true>(emine, s_wt, &emax);  // over earlier threads
  pos = pos0;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int seq = s0 + k;
    if (seq < p.num_seqs) {
      erun = last[k] > erun ? last[k] : erun;
      s_pos[seq] = pos;
      s_se[seq] = ((cnt[k] > 0 ? slot : -1) + 1) << 16 | (erun + 1);
      if (blockIdx.x == 0) p.seq_slot[seq] = make_int2(cnt[k] > 0 ? slot : -1, cnt[k]);
    }
    if (len[k] > 0) pos += len[k] + p.seq_cost;
    slot += cnt[k];
  }
  __syncthreads();
}

template <int D, bool C8, bool SP>
__global__ __launch_bounds__(64 * max_decode_waves(D), 1) void paged_decode_kernel(
    DecodeParams p, int waves_per_wg) {
  const int lane = threadIdx.x & 63, wave = uniform(int(threadIdx.x >> 6));
  const int groups = (p.kv_heads + waves_per_wg - 1) / waves_per_wg;
  // Small calls plan in LDS (decode_self_plan_wg); others read the
  // prologue's plan through scalar loads (ld_const: as vector loads each
  // waited behind the previous range's output stores).
  __shared__ int s_pos[kSelfPlanMaxSeqs], s_se[kSelfPlanMaxSeqs], s_wt[max_decode_waves(D)];
  int workers;
  int64_t share;
  if (p.self_plan) {
    decode_self_plan_wg(p, s_pos, s_se, s_wt, workers, share);
  } else {
    workers = ld_const(p.plan);
    share = share_of(p);
  }
  auto start_seq = [&](int v) {
    if (!p.self_plan) return int(ld_const(p.start_seq + v));
    int a = 0, b = p.num_seqs;  // first sequence whose running last-tile worker reaches v
    while (a < b) {
      const int m = (a + b) >> 1;
      if ((s_se[m] & 0xFFFF) - 1 >= v) b = m; else a = m + 1;
    }
    return a;
  };
  for (int v = blockIdx.x; v < workers; v += gridDim.x) {
    const Shares sh = make_shares(p, share);
    const int64_t lo = sh.lo(v), hi = sh.lo(v + 1);
    for (int seq = start_seq(v); seq < p.num_seqs; ++seq) {
      const int64_t first =
          (p.self_plan ? int64_t(s_pos[seq]) : ld_const(p.seq_pos + seq)) + p.seq_cost;  // tile 0
      if (first >= hi) break;
      if (!decode_seq(p, seq)) continue;
      const int len = uniform(clamp_len(p, seq));
      if (len <= 0) continue;
      const int tiles = (len + kSplitTile - 1) / kSplitTile;
      const int64_t a = lo - first, b = hi - first;
      const int j0 = a <= 0 ? 0 : int((a + kSplitTile - 1) / kSplitTile);
      int j1 = b <= 0 ? 0 : int((b + kSplitTile - 1) / kSplitTile);
      j1 = j1 < tiles ? j1 : tiles;
      if (j0 >= j1) continue;
      int slot = p.self_plan ? (s_se[seq] >> 16) - 1 : ld_const(&p.seq_slot[seq].x);
      if (slot >= 0) slot += v - sh.worker(first);
      const int t_end = j1 * kSplitTile < len ? j1 * kSplitTile : len;
      for (int grp = 0; grp < groups; ++grp) {
        const int kvh = uniform(grp * waves_per_wg + wave);  // wave-uniform for SGPR descriptors
        if (kvh < p.kv_heads) decode_item<D, C8, SP>(p, seq, j0 * kSplitTile, t_end, slot, kvh, lane);
      }
    }
  }
}

namespace {
template <int D, bool C8>
void launch_decode(const DecodeParams &p0, const RowWrite &wr, hipStream_t s) {
  const int waves = p0.kv_heads < max_decode_waves(D) ? p0.kv_heads : max_decode_waves(D);
  DecodeParams p = p0;
  p.seq_cost = decode_seq_cost(C8);
  p.self_plan = decode_self_plan(p, 64 * waves) ? 1 : 0;
  p.skew_pm = decode_skew_pm(C8, D);
  launch_prologue(p, wr, s);
  const int grid = p.grid;
  if (p.block_size == 16)  // the reference's bf16 page (paged_state_contract.h:25)
    paged_decode_kernel<D, C8, true><<<grid, 64 * waves, 0, s>>>(p, waves);
  else
    paged_decode_kernel<D, C8, false><<<grid, 64 * waves, 0, s>>>(p, waves);
  launch_merge<D>(p, s);
}

}  // namespace

// Decode rows of a packed varlen batch (p.cu_seqlens set), bf16 caches.
void launch_varlen_decode_rows(const DecodeParams &p, int head_dim, hipStream_t s) {
  const RowWrite none{};
  if (head_dim == 64) launch_decode<64, false>(p, none, s);
  else if (head_dim == 128) launch_decode<128, false>(p, none, s);
  else launch_decode<256, false>(p, none, s);
}

namespace {

int32_t decode_common(bool c8, const void *q, const void *k_cache, const void *v_cache,
                      const void *k_scale, const void *v_scale, const int32_t *block_tables,
                      int32_t table_stride, const int32_t *seq_lens, void *out, int32_t num_seqs,
                      int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t block_size,
                      int64_t num_blocks, int32_t max_context, float scale, void *workspace,
                      uint64_t workspace_bytes, void *stream, const RowWrite &wr) {
  if (!q || !k_cache || !v_cache || !block_tables || !seq_lens || !out ||
      (c8 && (!k_scale || !v_scale)))
    return fail(IFATTN_EINVAL, "paged decode: null pointer");
  if (num_seqs <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads ||
      q_heads / kv_heads > 16)
    return fail(IFATTN_EINVAL, "paged decode: need q_heads = group * kv_heads with group <= 16");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IFATTN_EINVAL, "paged decode: head_dim must be 64, 128 or 256");
  if (block_size < 16 || (block_size & (block_size - 1)))
    return fail(IFATTN_EINVAL, "paged decode: block_size must be a power of two >= 16");
  if (max_context <= 0 || num_blocks <= 0 || table_stride <= 0 ||
      int64_t(table_stride) * block_size < max_context)
    return fail(IFATTN_EINVAL, "paged decode: table_stride * block_size must cover max_context");
  if (num_seqs >= (1 << 20))
    return fail(IFATTN_EINVAL, "paged decode: num_seqs must be below 2^20");
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
  p.scale_log2 = scale * kLog2e;
  if (max_context > (1 << 20)) return fail(IFATTN_EINVAL, "paged decode: max_context above 1M tokens");
  const uint64_t need = ifattn_paged_decode_workspace_size(num_seqs, q_heads, head_dim, max_context);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(IFATTN_EWORKSPACE, "paged decode: workspace missing, short or misaligned");
  split_k_bind_workspace(p, workspace, q_heads, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (c8) {
    if (head_dim == 64) launch_decode<64, true>(p, wr, s);
    else if (head_dim == 128) launch_decode<128, true>(p, wr, s);
    else launch_decode<256, true>(p, wr, s);
  } else {
    if (head_dim == 64) launch_decode<64, false>(p, wr, s);
    else if (head_dim == 128) launch_decode<128, false>(p, wr, s);
    else launch_decode<256, false>(p, wr, s);
  }
  return launch_status("paged decode");
}
}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" uint64_t ifattn_paged_decode_workspace_size(int32_t num_seqs, int32_t q_heads,
                                                       int32_t head_dim, int32_t max_context) {
  if (num_seqs <= 0 || q_heads <= 0 || head_dim <= 0 || max_context <= 0) return 0;
  return split_k_workspace_bytes(num_seqs, q_heads, head_dim, max_context);
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
                       max_context, scale, workspace, workspace_bytes, stream, RowWrite{});
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
                       max_context, scale, workspace, workspace_bytes, stream, RowWrite{});
}

extern "C" int32_t ifattn_paged_decode_step_bf16(
    const void *q, const void *k_rows, const void *v_rows, void *k_cache, void *v_cache,
    const void *slot_mapping, int32_t slot_dtype, int64_t rows, const int32_t *block_tables,
    int32_t table_stride, const int32_t *seq_lens, void *out, int32_t num_seqs, int32_t q_heads,
    int32_t kv_heads, int32_t head_dim, int32_t block_size, int64_t num_blocks,
    int32_t max_context, float scale, void *workspace, uint64_t workspace_bytes, void *stream) {
  if (rows < 0 || (rows > 0 && (!k_rows || !v_rows || !slot_mapping)))
    return fail(IFATTN_EINVAL, "decode step: rows >= 0 with k/v rows and slot mapping");
  if (slot_dtype != IFATTN_DTYPE_I32 && slot_dtype != IFATTN_DTYPE_I64)
    return fail(IFATTN_EINVAL, "decode step: slot mapping dtype must be I32 (4) or I64 (5)");
  if (rows > 0 && (!aligned16(k_rows) || !aligned16(v_rows)))
    return fail(IFATTN_EINVAL, "decode step: k/v rows must be 16-byte aligned");
  RowWrite wr{};
  if (rows > 0) {
    wr.k_rows = static_cast<const uint8_t *>(k_rows);
    wr.v_rows = static_cast<const uint8_t *>(v_rows);
    wr.k_cache = static_cast<uint8_t *>(k_cache);
    wr.v_cache = static_cast<uint8_t *>(v_cache);
    wr.slots = slot_mapping;
    wr.slot_i64 = slot_dtype == IFATTN_DTYPE_I64;
    wr.rows = rows;
    wr.row_vecs = int64_t(kv_heads) * head_dim * 2 / 16;
    wr.num_slots = num_blocks * block_size;
  }
  return decode_common(false, q, k_cache, v_cache, nullptr, nullptr, block_tables, table_stride,
                       seq_lens, out, num_seqs, q_heads, kv_heads, head_dim, block_size, num_blocks,
                       max_context, scale, workspace, workspace_bytes, stream, wr);
}

// ---------------------------------------------------------------- no-allocation step
//
// Device scratch for ifattn_paged_decode_step_bf16_noalloc: the split-K plan
// (shares, per-sequence positions and slots) and partials of one call live here
// instead of in a caller workspace. Every GPU the library runs on holds its own
// copy until the process ends. Nothing in it has to start at zero (the
// prologue kernel writes the plan before the decode kernel reads it, and
// partials are written before the merge reads them).
static __device__ __align__(256) uint8_t scratch[IFATTN_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch[kMaxDevices] = {};

// Device address of this GPU's `scratch` (the host-side symbol is only a
// stand-in), looked up once per device with that device current.
int32_t scratch_address(void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(IFATTN_ELAUNCH, "decode step (no allocation): no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(IFATTN_ELAUNCH, "decode step (no allocation): scratch lookup",
                  hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return IFATTN_OK;
}
}  // namespace

extern "C" int32_t ifattn_paged_decode_step_bf16_noalloc(
    const void *q, const void *k_rows, const void *v_rows, void *k_cache, void *v_cache,
    const void *slot_mapping, int32_t slot_dtype, int64_t rows, const int32_t *block_tables,
    int32_t table_stride, const int32_t *seq_lens, void *out, int32_t num_seqs, int32_t q_heads,
    int32_t kv_heads, int32_t head_dim, int32_t block_size, int64_t num_blocks,
    int32_t max_context, float scale, void *stream) {
  const uint64_t need = ifattn_paged_decode_workspace_size(num_seqs, q_heads, head_dim, max_context);
  if (need > IFATTN_NOALLOC_SCRATCH_BYTES)
    return fail(IFATTN_EINVAL,
                "decode step (no allocation): the call needs more than the 32 MiB static scratch "
                "(fewer sequences or a shorter max_context)");
  void *ws = nullptr;
  if (const int32_t st = scratch_address(&ws)) return st;
  return ifattn_paged_decode_step_bf16(q, k_rows, v_rows, k_cache, v_cache, slot_mapping,
                                       slot_dtype, rows, block_tables, table_stride, seq_lens, out,
                                       num_seqs, q_heads, kv_heads, head_dim, block_size,
                                       num_blocks, max_context, scale, ws,
                                       IFATTN_NOALLOC_SCRATCH_BYTES, stream);
}
