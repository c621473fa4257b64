// CPU ORACLE — TEST INFRASTRUCTURE ONLY.
//
// A plain C++17 restatement of the reference's CPU algorithms for the
// continuous-batching attention path. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg load it, as the checker (or the timed CPU
// baseline); the product library never links or calls it.
//
// Arithmetic: fp32 accumulation everywhere (BASELINE's contract); the bf16
// rounding rule is round-to-nearest-even on the fp32 bits
// (crates/inferfabric-cli/src/npu_probe.rs:151-154). Work is split over
// (sequence, kv head) units on std::thread.
//
// Functions and what pins them (see tests/test_oracle.py):
//   oracle_kv_write        ScatterNdUpdate semantics, inferfabric_acl.cpp:1364-1376.
//                          Pinned: untouched rows unchanged, round trip.
//   oracle_quant_rows      per_token_head symmetric int8, cache_quantization.cpp:20-34
//                          with round-half-even. Pinned: reference probe vectors
//                          (cache_quantization_probe.cpp:17,25-26), hand tie cases.
//   oracle_quant_legacy    the same kernel's exact arithmetic (ties away, INT4 nibbles).
//                          Pinned: probe vectors, tie cases, nibble layout.
//   oracle_mla_pack_c8     656-byte row, docs/packed-mla-cache.md:27-43; oracle checks of
//                          packed_cache_probe.cpp:24-45. Pinned: tile scale/quant/rope bits.
//   oracle_mla_norm_rope_write  fused RMSNorm + half-rope + cache row, resident_cache_writer.h:5-20.
//                          Pinned: prefill_cache_writer_probe.cpp:38-61 fixtures and
//                          tolerances, double-precision restatement, exact rope bits.
//   oracle_paged_decode    attention.rs:221-253 (GQA kh = h/group at :226) without the bf16
//                          rounding of intermediates (fp32 contract), plus an optional
//                          mode that keeps the Rust oracle's roundings. Pinned: closed
//                          forms (q = 0 mean, constant-per-head V, two-token softmax),
//                          sequence_attention_probe.cpp:26-27,100 known answer.
//   oracle_gated_attention the Qwen session operation, inferfabric_acl.cpp:1343-1430.
//                          Pinned: equality with oracle_paged_decode when the mask opens
//                          a prefix (gate 1), mask-shift invariance, gate linearity,
//                          a two-position closed form with mask and gate.
//   oracle_qk_norm_rope_gate  the Qwen attention producer, inferfabric_acl.cpp:1236-1341
//                          and its CPU statement attention.rs:35-64. Pinned: position 0
//                          leaves the norm unrotated, rotation preserves pair norms,
//                          gamma 1 gives unit RMS, constant rows, sigmoid(0) = 1/2,
//                          a hand-computed rotation at position 1.
//   oracle_varlen_prefill  causal rule of openpangu_attention_metadata.h:20-22.
//                          Pinned: q = 0 causal prefix means, decode-row equivalence.
//   oracle_mla_decode      packed_cache_probe.cpp:47-66 / sliding_window_probe.cpp:144-163
//                          without sinks. Pinned: q = 0 latent mean, rope-only scores.
//   oracle_mla_attention   the same with query rows, windows, sparse index lists and
//                          learned sinks. Pinned: the two probes' fixtures against a
//                          float64 restatement, agreement with oracle_mla_decode,
//                          sparse list = dense range, order invariance.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline float bf(uint16_t v) {
  uint32_t u = uint32_t(v) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint16_t to_bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
inline float round_bf(float f) { return bf(to_bf(f)); }

template <typename F>
void parallel_for(int64_t n, int threads, F &&f) {
  if (threads <= 1 || n <= 1) {
    for (int64_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::atomic<int64_t> next{0};
  std::vector<std::thread> pool;
  const int t = int(std::min<int64_t>(threads, n));
  for (int k = 0; k < t; ++k)
    pool.emplace_back([&] {
      for (int64_t i; (i = next.fetch_add(1)) < n;) f(i);
    });
  for (auto &th : pool) th.join();
}

int default_threads(int threads) {
  if (threads > 0) return threads;
  // A GPU box gives one GPU's process a share of 16 host cores.
  unsigned h = std::thread::hardware_concurrency();
  return h ? int(std::min(h, 16u)) : 1;
}

// Symmetric RNE quantization of one group; returns the scale.
float quant_group_rne(const uint16_t *x, int width, int8_t *codes, float zero_scale) {
  float m = 0.0f;
  for (int j = 0; j < width; ++j) m = std::max(m, std::fabs(bf(x[j])));
  if (m == 0.0f) {
    std::memset(codes, 0, size_t(width));
    return zero_scale;
  }
  const float scale = m / 127.0f;
  for (int j = 0; j < width; ++j) {
    float v = bf(x[j]) / scale;
    int q = int(std::nearbyint(v));  // default FE_TONEAREST: ties to even
    codes[j] = int8_t(std::max(-127, std::min(127, q)));
  }
  return scale;
}

}  // namespace

extern "C" {

// cache[slots[r]] = rows[r]; out-of-range / negative slots are skipped.
void oracle_kv_write(const uint8_t *rows, uint8_t *cache, const int64_t *slots, int64_t n,
                     int64_t row_bytes, int64_t num_slots) {
  for (int64_t r = 0; r < n; ++r) {
    if (slots[r] < 0 || slots[r] >= num_slots) continue;
    std::memcpy(cache + slots[r] * row_bytes, rows + r * row_bytes, size_t(row_bytes));
  }
}

// Row-group quantization: `groups` groups of `width` bf16 values, one scale each.
void oracle_quant_rows(const uint16_t *x, int64_t groups, int32_t width, int8_t *codes,
                       float *scales, float zero_scale) {
  for (int64_t g = 0; g < groups; ++g)
    scales[g] = quant_group_rne(x + g * width, width, codes + g * width, zero_scale);
}

// if_cache_quantize arithmetic for one row (cache_quantization.cpp:20-34).
void oracle_quant_legacy(const uint16_t *x, int32_t width, int32_t bits, uint8_t *packed,
                         float *scale_out) {
  float maximum = 0;
  for (int j = 0; j < width; ++j) {
    float a = std::fabs(bf(x[j]));
    if (a > maximum) maximum = a;
  }
  const int limit = bits == 8 ? 127 : 7;
  const float scale = maximum == 0 ? 1.0f : maximum / float(limit);
  *scale_out = scale;
  const int per = 8 / bits;
  for (int j = 0; j < width; j += per) {
    uint8_t byte = 0;
    for (int k = 0; k < per; ++k) {
      volatile float value = bf(x[j + k]) / scale;
      volatile float shifted = value + (value >= 0 ? 0.5f : -0.5f);
      int q = int(shifted);
      q = q > limit ? limit : (q < -limit ? -limit : q);
      byte |= uint8_t((q & (bits == 8 ? 255 : 15)) << (k * bits));
    }
    packed[j * bits / 8] = byte;
  }
}

// if_cache_dequantize of rows <= last (cache_quantization.cpp:39-57).
void oracle_dequant_legacy(const uint8_t *packed, const float *scales, uint16_t *out,
                           int64_t last, int32_t width, int32_t capacity, int32_t bits) {
  for (int64_t row = 0; row < capacity; ++row) {
    float scale = row <= last ? scales[row] : 0;
    for (int j = 0; j < width; ++j) {
      int q = 0;
      if (row <= last) {
        uint8_t byte = packed[row * (width * bits / 8) + j * bits / 8];
        q = bits == 8 ? int(int8_t(byte)) : int((byte >> ((j % 2) * 4)) & 15);
        if (bits == 4 && q >= 8) q -= 16;
      }
      out[row * width + j] = to_bf(float(q) * scale);
    }
  }
}

// 576 bf16 -> 656-byte packed row (int8 latent | bf16 rope | f32 scale[4]).
void oracle_mla_pack_c8(const uint16_t *rows, int64_t n, uint8_t *out) {
  for (int64_t r = 0; r < n; ++r) {
    const uint16_t *x = rows + r * 576;
    uint8_t *o = out + r * 656;
    for (int t = 0; t < 4; ++t) {
      float s = quant_group_rne(x + 128 * t, 128, reinterpret_cast<int8_t *>(o + 128 * t), 0.0f);
      std::memcpy(o + 640 + 4 * t, &s, 4);
    }
    std::memcpy(o + 512, x + 512, 128);
  }
}

// Fused MLA cache writer: RMSNorm(512) * gamma, half rotary on the 64 rope
// values, then the cache row (bf16 576-wide, or the packed C8 656-byte row with
// per-128 tile scales). Follows resident_cache_writer.h:5-20 and the checks of
// prefill_cache_writer_probe.cpp:38-61 (norm 1/sqrt(mean(x^2)+eps), scale =
// tile max/127 with 0 for a zero tile, nearest-even codes, rope
// bf16(a*cos + (d<32 ? -b : b)*sin) with b = x[512 + (d+32)%64]).
// The fp32 operation order is fixed so that the device writer is bit-exact:
// each of 64 lanes sums the squares of its 8 consecutive values in order, the
// 64 lane sums are combined by a xor butterfly (masks 32..1), rstd =
// 1/sqrt(sum/512 + eps), y = (x*rstd)*gamma, C8 codes quantize y (fp32, no
// bf16 step). slots < 0 or >= num_slots are skipped.
void oracle_mla_norm_rope_write(const uint16_t *x, const uint16_t *gamma, const uint16_t *cosv,
                                const uint16_t *sinv, const int64_t *slots, int64_t rows,
                                float eps, uint8_t *cache, int32_t packed, int64_t num_slots) {
  const int64_t stride = packed ? 656 : 1152;
  for (int64_t r = 0; r < rows; ++r) {
    if (slots[r] < 0 || slots[r] >= num_slots) continue;
    const uint16_t *in = x + r * 576;
    uint8_t *o = cache + slots[r] * stride;
    float lane[64];
    for (int l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (int i = 0; i < 8; ++i) {
        const float v = bf(in[8 * l + i]);
        const float sq = v * v;
        acc = acc + sq;
      }
      lane[l] = acc;
    }
    for (int m = 32; m >= 1; m >>= 1) {
      float nxt[64];
      for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ m];
      std::memcpy(lane, nxt, sizeof(lane));
    }
    const float mean = lane[0] * (1.0f / 512.0f);
    const float rstd = 1.0f / std::sqrt(mean + eps);
    float y[512];
    for (int d = 0; d < 512; ++d) {
      const float t = bf(in[d]) * rstd;
      y[d] = t * bf(gamma[d]);
    }
    if (packed) {
      for (int t = 0; t < 4; ++t) {
        float m = 0.0f;
        for (int d = 128 * t; d < 128 * t + 128; ++d) m = std::max(m, std::fabs(y[d]));
        const float scale = m == 0.0f ? 0.0f : m / 127.0f;
        for (int d = 128 * t; d < 128 * t + 128; ++d) {
          int q = 0;
          if (scale != 0.0f) q = int(std::nearbyint(y[d] / scale));
          o[d] = uint8_t(int8_t(std::max(-127, std::min(127, q))));
        }
        std::memcpy(o + 640 + 4 * t, &scale, 4);
      }
    } else {
      for (int d = 0; d < 512; ++d) {
        const uint16_t b = to_bf(y[d]);
        std::memcpy(o + 2 * d, &b, 2);
      }
    }
    uint8_t *rope = o + (packed ? 512 : 1024);
    for (int d = 0; d < 64; ++d) {
      const float a = bf(in[512 + d]), b = bf(in[512 + (d + 32) % 64]);
      const float c = bf(cosv[r * 64 + d]), sn = bf(sinv[r * 64 + d]);
      const float p0 = a * c;
      const float p1 = (d < 32 ? -b : b) * sn;
      const uint16_t v = to_bf(p0 + p1);
      std::memcpy(rope + 2 * d, &v, 2);
    }
  }
}

// Paged GQA decode. c8 != 0: caches are int8 with fp32 scales [slots, kv_heads].
// ref_rounding != 0 keeps the Rust oracle's bf16 roundings of the raw score,
// the scaled score and the probability (attention.rs:235,241).
// out: fp32 [n, hq, d].
void oracle_paged_decode(const uint16_t *q, const void *k_cache, const void *v_cache,
                         const float *k_scale, const float *v_scale, int32_t c8,
                         const int32_t *tables, int32_t stride, const int32_t *lens, float *out,
                         int32_t n, int32_t hq, int32_t hkv, int32_t d, int32_t bs, float scale,
                         int32_t ref_rounding, int32_t threads) {
  const int group = hq / hkv;
  auto kval = [&](int64_t slot, int kh, int e) -> float {
    const int64_t i = (slot * hkv + kh) * d + e;
    if (c8) return float(static_cast<const int8_t *>(k_cache)[i]) * k_scale[slot * hkv + kh];
    return bf(static_cast<const uint16_t *>(k_cache)[i]);
  };
  auto vval = [&](int64_t slot, int kh, int e) -> float {
    const int64_t i = (slot * hkv + kh) * d + e;
    if (c8) return float(static_cast<const int8_t *>(v_cache)[i]) * v_scale[slot * hkv + kh];
    return bf(static_cast<const uint16_t *>(v_cache)[i]);
  };
  parallel_for(int64_t(n) * hkv, default_threads(threads), [&](int64_t unit) {
    const int b = int(unit / hkv), kh = int(unit % hkv);
    const int len = lens[b];
    std::vector<int64_t> slot(std::max(len, 0));
    for (int j = 0; j < len; ++j)
      slot[j] = int64_t(tables[int64_t(b) * stride + j / bs]) * bs + j % bs;
    std::vector<float> s(std::max(len, 0));
    for (int h = kh * group; h < (kh + 1) * group; ++h) {
      float *o = out + (int64_t(b) * hq + h) * d;
      if (len <= 0) {
        std::fill(o, o + d, 0.0f);
        continue;
      }
      const uint16_t *qh = q + (int64_t(b) * hq + h) * d;
      float mx = -INFINITY;
      for (int j = 0; j < len; ++j) {
        float acc = 0.0f;
        for (int e = 0; e < d; ++e) acc += bf(qh[e]) * kval(slot[j], kh, e);
        s[j] = ref_rounding ? round_bf(round_bf(acc) * scale) : acc * scale;
        mx = std::max(mx, s[j]);
      }
      float sum = 0.0f;
      for (int j = 0; j < len; ++j) sum += std::exp(s[j] - mx);
      for (int j = 0; j < len; ++j) {
        float p = std::exp(s[j] - mx) / sum;
        s[j] = ref_rounding ? round_bf(p) : p;
      }
      for (int e = 0; e < d; ++e) {
        float acc = 0.0f;
        for (int j = 0; j < len; ++j) acc += s[j] * vval(slot[j], kh, e);
        o[e] = acc;
      }
    }
  });
}

// Qwen-shape gated attention over per-position physical rows
// (inferfabric_acl_paged_attention_prepare, native/src/inferfabric_acl.cpp:1343-1430:
// scatter of the step's K/V rows, gather by `table`, scores * scale + additive
// fp32 mask, fp32 softmax, PV, product with the gate). Caches [slots, hkv*d]
// bf16; q/gate/out [batch, hq, d]; table int64 and mask fp32 [batch, context].
// The caches must already hold the step's rows (apply oracle_kv_write first).
// fp32 throughout (no bf16 rounding between the steps). A request whose mask is
// -inf everywhere gets zeros (the reference's softmax would give NaN).
void oracle_gated_attention(const uint16_t *q, const uint16_t *keys, const uint16_t *values,
                            const int64_t *table, const float *mask, const uint16_t *gate,
                            float *out, int32_t batch, int32_t context, int32_t hq, int32_t hkv,
                            int32_t d, float scale, int32_t threads) {
  const int group = hq / hkv;
  parallel_for(int64_t(batch) * hq, default_threads(threads), [&](int64_t unit) {
    const int b = int(unit / hq), h = int(unit % hq), kh = h / group;
    const uint16_t *qh = q + (int64_t(b) * hq + h) * d;
    std::vector<float> s(context);
    float mx = -INFINITY;
    for (int j = 0; j < context; ++j) {
      const float m = mask[int64_t(b) * context + j];
      if (m == -INFINITY) {
        s[j] = -INFINITY;
        continue;
      }
      const int64_t row = table[int64_t(b) * context + j];
      float acc = 0.0f;
      for (int e = 0; e < d; ++e) acc += bf(qh[e]) * bf(keys[(row * hkv + kh) * d + e]);
      s[j] = acc * scale + m;
      mx = std::max(mx, s[j]);
    }
    float *o = out + (int64_t(b) * hq + h) * d;
    std::fill(o, o + d, 0.0f);
    if (mx == -INFINITY) return;
    float sum = 0.0f;
    for (int j = 0; j < context; ++j) {
      s[j] = s[j] == -INFINITY ? 0.0f : std::exp(s[j] - mx);
      sum += s[j];
    }
    for (int j = 0; j < context; ++j) {
      if (s[j] == 0.0f) continue;
      const int64_t row = table[int64_t(b) * context + j];
      const float p = s[j] / sum;
      for (int e = 0; e < d; ++e) o[e] += p * bf(values[(row * hkv + kh) * d + e]);
    }
    const uint16_t *gh = gate + (int64_t(b) * hq + h) * d;
    for (int e = 0; e < d; ++e) o[e] *= bf(gh[e]);
  });
}

// Qwen q/k producer (inferfabric_acl_attention_qk_prepare,
// native/src/inferfabric_acl.cpp:1236-1341; CPU statement
// crates/inferfabric-cli/src/npu_probe/attention.rs:35-64). Per request r and head:
// n_j = bf16((x_j * inv) * gamma_j), inv = 1 / sqrt(sum(x^2) / 256 + 1e-6);
// for j < 32 angle = position[r] * f_j with f_j = 1 / 1e7^(j/32) in fp32
// (the C++ operator's table, :1249-1257; the Rust statement divides by 1e7^(j/32)
// instead), c, s = bf16(cos), bf16(sin);
// out_j = bf16(bf16(n_j c) - bf16(n_{j+32} s)), out_{j+32} = bf16(bf16(n_{j+32} c) + bf16(n_j s)).
// q heads read channels [0, 256) of a 512-wide packed head whose upper half is
// the gate: gate = bf16(1 / (1 + exp(-g))) (:1329-1339). Outputs are bf16 bits.
void oracle_qk_norm_rope_gate(const uint16_t *packed_q, const uint16_t *k, const float *q_gamma,
                              const float *k_gamma, const int64_t *positions, uint16_t *q_out,
                              uint16_t *k_out, uint16_t *gate, int32_t batch) {
  constexpr int kD = 256;
  float freq[32];
  for (int i = 0; i < 32; ++i) freq[i] = 1.0f / std::pow(10000000.0f, float(i) / 32.0f);
  for (int r = 0; r < batch; ++r) {
    for (int which = 0; which < 2; ++which) {
      const int heads = which == 0 ? 8 : 2, stride = which == 0 ? 2 * kD : kD;
      const float *gamma = which == 0 ? q_gamma : k_gamma;
      for (int h = 0; h < heads; ++h) {
        const uint16_t *x = (which == 0 ? packed_q : k) + (int64_t(r) * heads + h) * stride;
        uint16_t *o = (which == 0 ? q_out : k_out) + (int64_t(r) * heads + h) * kD;
        float ss = 0.0f;
        for (int j = 0; j < kD; ++j) ss += bf(x[j]) * bf(x[j]);
        const float inv = 1.0f / std::sqrt(ss / float(kD) + 1e-6f);
        float n[kD];
        for (int j = 0; j < kD; ++j) n[j] = round_bf((bf(x[j]) * inv) * gamma[j]);
        for (int j = 0; j < kD; ++j) o[j] = to_bf(n[j]);
        for (int j = 0; j < 32; ++j) {
          const float angle = float(positions[r]) * freq[j];
          const float c = round_bf(std::cos(angle)), sn = round_bf(std::sin(angle));
          o[j] = to_bf(round_bf(n[j] * c) - round_bf(n[j + 32] * sn));
          o[j + 32] = to_bf(round_bf(n[j + 32] * c) + round_bf(n[j] * sn));
        }
        if (which == 0)
          for (int j = 0; j < kD; ++j)
            gate[(int64_t(r) * heads + h) * kD + j] =
                to_bf(1.0f / (1.0f + std::exp(-bf(x[kD + j]))));
      }
    }
  }
}

// Packed varlen causal attention over paged bf16 caches. Row t of sequence s
// (count = cu[s+1]-cu[s] rows, kv_len = kv_lens[s]) sees keys
// [0, kv_len - count + t]. out: fp32 [total_q, hq, d].
void oracle_varlen_prefill(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                           const int32_t *tables, int32_t stride, const int32_t *cu,
                           const int32_t *kv_lens, float *out, int32_t nseq, int32_t hq,
                           int32_t hkv, int32_t d, int32_t bs, float scale, int32_t threads) {
  const int group = hq / hkv;
  const int64_t total = cu[nseq];
  std::vector<int32_t> seq_of(total);
  for (int s = 0; s < nseq; ++s)
    for (int64_t r = cu[s]; r < cu[s + 1]; ++r) seq_of[r] = s;
  parallel_for(total * hkv, default_threads(threads), [&](int64_t unit) {
    const int64_t row = unit / hkv;
    const int kh = int(unit % hkv);
    const int s = seq_of[row];
    const int count = cu[s + 1] - cu[s];
    const int visible = kv_lens[s] - count + int(row - cu[s]) + 1;
    std::vector<int64_t> slot(std::max(visible, 0));
    for (int j = 0; j < visible; ++j)
      slot[j] = int64_t(tables[int64_t(s) * stride + j / bs]) * bs + j % bs;
    std::vector<float> sc(std::max(visible, 0));
    for (int h = kh * group; h < (kh + 1) * group; ++h) {
      float *o = out + (row * hq + h) * d;
      if (visible <= 0) {
        std::fill(o, o + d, 0.0f);
        continue;
      }
      const uint16_t *qh = q + (row * hq + h) * d;
      float mx = -INFINITY;
      for (int j = 0; j < visible; ++j) {
        const uint16_t *kr = k_cache + (slot[j] * hkv + kh) * d;
        float acc = 0.0f;
        for (int e = 0; e < d; ++e) acc += bf(qh[e]) * bf(kr[e]);
        sc[j] = acc * scale;
        mx = std::max(mx, sc[j]);
      }
      float sum = 0.0f;
      for (int j = 0; j < visible; ++j) sum += std::exp(sc[j] - mx);
      for (int j = 0; j < visible; ++j) sc[j] = std::exp(sc[j] - mx) / sum;
      for (int e = 0; e < d; ++e) {
        float acc = 0.0f;
        for (int j = 0; j < visible; ++j)
          acc += sc[j] * bf(v_cache[(slot[j] * hkv + kh) * d + e]);
        o[e] = acc;
      }
    }
  });
}

// MLA latent decode. bf16 rows of 576, or packed 656-byte C8 rows (c8 != 0).
// out: fp32 [n, heads, 512].
void oracle_mla_decode(const uint16_t *q, const void *cache, int32_t c8, const int32_t *tables,
                       int32_t stride, const int32_t *lens, float *out, int32_t n, int32_t heads,
                       int32_t bs, float scale, int32_t threads) {
  auto val = [&](int64_t slot, int e) -> float {
    if (!c8) return bf(static_cast<const uint16_t *>(cache)[slot * 576 + e]);
    const uint8_t *row = static_cast<const uint8_t *>(cache) + slot * 656;
    if (e < 512) {
      float sc;
      std::memcpy(&sc, row + 640 + (e / 128) * 4, 4);
      return float(int8_t(row[e])) * sc;
    }
    uint16_t v;
    std::memcpy(&v, row + 512 + (e - 512) * 2, 2);
    return bf(v);
  };
  parallel_for(int64_t(n) * heads, default_threads(threads), [&](int64_t unit) {
    const int b = int(unit / heads);
    const int len = lens[b];
    float *o = out + unit * 512;
    if (len <= 0) {
      std::fill(o, o + 512, 0.0f);
      return;
    }
    const uint16_t *qh = q + unit * 576;
    std::vector<float> s(len);
    std::vector<int64_t> slot(len);
    float mx = -INFINITY;
    for (int j = 0; j < len; ++j) {
      slot[j] = int64_t(tables[int64_t(b) * stride + j / bs]) * bs + j % bs;
      float acc = 0.0f;
      for (int e = 0; e < 576; ++e) acc += bf(qh[e]) * val(slot[j], e);
      s[j] = acc * scale;
      mx = std::max(mx, s[j]);
    }
    float sum = 0.0f;
    for (int j = 0; j < len; ++j) sum += std::exp(s[j] - mx);
    for (int j = 0; j < len; ++j) s[j] = std::exp(s[j] - mx) / sum;
    for (int e = 0; e < 512; ++e) {
      float acc = 0.0f;
      for (int j = 0; j < len; ++j) acc += s[j] * val(slot[j], e);
      o[e] = acc;
    }
  });
}

// General packed-MLA attention over query rows: the BF16 window attention with
// learned sinks (sliding_window_probe.cpp:144-163) and the packed C8 sparse
// attention with learned sinks (packed_cache_probe.cpp:47-66). Row t of
// sequence s (rows cu_q[s]..cu_q[s+1]-1, or row = s when cu_q is null) sees
// causal = kv_lens[s] - count + (t - start) + 1 keys (openpangu_attention_metadata.h:20-22).
// Dense (indices null): positions [max(0, causal - window), causal), window 0 =
// unbounded. Sparse: the logical positions indices[t][j], j < min(causal, topk),
// that are >= 0 (openpangu_attention_metadata.h:13-33). Sink rows (keys [n,576],
// values [n,512] bf16) join every row's softmax. out: fp32 [rows, heads, 512];
// a row with neither keys nor sinks is zero.
void oracle_mla_attention(const uint16_t *q, const void *cache, int32_t c8, const int32_t *tables,
                          int32_t stride, const int32_t *cu_q, const int32_t *kv_lens,
                          int32_t num_seqs, int32_t num_rows, const int32_t *indices, int32_t topk,
                          int32_t window, const uint16_t *sink_k, const uint16_t *sink_v,
                          int32_t n_sinks, float *out, int32_t heads, int32_t bs, float scale,
                          int32_t threads) {
  auto val = [&](int64_t slot, int e) -> float {
    if (!c8) return bf(static_cast<const uint16_t *>(cache)[slot * 576 + e]);
    const uint8_t *row = static_cast<const uint8_t *>(cache) + slot * 656;
    if (e < 512) {
      float sc;
      std::memcpy(&sc, row + 640 + (e / 128) * 4, 4);
      return float(int8_t(row[e])) * sc;
    }
    uint16_t v;
    std::memcpy(&v, row + 512 + (e - 512) * 2, 2);
    return bf(v);
  };
  std::vector<int> row_seq(num_rows), row_pos(num_rows);
  for (int s = 0; s < num_seqs; ++s) {
    const int start = cu_q ? cu_q[s] : s, end = cu_q ? cu_q[s + 1] : s + 1;
    for (int t = start; t < end && t < num_rows; ++t) {
      row_seq[t] = s;
      row_pos[t] = kv_lens[s] - (end - start) + (t - start);  // position of row t
    }
  }
  parallel_for(int64_t(num_rows) * heads, default_threads(threads), [&](int64_t unit) {
    const int t = int(unit / heads);
    const int seq = row_seq[t];
    const int causal = std::max(0, row_pos[t] + 1);
    std::vector<int64_t> slots;
    if (indices) {
      for (int j = 0; j < std::min(causal, topk); ++j) {
        const int pos = indices[int64_t(t) * topk + j];
        if (pos < 0) continue;
        slots.push_back(int64_t(tables[int64_t(seq) * stride + pos / bs]) * bs + pos % bs);
      }
    } else {
      const int lo = window > 0 ? std::max(0, causal - window) : 0;
      for (int pos = lo; pos < causal; ++pos)
        slots.push_back(int64_t(tables[int64_t(seq) * stride + pos / bs]) * bs + pos % bs);
    }
    const int nk = int(slots.size()), n = nk + n_sinks;
    float *o = out + unit * 512;
    if (n == 0) {
      std::fill(o, o + 512, 0.0f);
      return;
    }
    const uint16_t *qh = q + unit * 576;
    std::vector<float> sc(n);
    float mx = -INFINITY;
    for (int j = 0; j < n; ++j) {
      float acc = 0.0f;
      if (j < nk)
        for (int e = 0; e < 576; ++e) acc += bf(qh[e]) * val(slots[j], e);
      else
        for (int e = 0; e < 576; ++e) acc += bf(qh[e]) * bf(sink_k[int64_t(j - nk) * 576 + e]);
      sc[j] = acc * scale;
      mx = std::max(mx, sc[j]);
    }
    float sum = 0.0f;
    for (int j = 0; j < n; ++j) sum += std::exp(sc[j] - mx);
    for (int j = 0; j < n; ++j) sc[j] = std::exp(sc[j] - mx) / sum;
    for (int e = 0; e < 512; ++e) {
      float acc = 0.0f;
      for (int j = 0; j < n; ++j)
        acc += sc[j] * (j < nk ? val(slots[j], e) : bf(sink_v[int64_t(j - nk) * 512 + e]));
      o[e] = acc;
    }
  });
}

int32_t oracle_hardware_threads(void) { return default_threads(0); }

}  // extern "C"
