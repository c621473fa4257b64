// Qwen attention producer: per-head zero-centred RMS norm of q and k, partial
// RoPE on the first 64 of 256 channels, and the sigmoid output gate, in one
// launch. It computes what inferfabric_acl_attention_qk_prepare builds out of
// ACLNN steps (native/src/inferfabric_acl.cpp:1236-1341; CPU statement
// crates/inferfabric-cli/src/npu_probe/attention.rs:35-64):
//   packed q [batch, 8, 512] bf16: per head 256 query channels, then 256 gate channels
//   k        [batch, 2, 256] bf16
//   norm  n_j = bf16(x_j * (1 / sqrt(mean(x^2) + 1e-6)) * gamma_j)   (gamma fp32 = 1 + w)
//   rope  for j < 32, angle = position * f_j, f_j = 1 / 1e7^(j / 32),
//         c = bf16(cos angle), s = bf16(sin angle):
//         out_j      = bf16(bf16(n_j * c) - bf16(n_{j+32} * s))
//         out_{j+32} = bf16(bf16(n_{j+32} * c) + bf16(n_j * s))
//         out_j = n_j for 64 <= j < 256
//   gate  g = bf16(sigmoid(packed q gate channel))
// One workgroup per request, one wave per head (8 q heads, then 2 k heads);
// lane l owns channels 4l..4l+3, so a rotation pair (j, j+32) sits in lanes
// l and l ^ 8. HBM-bound: 8 KiB + 1 KiB in, 4 KiB + 1 KiB + 4 KiB out per request.
#include "common.h"
#include "ifattn_internal.h"

#include <cmath>

namespace ifattn {
namespace {

constexpr int kQHeads = 8, kKHeads = 2, kHd = 256;

struct QkParams {
  const uint16_t *packed_q;
  const uint16_t *k;
  const float *q_gamma;
  const float *k_gamma;
  const int64_t *positions;
  uint16_t *q_out;
  uint16_t *k_out;
  uint16_t *gate;
  float freq[32];
};

__device__ __forceinline__ float bf(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

__global__ __launch_bounds__(64 * (kQHeads + kKHeads)) void qk_norm_rope_gate_kernel(QkParams p) {
  const int r = blockIdx.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool is_q = w < kQHeads;
  const int h = is_q ? w : w - kQHeads;
  const uint16_t *src = is_q ? p.packed_q + (int64_t(r) * kQHeads + h) * 2 * kHd
                             : p.k + (int64_t(r) * kKHeads + h) * kHd;
  const float *gamma = is_q ? p.q_gamma : p.k_gamma;
  uint16_t *dst = is_q ? p.q_out + (int64_t(r) * kQHeads + h) * kHd
                       : p.k_out + (int64_t(r) * kKHeads + h) * kHd;
  const u32x2 raw = *reinterpret_cast<const u32x2 *>(src + 4 * lane);
  float x[4] = {bf16_bits_to_f32(raw[0] & 0xFFFFu), bf16_bits_to_f32(raw[0] >> 16),
                bf16_bits_to_f32(raw[1] & 0xFFFFu), bf16_bits_to_f32(raw[1] >> 16)};
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) ss = wave_sum_xor(ss, m);
  const float inv = 1.0f / sqrtf(ss / float(kHd) + 1e-6f);
  const float4 g4 = *reinterpret_cast<const float4 *>(gamma + 4 * lane);
  const float gm[4] = {g4.x, g4.y, g4.z, g4.w};
  float n[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) n[i] = bf((x[i] * inv) * gm[i]);
  // Rotation: lanes 0..7 hold the real halves (channels 0..31), lanes 8..15
  // the imaginary halves (32..63); each lane fetches its partner's values.
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float other = __shfl_xor(n[i], 8, 64);
    if (lane < 16) {
      const int j = 4 * (lane & 7) + i;
      const float angle = float(p.positions[r]) * p.freq[j];
      const float c = bf(cosf(angle)), s = bf(sinf(angle));
      o[i] = lane < 8 ? bf(bf(n[i] * c) - bf(other * s)) : bf(bf(n[i] * c) + bf(other * s));
    } else {
      o[i] = n[i];
    }
  }
  *reinterpret_cast<u32x2 *>(dst + 4 * lane) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  if (is_q) {
    const u32x2 gr = *reinterpret_cast<const u32x2 *>(src + kHd + 4 * lane);
    const float gv[4] = {bf16_bits_to_f32(gr[0] & 0xFFFFu), bf16_bits_to_f32(gr[0] >> 16),
                         bf16_bits_to_f32(gr[1] & 0xFFFFu), bf16_bits_to_f32(gr[1] >> 16)};
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = 1.0f / (1.0f + expf(-gv[i]));
    *reinterpret_cast<u32x2 *>(p.gate + (int64_t(r) * kQHeads + h) * kHd + 4 * lane) =
        u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
  }
}

}  // namespace
}  // namespace ifattn

using namespace ifattn;

extern "C" int32_t ifattn_qk_norm_rope_gate_bf16(const void *packed_q, const void *k,
                                                 const float *q_gamma, const float *k_gamma,
                                                 const int64_t *positions, void *q_out, void *k_out,
                                                 void *gate, int64_t batch, void *stream) {
  if (batch <= 0 || batch > 64)
    return fail(IFATTN_EINVAL, "qk norm rope gate: batch 1..64");
  if (!packed_q || !k || !q_gamma || !k_gamma || !positions || !q_out || !k_out || !gate)
    return fail(IFATTN_EINVAL, "qk norm rope gate: null pointer");
  if (!aligned8(packed_q) || !aligned8(k) || !aligned16(q_gamma) || !aligned16(k_gamma) ||
      !aligned8(positions) || !aligned8(q_out) || !aligned8(k_out) || !aligned8(gate))
    return fail(IFATTN_EINVAL, "qk norm rope gate: misaligned tensor");
  QkParams p{};
  p.packed_q = static_cast<const uint16_t *>(packed_q);
  p.k = static_cast<const uint16_t *>(k);
  p.q_gamma = q_gamma;
  p.k_gamma = k_gamma;
  p.positions = positions;
  p.q_out = static_cast<uint16_t *>(q_out);
  p.k_out = static_cast<uint16_t *>(k_out);
  p.gate = static_cast<uint16_t *>(gate);
  // Inverse frequencies in fp32 on the host, as the reference builds its table
  // (inferfabric_acl.cpp:1250-1252); they travel in the kernel arguments.
  for (int i = 0; i < 32; ++i) p.freq[i] = 1.0f / std::pow(10000000.0f, float(i) / 32.0f);
  qk_norm_rope_gate_kernel<<<unsigned(batch), 64 * (kQHeads + kKHeads), 0,
                             static_cast<hipStream_t>(stream)>>>(p);
  return launch_status("qk norm rope gate");
}
