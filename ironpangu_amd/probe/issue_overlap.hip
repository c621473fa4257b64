// Issue-overlap probe for the measurement leg of bench.py (not part of the
// operator library): how MFMA, VALU, transcendental and LDS-read work of the
// prefill kernel's tile loop share one SIMD. Each mode runs 256 workgroups of
// eight waves (two per SIMD) for `iters` iterations; an iteration is the work
// named by the mode. Results (time per iteration) tell whether work of one kind
// hides behind another: in the same wave with the instructions interleaved, or
// in the other wave of the SIMD.
//
// Modes (per wave and iteration):
//   0  16 MFMA 16x16x32 bf16 (eight independent accumulators)
//   1  32 v_exp_f32
//   2  32 v_fma_f32
//   3  waves 0-3: the MFMAs of mode 0; waves 4-7 (the other wave of each SIMD): mode 1
//   4  waves 0-3: mode 0; waves 4-7: mode 2
//   5  mode 0 and mode 1 in one wave, two exponentials after each MFMA
//   6  mode 0 and mode 2 in one wave, two FMAs after each MFMA
//   7  8 ds_read_b128, conflict-free (the K-operand pattern)
//   8  8 pairs of ds_read_b64_tr_b16 (the transposing V-operand pattern)
//   9  8 ds_read_b128 feeding 16 MFMAs
// Results are folded into a value stored only if it matches an impossible one.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef const __attribute__((address_space(3))) char lds_char;

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// One wave's loop: MFMAs (MF), exponentials (EX) or FMAs (FM) per MFMA slot,
// operands from LDS with pattern LD (0: registers, 1: K pattern, 2: V pattern).
template <bool MF, bool EX, bool FM, int LD>
__device__ __forceinline__ float wave_loop(const uint8_t *lds, int iters, int lane) {
  const u32x4 q0 = {uint32_t(lane), 1, 2, 3}, q1 = {3, uint32_t(lane), 1, 2};
  f32x4 acc[8] = {};
  float e[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) e[i] = -0.001f * float(lane + i);
  u32x4 x = {0, 0, 0, 0};
  const int c = lane & 15, g = lane >> 4;
  // K pattern: row c, chunk g of a 256-B row, XOR-swizzled by the row.
  const uint32_t kbase = uint32_t(c) * 256 + 16 * uint32_t(g ^ c);
  // V pattern: rows 4g + c/4 and +16, dims 4(c&3) + 16b, swizzle of the prefill ring.
  const int vrow = 4 * g + (c >> 2);
  const int vkey = ((vrow << 1) | ((vrow >> 3) & 1)) & 15;
  for (int it = 0; it < iters; ++it) {
    u32x4 k[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (LD == 1) {
        k[r] = *reinterpret_cast<const u32x4 *>(lds + ((kbase + r * 4096 + it * 64) & 65535));
      } else if (LD == 2) {
        const int d = 16 * r + 4 * (c & 3);
        const uint32_t o = (uint32_t(vrow) * 256 + 16 * uint32_t((d >> 3) ^ vkey) + 2 * (d & 7) +
                            uint32_t(it & 3) * 16384) & 65535;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)((lds_char *)lds + o));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)((lds_char *)lds + o + 4096));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        k[r] = u32x4{l2[0], l2[1], h2[0], h2[1]};
      } else {
        k[r] = q0 + uint32_t(r);  // loop-invariant operands
      }
    }
    if (LD != 0 && !MF) {
#pragma unroll
      for (int r = 0; r < 8; ++r) x ^= k[r];
    }
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if (MF) acc[m & 7] = mfma(k[m & 7], (m & 1) ? q0 : q1, acc[m & 7]);
      if (EX) {
        e[(2 * m) & 15] = __builtin_amdgcn_exp2f(e[(2 * m) & 15]) - 1.0f;
        e[(2 * m + 1) & 15] = __builtin_amdgcn_exp2f(e[(2 * m + 1) & 15]) - 1.0f;
      }
      if (FM) {
        e[(2 * m) & 15] = __builtin_fmaf(e[(2 * m) & 15], 0.999f, -0.001f);
        e[(2 * m + 1) & 15] = __builtin_fmaf(e[(2 * m + 1) & 15], 0.999f, -0.001f);
      }
    }
    if (MF && (EX || FM)) {  // keep one MFMA then its VALU work, in order
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, EX ? 4 : 2, 0);
      }
    }
  }
  float s = float(x[0] ^ x[1] ^ x[2] ^ x[3]);
#pragma unroll
  for (int m = 0; m < 8; ++m) s += acc[m][0] + acc[m][3];
#pragma unroll
  for (int i = 0; i < 16; ++i) s += e[i];
  return s;
}

template <int MODE>
__global__ __launch_bounds__(512) void issue_kernel(float *sink, int iters) {
  __shared__ __align__(16) uint8_t lds[65536];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  for (int i = threadIdx.x; i < 65536 / 4; i += 512) reinterpret_cast<uint32_t *>(lds)[i] = i * 2654435761u;
  __syncthreads();
  float s;
  if constexpr (MODE == 0) s = wave_loop<true, false, false, 0>(lds, iters, lane);
  else if constexpr (MODE == 1) s = wave_loop<false, true, false, 0>(lds, iters, lane);
  else if constexpr (MODE == 2) s = wave_loop<false, false, true, 0>(lds, iters, lane);
  else if constexpr (MODE == 3)  // waves w and w + 4 share a SIMD
    s = w < 4 ? wave_loop<true, false, false, 0>(lds, iters, lane) : wave_loop<false, true, false, 0>(lds, iters, lane);
  else if constexpr (MODE == 4)
    s = w < 4 ? wave_loop<true, false, false, 0>(lds, iters, lane) : wave_loop<false, false, true, 0>(lds, iters, lane);
  else if constexpr (MODE == 5) s = wave_loop<true, true, false, 0>(lds, iters, lane);
  else if constexpr (MODE == 6) s = wave_loop<true, false, true, 0>(lds, iters, lane);
  else if constexpr (MODE == 7) s = wave_loop<false, false, false, 1>(lds, iters, lane);
  else if constexpr (MODE == 8) s = wave_loop<false, false, false, 2>(lds, iters, lane);
  else s = wave_loop<true, false, false, 1>(lds, iters, lane);
  if (s == 1234.5f) sink[blockIdx.x] = s;
}

template <int MODE>
void launch(float *sink, int iters, hipStream_t s) {
  issue_kernel<MODE><<<256, 512, 0, s>>>(sink, iters);
}

}  // namespace

extern "C" int32_t ifattn_probe_issue(int32_t mode, int32_t iters, void *sink, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  float *f = static_cast<float *>(sink);
  switch (mode) {
    case 0: launch<0>(f, iters, s); break;
    case 1: launch<1>(f, iters, s); break;
    case 2: launch<2>(f, iters, s); break;
    case 3: launch<3>(f, iters, s); break;
    case 4: launch<4>(f, iters, s); break;
    case 5: launch<5>(f, iters, s); break;
    case 6: launch<6>(f, iters, s); break;
    case 7: launch<7>(f, iters, s); break;
    case 8: launch<8>(f, iters, s); break;
    case 9: launch<9>(f, iters, s); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
