// IFKernelV1-layout operator plug-ins over the ifattn C ABI, in two versions:
// abi_version 1 (the reference loader's: I8/BF16/F32 only, integer ports as I8
// byte views, in-place caches declared write-only) and abi_version 2 (I32/I64
// dtypes and read-write access).
// prepare: descriptor validation in the manner of the reference loader
// (native/src/compiled_kernel.cpp:20-41,71-83) plus per-contract shape checks,
// host state only. enqueue: one call into the launchers, no allocation, no
// synchronization, no device reads on the host.
#include <cmath>
#include <cstring>
#include <new>
#include <string>

#include "../../include/ifattn.h"
#include "../../include/inferfabric_kernel_v1.h"
#include "ifattn_internal.h"

namespace {

enum Op : int {
  kWriteBf16 = 0,
  kWriteC8,
  kDecodeBf16,
  kDecodeC8,
  kPrefillBf16,
  kMlaBf16,
  kMlaC8,
  kMlaWriteC8,
  kMlaNormRopeBf16,
  kMlaNormRopeC8,
  kMlaWindow512,
  kMlaWindow2048,
  kMlaSparseC8,
  kGatedBf16,
  kOpCount
};

const char *const kContract[kOpCount] = {
    "inferfabric.kv_cache_write.bf16.v2",   "inferfabric.kv_cache_write.c8.v2",
    "inferfabric.paged_decode.gqa.bf16.v2", "inferfabric.paged_decode.gqa.c8.v2",
    "inferfabric.varlen_prefill.bf16.v2",   "inferfabric.mla_decode.bf16.v2",
    "inferfabric.mla_decode.c8.v2",         "inferfabric.mla_cache_write.c8.v2",
    "inferfabric.mla_norm_rope_cache.bf16.v2", "inferfabric.mla_norm_rope_cache.c8.v2",
    "inferfabric.mla_window_attention.w512.bf16.v2",
    "inferfabric.mla_window_attention.w2048.bf16.v2",
    "inferfabric.mla_sparse_attention.c8.v2",
    "inferfabric.paged_attention.qwen_gated.bf16.v2",
};
// The same operators under abi_version 1 (the reference loader's version):
// contract names end in ".v1" and integer ports travel as I8 byte views.
const char *const kContractV1[kOpCount] = {
    "inferfabric.kv_cache_write.bf16.v1",   "inferfabric.kv_cache_write.c8.v1",
    "inferfabric.paged_decode.gqa.bf16.v1", "inferfabric.paged_decode.gqa.c8.v1",
    "inferfabric.varlen_prefill.bf16.v1",   "inferfabric.mla_decode.bf16.v1",
    "inferfabric.mla_decode.c8.v1",         "inferfabric.mla_cache_write.c8.v1",
    "inferfabric.mla_norm_rope_cache.bf16.v1", "inferfabric.mla_norm_rope_cache.c8.v1",
    "inferfabric.mla_window_attention.w512.bf16.v1",
    "inferfabric.mla_window_attention.w2048.bf16.v1",
    "inferfabric.mla_sparse_attention.c8.v1",
    nullptr,  // reads and writes its caches in one call: no version-1 form
};
constexpr const char *kTarget = "gfx950";

// Version-1 port map of each operator: input ports that carry integers (an I8
// byte view whose last extent is 4x the int32 extent, or 8x for the int64 slot
// mappings) and output ports that the operator updates in place (declared
// write-only in version 1: the operator writes the mapped rows and reads
// nothing else of them).
struct PortMap {
  uint8_t int32_inputs, int64_inputs;  // bit i = input port i
  uint8_t in_place_outputs;            // bit i = output port i
};
constexpr PortMap kPorts[kOpCount] = {
    {0x00, 0x04, 0x03},  // kv write bf16: slots ; k, v caches
    {0x00, 0x04, 0x0f},  // kv write c8: slots ; caches and scales
    {0x18, 0x00, 0x00},  // decode bf16: tables, lengths
    {0x60, 0x00, 0x00},  // decode c8
    {0x38, 0x00, 0x00},  // prefill: tables, cu_seqlens, kv_lens
    {0x0c, 0x00, 0x00},  // mla decode bf16
    {0x0c, 0x00, 0x00},  // mla decode c8
    {0x00, 0x02, 0x01},  // mla c8 row write
    {0x00, 0x10, 0x01},  // norm/rope writer bf16
    {0x00, 0x10, 0x01},  // norm/rope writer c8
    {0x1c, 0x00, 0x00},  // window 512
    {0x1c, 0x00, 0x00},  // window 2048
    {0x3c, 0x00, 0x00},  // sparse: indices, tables, cu_seqlens, kv_lens
    {0x00, 0x00, 0x00},
};

struct State {
  int op;
  IFKernelTensorV1 inputs[8], outputs[4];  // as version 2 sees them
  uint64_t workspace;
  int32_t slot_dtype;
  int64_t rows, row_bytes, num_slots, num_blocks;
  int32_t n, q_heads, kv_heads, head_dim, block_size, stride, max_ctx, total_q;
  int32_t window, topk, n_sinks;
  float scale;
};

struct Reject {
  const char *what;
};
void require(bool ok, const char *what) {
  if (!ok) throw Reject{what};
}

uint64_t elem_bytes(uint32_t dtype) {
  switch (dtype) {
    case IF_KERNEL_DTYPE_I8: return 1;
    case IF_KERNEL_DTYPE_BF16: return 2;
    case IF_KERNEL_DTYPE_F32: return 4;
    case IF_KERNEL_DTYPE_I32: return 4;
    case IF_KERNEL_DTYPE_I64: return 8;
    default: return 0;
  }
}

void check_tensor(const IFKernelTensorV1 &t, uint32_t dtype, uint32_t access, uint32_t rank) {
  require(t.struct_bytes == sizeof(IFKernelTensorV1), "tensor descriptor size");
  require(t.data != nullptr, "tensor data pointer");
  require(t.rank == rank, "tensor rank");
  require(t.dtype == dtype, "tensor dtype");
  require(t.access == access, "tensor access");
  uint64_t stride = 1;
  for (uint32_t i = t.rank; i-- > 0;) {
    require(t.shape[i] > 0, "tensor extent must be positive");
    require(t.strides[i] == int64_t(stride), "tensor must be contiguous");
    require(uint64_t(t.shape[i]) <= UINT64_MAX / stride, "tensor shape overflow");
    stride *= uint64_t(t.shape[i]);
  }
  const uint64_t eb = elem_bytes(dtype);
  require(stride <= UINT64_MAX / eb && stride * eb <= t.allocation_bytes, "tensor allocation bound");
}

uint64_t nbytes(const IFKernelTensorV1 &t) {
  uint64_t n = elem_bytes(t.dtype);
  for (uint32_t i = 0; i < t.rank; ++i) n *= uint64_t(t.shape[i]);
  return n;
}

bool overlap(const IFKernelTensorV1 &a, const IFKernelTensorV1 &b) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a.data), y = reinterpret_cast<uintptr_t>(b.data);
  return x < y + nbytes(b) && y < x + nbytes(a);
}

void check_slots(const IFKernelTensorV1 &t, int64_t rows, State &s) {
  require(t.struct_bytes == sizeof(IFKernelTensorV1) && t.data && t.rank == 1 &&
              t.access == IF_KERNEL_ACCESS_READ &&
              (t.dtype == IF_KERNEL_DTYPE_I64 || t.dtype == IF_KERNEL_DTYPE_I32),
          "slot_mapping: I64 or I32 [rows], read");
  check_tensor(t, t.dtype, IF_KERNEL_ACCESS_READ, 1);
  require(t.shape[0] == rows, "slot_mapping length differs from rows");
  s.slot_dtype = t.dtype == IF_KERNEL_DTYPE_I64 ? IFATTN_DTYPE_I64 : IFATTN_DTYPE_I32;
}

bool same_shape(const IFKernelTensorV1 &a, const IFKernelTensorV1 &b) {
  if (a.rank != b.rank) return false;
  for (uint32_t i = 0; i < a.rank; ++i)
    if (a.shape[i] != b.shape[i]) return false;
  return true;
}

void prepare_op(State &s, const IFKernelTensorV1 *in, uint32_t nin, const IFKernelTensorV1 *out,
                uint32_t nout) {
  constexpr uint32_t R = IF_KERNEL_ACCESS_READ, W = IF_KERNEL_ACCESS_WRITE,
                     RW = IF_KERNEL_ACCESS_READ_WRITE;
  constexpr uint32_t BF = IF_KERNEL_DTYPE_BF16, I8 = IF_KERNEL_DTYPE_I8, F32 = IF_KERNEL_DTYPE_F32,
                     I32 = IF_KERNEL_DTYPE_I32;
  switch (s.op) {
    case kWriteBf16:
    case kWriteC8: {
      const bool c8 = s.op == kWriteC8;
      require(nin == 3 && nout == (c8 ? 4u : 2u), "write: 3 inputs, 2 (bf16) or 4 (c8) outputs");
      check_tensor(in[0], BF, R, 3);
      check_tensor(in[1], BF, R, 3);
      require(same_shape(in[0], in[1]), "k/v rows differ");
      s.rows = in[0].shape[0];
      check_slots(in[2], s.rows, s);
      check_tensor(out[0], c8 ? I8 : BF, RW, 4);
      check_tensor(out[1], c8 ? I8 : BF, RW, 4);
      require(same_shape(out[0], out[1]), "k/v caches differ");
      require(out[0].shape[2] == in[0].shape[1] && out[0].shape[3] == in[0].shape[2],
              "cache row differs from input row");
      s.kv_heads = int32_t(in[0].shape[1]);
      s.head_dim = int32_t(in[0].shape[2]);
      s.num_slots = out[0].shape[0] * out[0].shape[1];
      s.row_bytes = int64_t(s.kv_heads) * s.head_dim * 2;
      require(c8 || s.row_bytes % 16 == 0, "bf16 row must be a multiple of 16 bytes");
      if (c8) {
        check_tensor(out[2], F32, RW, 3);
        check_tensor(out[3], F32, RW, 3);
        require(out[2].shape[0] == out[0].shape[0] && out[2].shape[1] == out[0].shape[1] &&
                    out[2].shape[2] == out[0].shape[2] && same_shape(out[2], out[3]),
                "scales must be [blocks, block_size, kv_heads]");
        require(s.head_dim % 8 == 0 && s.head_dim <= 512, "c8 head_dim: multiple of 8, <= 512");
      }
      return;
    }
    case kDecodeBf16:
    case kDecodeC8: {
      const bool c8 = s.op == kDecodeC8;
      require(nin == (c8 ? 7u : 5u) && nout == 1, "decode: 5 (bf16) or 7 (c8) inputs, 1 output");
      check_tensor(in[0], BF, R, 3);
      check_tensor(in[1], c8 ? I8 : BF, R, 4);
      check_tensor(in[2], c8 ? I8 : BF, R, 4);
      require(same_shape(in[1], in[2]), "k/v caches differ");
      const int t = c8 ? 5 : 3;
      if (c8) {
        check_tensor(in[3], F32, R, 3);
        check_tensor(in[4], F32, R, 3);
        require(same_shape(in[3], in[4]) && in[3].shape[0] == in[1].shape[0] &&
                    in[3].shape[1] == in[1].shape[1] && in[3].shape[2] == in[1].shape[2],
                "scales must be [blocks, block_size, kv_heads]");
      }
      check_tensor(in[t], I32, R, 2);
      check_tensor(in[t + 1], I32, R, 1);
      check_tensor(out[0], BF, W, 3);
      s.n = int32_t(in[0].shape[0]);
      s.q_heads = int32_t(in[0].shape[1]);
      s.head_dim = int32_t(in[0].shape[2]);
      s.num_blocks = in[1].shape[0];
      s.block_size = int32_t(in[1].shape[1]);
      s.kv_heads = int32_t(in[1].shape[2]);
      require(in[1].shape[3] == s.head_dim, "cache head_dim differs from q");
      require(in[t].shape[0] >= s.n && in[t + 1].shape[0] >= s.n, "tables/lengths shorter than q");
      s.stride = int32_t(in[t].shape[1]);
      require(int64_t(s.stride) * s.block_size <= (int64_t(1) << 20), "max_context above 1M");
      s.max_ctx = s.stride * s.block_size;
      require(same_shape(out[0], in[0]), "out must match q");
      s.scale = 1.0f / std::sqrt(float(s.head_dim));
      s.workspace = ifattn_paged_decode_workspace_size(s.n, s.q_heads, s.head_dim, s.max_ctx);
      return;
    }
    case kPrefillBf16: {
      require(nin == 6 && nout == 1, "prefill: 6 inputs, 1 output");
      check_tensor(in[0], BF, R, 3);
      check_tensor(in[1], BF, R, 4);
      check_tensor(in[2], BF, R, 4);
      require(same_shape(in[1], in[2]), "k/v caches differ");
      check_tensor(in[3], I32, R, 2);
      check_tensor(in[4], I32, R, 1);
      check_tensor(in[5], I32, R, 1);
      check_tensor(out[0], BF, W, 3);
      s.total_q = int32_t(in[0].shape[0]);
      s.q_heads = int32_t(in[0].shape[1]);
      s.head_dim = int32_t(in[0].shape[2]);
      s.num_blocks = in[1].shape[0];
      s.block_size = int32_t(in[1].shape[1]);
      s.kv_heads = int32_t(in[1].shape[2]);
      require(in[1].shape[3] == s.head_dim, "cache head_dim differs from q");
      s.n = int32_t(in[4].shape[0] - 1);
      require(s.n >= 1 && in[5].shape[0] >= s.n && in[3].shape[0] >= s.n,
              "cu_seqlens [n+1], kv_lens [n], tables [n, entries]");
      s.stride = int32_t(in[3].shape[1]);
      require(int64_t(s.stride) * s.block_size <= 262144, "max_kv_len above 262144");
      s.max_ctx = s.stride * s.block_size;
      require(same_shape(out[0], in[0]), "out must match q");
      s.scale = 1.0f / std::sqrt(float(s.head_dim));
      s.workspace = ifattn_varlen_prefill_workspace_size(s.n, s.total_q, s.q_heads, s.head_dim,
                                                         s.max_ctx);
      return;
    }
    case kMlaBf16:
    case kMlaC8: {
      const bool c8 = s.op == kMlaC8;
      require(nin == 4 && nout == 1, "mla decode: 4 inputs, 1 output");
      check_tensor(in[0], BF, R, 3);
      require(in[0].shape[2] == 576, "q must be [n, heads, 576]");
      check_tensor(in[1], c8 ? I8 : BF, R, 3);
      require(in[1].shape[2] == (c8 ? 656 : 576), "cache row width 576 (bf16) or 656 (c8)");
      check_tensor(in[2], I32, R, 2);
      check_tensor(in[3], I32, R, 1);
      check_tensor(out[0], BF, W, 3);
      s.n = int32_t(in[0].shape[0]);
      s.q_heads = int32_t(in[0].shape[1]);
      s.num_blocks = in[1].shape[0];
      s.block_size = int32_t(in[1].shape[1]);
      require(in[2].shape[0] >= s.n && in[3].shape[0] >= s.n, "tables/lengths shorter than q");
      s.stride = int32_t(in[2].shape[1]);
      require(int64_t(s.stride) * s.block_size <= (int64_t(1) << 20), "max_context above 1M");
      s.max_ctx = s.stride * s.block_size;
      require(out[0].shape[0] == s.n && out[0].shape[1] == s.q_heads && out[0].shape[2] == 512,
              "out must be [n, heads, 512]");
      s.scale = 1.0f / std::sqrt(192.0f);
      s.workspace = ifattn_mla_decode_workspace_size(s.n, s.q_heads, s.max_ctx, s.block_size);
      return;
    }
    case kMlaWriteC8: {
      require(nin == 2 && nout == 1, "mla write: 2 inputs, 1 output");
      check_tensor(in[0], BF, R, 2);
      require(in[0].shape[1] == 576, "rows must be [rows, 576]");
      s.rows = in[0].shape[0];
      check_slots(in[1], s.rows, s);
      check_tensor(out[0], I8, RW, 3);
      require(out[0].shape[2] == 656, "cache must be [blocks, block_size, 656]");
      s.num_slots = out[0].shape[0] * out[0].shape[1];
      return;
    }
    case kMlaNormRopeBf16:
    case kMlaNormRopeC8: {
      const bool c8 = s.op == kMlaNormRopeC8;
      require(nin == 5 && nout == 1, "mla norm/rope write: 5 inputs, 1 output");
      check_tensor(in[0], BF, R, 2);
      require(in[0].shape[1] == 576, "x must be [rows, 576]");
      s.rows = in[0].shape[0];
      require(s.rows >= 1 && s.rows <= 4096, "rows must be 1..4096");
      check_tensor(in[1], BF, R, 1);
      require(in[1].shape[0] == 512, "gamma must be [512]");
      check_tensor(in[2], BF, R, 2);
      check_tensor(in[3], BF, R, 2);
      require(in[2].shape[0] == s.rows && in[2].shape[1] == 64 && same_shape(in[2], in[3]),
              "cos/sin must be [rows, 64]");
      check_slots(in[4], s.rows, s);
      check_tensor(out[0], c8 ? I8 : BF, RW, 3);
      require(out[0].shape[2] == (c8 ? 656 : 576), "cache rows: 576 bf16 or 656 bytes");
      s.num_slots = out[0].shape[0] * out[0].shape[1];
      return;
    }
    case kMlaWindow512:
    case kMlaWindow2048:
    case kMlaSparseC8: {
      const bool sparse = s.op == kMlaSparseC8;
      const uint32_t t = sparse ? 3 : 2;  // first metadata port after q, cache (, indices)
      require(nin == t + 5 && nout == 1,
              sparse ? "mla sparse attention: 8 inputs, 1 output" : "mla window attention: 7 inputs, 1 output");
      check_tensor(in[0], BF, R, 3);
      require(in[0].shape[2] == 576, "q must be [rows, heads, 576]");
      check_tensor(in[1], sparse ? I8 : BF, R, 3);
      require(in[1].shape[2] == (sparse ? 656 : 576), "cache rows: 576 bf16 or 656 bytes");
      s.total_q = int32_t(in[0].shape[0]);
      s.q_heads = int32_t(in[0].shape[1]);
      require(s.q_heads <= 16 && s.total_q < (1 << 20), "at most 16 heads and 2^20-1 rows");
      s.num_blocks = in[1].shape[0];
      s.block_size = int32_t(in[1].shape[1]);
      if (sparse) {
        check_tensor(in[2], I32, R, 2);
        require(in[2].shape[0] == s.total_q, "indices must be [rows, topk]");
        s.topk = int32_t(in[2].shape[1]);
      }
      check_tensor(in[t], I32, R, 2);
      check_tensor(in[t + 1], I32, R, 1);
      check_tensor(in[t + 2], I32, R, 1);
      s.n = int32_t(in[t + 1].shape[0] - 1);
      require(s.n >= 1 && in[t].shape[0] >= s.n && in[t + 2].shape[0] >= s.n,
              "tables [seqs, entries], cu_seqlens_q [seqs+1], kv_lens [seqs]");
      s.stride = int32_t(in[t].shape[1]);
      require(int64_t(s.stride) * s.block_size <= (int64_t(1) << 20), "max_context above 1M");
      s.max_ctx = s.stride * s.block_size;
      check_tensor(in[t + 3], BF, R, 2);
      check_tensor(in[t + 4], BF, R, 2);
      s.n_sinks = int32_t(in[t + 3].shape[0]);
      require(in[t + 3].shape[1] == 576 && in[t + 4].shape[0] == s.n_sinks &&
                  in[t + 4].shape[1] == 512 && s.n_sinks <= 128,
              "sinks: keys [n <= 128, 576], values [n, 512]");
      check_tensor(out[0], BF, W, 3);
      require(out[0].shape[0] == s.total_q && out[0].shape[1] == s.q_heads && out[0].shape[2] == 512,
              "out must be [rows, heads, 512]");
      s.window = s.op == kMlaWindow512 ? 512 : (s.op == kMlaWindow2048 ? 2048 : 0);
      s.scale = 1.0f / std::sqrt(192.0f);
      s.workspace = ifattn_mla_attention_workspace_size(s.total_q, s.q_heads, s.max_ctx, s.window,
                                                        s.topk, s.n_sinks, s.block_size);
      return;
    }
    case kGatedBf16: {
      require(nin == 7 && nout == 3, "gated attention: 7 inputs, 3 outputs");
      check_tensor(in[0], BF, R, 3);
      require(in[0].shape[1] == 8 && in[0].shape[2] == 256, "q must be [batch, 8, 256]");
      s.n = int32_t(in[0].shape[0]);
      require(s.n <= 64, "batch must be 1..64");
      check_tensor(in[1], BF, R, 2);
      check_tensor(in[2], BF, R, 2);
      require(in[1].shape[0] == s.n && in[1].shape[1] == 512 && same_shape(in[1], in[2]),
              "k, v rows must be [batch, 512]");
      check_tensor(in[3], BF, R, 3);
      require(same_shape(in[3], in[0]), "gate must match q");
      check_tensor(in[4], IF_KERNEL_DTYPE_I64, R, 1);
      require(in[4].shape[0] == s.n, "append must be [batch]");
      check_tensor(in[5], IF_KERNEL_DTYPE_I64, R, 2);
      check_tensor(in[6], F32, R, 2);
      require(in[5].shape[0] == s.n && same_shape(in[5], in[6]),
              "table (I64) and mask (F32) must be [batch, context]");
      s.max_ctx = int32_t(in[5].shape[1] <= 262144 ? in[5].shape[1] : 0);
      require(s.max_ctx > 0, "context must be 1..262144");
      check_tensor(out[0], BF, RW, 2);
      check_tensor(out[1], BF, RW, 2);
      require(out[0].shape[1] == 512 && same_shape(out[0], out[1]) && out[0].shape[0] <= 1048576,
              "keys, values must be [slots <= 2^20, 512]");
      s.num_slots = out[0].shape[0];
      check_tensor(out[2], BF, W, 3);
      require(same_shape(out[2], in[0]), "out must match q");
      s.workspace = ifattn_gated_paged_attention_workspace_size(s.n, s.max_ctx);
      return;
    }
    default:
      require(false, "unknown operator");
  }
}

// Version-1 descriptors -> the version-2 view prepare_op checks: integer byte
// views become I32/I64 tensors, in-place caches become read-write.
void widen_v1(int op, const IFKernelTensorV1 *in, uint32_t nin, const IFKernelTensorV1 *out,
              uint32_t nout, IFKernelTensorV1 *in2, IFKernelTensorV1 *out2) {
  const PortMap &m = kPorts[op];
  for (uint32_t i = 0; i < nin; ++i) {
    in2[i] = in[i];
    const bool i32 = m.int32_inputs >> i & 1, i64 = m.int64_inputs >> i & 1;
    require(in[i].dtype != IF_KERNEL_DTYPE_I32 && in[i].dtype != IF_KERNEL_DTYPE_I64 &&
                in[i].access != IF_KERNEL_ACCESS_READ_WRITE,
            "version 1 carries no I32/I64 dtypes and no read-write access");
    if (!i32 && !i64) continue;
    require(in[i].dtype == IF_KERNEL_DTYPE_I8 && in[i].rank >= 1 && in[i].rank <= 8,
            "version 1 integer port: I8 byte view");
    const int64_t w = i64 ? 8 : 4;
    const uint32_t last = in[i].rank - 1;
    require(in[i].shape[last] > 0 && in[i].shape[last] % w == 0,
            "version 1 integer port: last extent a multiple of the integer size");
    in2[i].dtype = i64 ? IF_KERNEL_DTYPE_I64 : IF_KERNEL_DTYPE_I32;
    in2[i].shape[last] = in[i].shape[last] / w;
    require(in[i].strides[last] == 1, "tensor must be contiguous");
    int64_t stride = 1;
    for (uint32_t d = in[i].rank; d-- > 0;) {
      require(d == last || in[i].strides[d] == in[i].strides[d + 1] * in[i].shape[d + 1],
              "tensor must be contiguous");
      in2[i].strides[d] = stride;
      stride *= in2[i].shape[d];
    }
  }
  for (uint32_t i = 0; i < nout; ++i) {
    out2[i] = out[i];
    require(out[i].dtype != IF_KERNEL_DTYPE_I32 && out[i].dtype != IF_KERNEL_DTYPE_I64 &&
                out[i].access == IF_KERNEL_ACCESS_WRITE,
            "version 1 outputs: write access, no I32/I64 dtypes");
    if (m.in_place_outputs >> i & 1) out2[i].access = IF_KERNEL_ACCESS_READ_WRITE;
  }
}

template <int OP, int VERSION>
int32_t prepare(const IFKernelTensorV1 *inputs, uint32_t input_count,
                const IFKernelTensorV1 *outputs, uint32_t output_count, IFKernelPreparedV1 *out) {
  if (!out) return ifattn::fail(IFATTN_EINVAL, "prepare: null output");
  *out = IFKernelPreparedV1{};
  if (!inputs || !outputs || input_count > 8 || output_count > 4)
    return ifattn::fail(IFATTN_EINVAL, "prepare: port count");
  State *s = new (std::nothrow) State{};
  if (!s) return ifattn::fail(IFATTN_EINVAL, "prepare: host allocation");
  s->op = OP;
  try {
    if (VERSION == 1) {
      widen_v1(OP, inputs, input_count, outputs, output_count, s->inputs, s->outputs);
      inputs = s->inputs;
      outputs = s->outputs;
    }
    prepare_op(*s, inputs, input_count, outputs, output_count);
    for (uint32_t i = 0; i < output_count; ++i) {
      for (uint32_t j = 0; j < input_count; ++j)
        require(!overlap(outputs[i], inputs[j]), "output aliases an input");
      for (uint32_t j = 0; j < i; ++j) require(!overlap(outputs[i], outputs[j]), "outputs alias");
    }
  } catch (const Reject &r) {
    delete s;
    return ifattn::fail(IFATTN_EINVAL, r.what);
  }
  if (VERSION != 1) {
    std::memcpy(s->inputs, inputs, sizeof(IFKernelTensorV1) * input_count);
    std::memcpy(s->outputs, outputs, sizeof(IFKernelTensorV1) * output_count);
  }
  out->state = s;
  out->workspace_bytes = s->workspace;
  out->workspace_alignment = 256;
  return IFATTN_OK;
}

int32_t enqueue(void *state, void *workspace, uint64_t bytes, void *stream) {
  State *s = static_cast<State *>(state);
  if (!s) return ifattn::fail(IFATTN_EINVAL, "enqueue: null state");
  if (bytes < s->workspace || (s->workspace && !workspace))
    return ifattn::fail(IFATTN_EWORKSPACE, "enqueue: workspace smaller than prepared");
  const IFKernelTensorV1 *in = s->inputs, *out = s->outputs;
  switch (s->op) {
    case kWriteBf16:
      return ifattn_kv_cache_write(in[0].data, in[1].data, out[0].data, out[1].data, in[2].data,
                                   s->slot_dtype, s->rows, s->row_bytes, s->num_slots, stream);
    case kWriteC8:
      return ifattn_kv_cache_write_c8(in[0].data, in[1].data, out[0].data, out[1].data,
                                      out[2].data, out[3].data, in[2].data, s->slot_dtype, s->rows,
                                      s->kv_heads, s->head_dim, s->num_slots, stream);
    case kDecodeBf16:
      return ifattn_paged_decode_bf16(in[0].data, in[1].data, in[2].data,
                                      static_cast<const int32_t *>(in[3].data), s->stride,
                                      static_cast<const int32_t *>(in[4].data), out[0].data, s->n,
                                      s->q_heads, s->kv_heads, s->head_dim, s->block_size,
                                      s->num_blocks, s->max_ctx, s->scale, workspace, bytes, stream);
    case kDecodeC8:
      return ifattn_paged_decode_c8(in[0].data, in[1].data, in[2].data, in[3].data, in[4].data,
                                    static_cast<const int32_t *>(in[5].data), s->stride,
                                    static_cast<const int32_t *>(in[6].data), out[0].data, s->n,
                                    s->q_heads, s->kv_heads, s->head_dim, s->block_size,
                                    s->num_blocks, s->max_ctx, s->scale, workspace, bytes, stream);
    case kPrefillBf16:
      return ifattn_varlen_prefill_bf16(
          in[0].data, in[1].data, in[2].data, static_cast<const int32_t *>(in[3].data), s->stride,
          static_cast<const int32_t *>(in[4].data), static_cast<const int32_t *>(in[5].data),
          out[0].data, s->n, s->total_q, s->total_q, s->max_ctx, s->q_heads, s->kv_heads,
          s->head_dim, s->block_size, s->num_blocks, s->scale, workspace, bytes, stream);
    case kMlaBf16:
    case kMlaC8:
      return (s->op == kMlaC8 ? ifattn_mla_decode_c8 : ifattn_mla_decode_bf16)(
          in[0].data, in[1].data, static_cast<const int32_t *>(in[2].data), s->stride,
          static_cast<const int32_t *>(in[3].data), out[0].data, s->n, s->q_heads, s->block_size,
          s->num_blocks, s->max_ctx, s->scale, workspace, bytes, stream);
    case kMlaWriteC8:
      return ifattn_mla_cache_write_c8(in[0].data, out[0].data, in[1].data, s->slot_dtype, s->rows,
                                       s->num_slots, stream);
    case kMlaNormRopeBf16:
    case kMlaNormRopeC8:
      // eps 1e-5: the epsilon the reference passes (resident_cache_writer.h:16).
      return ifattn_mla_norm_rope_cache_write(in[0].data, in[1].data, in[2].data, in[3].data,
                                              in[4].data, s->slot_dtype, s->rows, 1e-5f,
                                              out[0].data, s->op == kMlaNormRopeC8 ? 1 : 0,
                                              s->num_slots, stream);
    case kMlaWindow512:
    case kMlaWindow2048:
      return ifattn_mla_window_attention_bf16(
          in[0].data, in[1].data, static_cast<const int32_t *>(in[2].data), s->stride,
          static_cast<const int32_t *>(in[3].data), static_cast<const int32_t *>(in[4].data), s->n,
          s->total_q, s->window, in[5].data, in[6].data, s->n_sinks, out[0].data, s->q_heads,
          s->block_size, s->num_blocks, s->max_ctx, s->scale, workspace, bytes, stream);
    case kMlaSparseC8:
      return ifattn_mla_sparse_attention_c8(
          in[0].data, in[1].data, static_cast<const int32_t *>(in[2].data), s->topk,
          static_cast<const int32_t *>(in[3].data), s->stride,
          static_cast<const int32_t *>(in[4].data), static_cast<const int32_t *>(in[5].data), s->n,
          s->total_q, in[6].data, in[7].data, s->n_sinks, out[0].data, s->q_heads, s->block_size,
          s->num_blocks, s->max_ctx, s->scale, workspace, bytes, stream);
    case kGatedBf16:
      return ifattn_gated_paged_attention_bf16(
          in[0].data, in[1].data, in[2].data, in[3].data, out[0].data, out[1].data,
          static_cast<const int64_t *>(in[4].data), static_cast<const int64_t *>(in[5].data),
          static_cast<const float *>(in[6].data), out[2].data, s->n, s->num_slots, s->max_ctx,
          workspace, bytes, stream);
    default:
      return ifattn::fail(IFATTN_EINVAL, "enqueue: unknown operator");
  }
}

void release(void *state) { delete static_cast<State *>(state); }

template <int OP, int VERSION>
IFKernelV1 table() {
  return IFKernelV1{sizeof(IFKernelV1), uint32_t(VERSION),
                    VERSION == 1 ? kContractV1[OP] : kContract[OP], kTarget, &prepare<OP, VERSION>,
                    &enqueue, &release};
}

template <int... OPS>
struct Tables {
  const IFKernelV1 v1[kOpCount] = {table<OPS, 1>()...};
  const IFKernelV1 v2[kOpCount] = {table<OPS, 2>()...};
};
const Tables<0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13> kTables;
static_assert(kOpCount == 14, "one table entry per operator");

}  // namespace

extern "C" const IFKernelV1 *ifattn_kernel_v1_contract(const char *contract,
                                                       uint32_t requested_version) {
  if (!contract || (requested_version != 1 && requested_version != 2)) return nullptr;
  for (int i = 0; i < kOpCount; ++i) {
    const char *name = requested_version == 1 ? kContractV1[i] : kContract[i];
    if (name && std::strcmp(contract, name) == 0)
      return requested_version == 1 ? &kTables.v1[i] : &kTables.v2[i];
  }
  return nullptr;
}

extern "C" const IFKernelV1 *ifattn_kernel_v1_operator(int32_t index, uint32_t requested_version) {
  if (index < 0 || index >= kOpCount) return nullptr;
  if (requested_version == 2) return &kTables.v2[index];
  if (requested_version == 1 && kContractV1[index]) return &kTables.v1[index];
  return nullptr;
}
