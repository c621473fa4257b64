/* Operator plug-in ABI for the attention-path kernels.
 *
 * Same POD layout and calling contract as the reference's
 * native/include/inferfabric_kernel_v1.h:8-34 (the loader is
 * native/src/compiled_kernel.cpp:39-128), so an existing CompiledKernel loader
 * can dlopen these libraries unchanged. Interface declarations have to match
 * field for field; the text here is this project's own.
 *
 * Two versions of every operator, chosen by requested_version:
 *
 *   abi_version 1 -- the reference loader's version (it calls
 *     inferfabric_kernel_v1(1) and requires abi_version == 1). Contract names
 *     end in ".v1". Only the reference's dtypes (I8, BF16, F32) and accesses
 *     (read, write) appear: every integer port (block tables, lengths,
 *     cu_seqlens, index lists: int32; slot mappings: int64) is an I8 tensor
 *     holding the little-endian integers, its last extent 4x (int32) or 8x
 *     (int64) the integer count. Caches that a write operator updates in place
 *     are outputs with write access: the operator writes the rows the slot
 *     mapping names and leaves every other row as it was.
 *   abi_version 2 -- the same struct with dtype 4 = I32, 5 = I64 and access
 *     3 = read + write. Contract names end in ".v2".
 *
 * The gated Qwen-shape attention reads the caches it appends to, which version
 * 1 cannot express (outputs must not alias inputs); it exists as ".v2" only.
 * The contract string fixes the semantics, including the softmax scale
 * (1/sqrt(head_dim) for GQA, 1/sqrt(192) for MLA, 1/16 for the gated
 * attention) since the ABI carries no scalars. target is "gfx950". stream is
 * a hipStream_t passed as void*.
 *
 * prepare validates every descriptor and allocates only host state; enqueue
 * launches the kernels asynchronously on `stream`, allocates nothing, never
 * synchronizes and reads no device data on the host (graph-capture safe).
 */
#ifndef INFERFABRIC_KERNEL_V1_H
#define INFERFABRIC_KERNEL_V1_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define IF_KERNEL_DTYPE_I8 1
#define IF_KERNEL_DTYPE_BF16 2
#define IF_KERNEL_DTYPE_F32 3
#define IF_KERNEL_DTYPE_I32 4 /* abi_version 2 */
#define IF_KERNEL_DTYPE_I64 5 /* abi_version 2 */
#define IF_KERNEL_ACCESS_READ 1
#define IF_KERNEL_ACCESS_WRITE 2
#define IF_KERNEL_ACCESS_READ_WRITE 3 /* abi_version 2 */

typedef struct {
  uint32_t struct_bytes, dtype, rank, access;
  void *data;
  uint64_t allocation_bytes;
  int64_t shape[8], strides[8]; /* strides in elements, contiguous only */
} IFKernelTensorV1;

typedef struct {
  void *state;
  uint64_t workspace_bytes, workspace_alignment;
} IFKernelPreparedV1;

typedef struct {
  uint32_t struct_bytes, abi_version;
  const char *contract;
  const char *target;
  int32_t (*prepare)(const IFKernelTensorV1 *inputs, uint32_t input_count,
                     const IFKernelTensorV1 *outputs, uint32_t output_count,
                     IFKernelPreparedV1 *out);
  int32_t (*enqueue)(void *state, void *workspace, uint64_t bytes, void *stream);
  void (*release)(void *state);
} IFKernelV1;

typedef const IFKernelV1 *(*IFKernelEntryV1)(uint32_t requested_version);

/* Each libifk_<operator>.so exports the reference's entry symbol:
 *   const IFKernelV1 *inferfabric_kernel_v1(uint32_t requested_version);
 * Contracts (inputs ; outputs):
 *   libifk_kv_cache_write_bf16   "inferfabric.kv_cache_write.bf16.v2"
 *       k_rows, v_rows bf16 [rows, kv_heads, head_dim], slot_mapping I64|I32 [rows] ;
 *       k_cache, v_cache bf16 [blocks, block_size, kv_heads, head_dim] (access 3)
 *   libifk_kv_cache_write_c8     "inferfabric.kv_cache_write.c8.v2"
 *       k_rows, v_rows bf16, slot_mapping ;
 *       k_cache, v_cache I8 [blocks, block_size, kv_heads, head_dim],
 *       k_scale, v_scale F32 [blocks, block_size, kv_heads] (access 3)
 *   libifk_paged_decode_gqa_bf16 "inferfabric.paged_decode.gqa.bf16.v2"
 *       q bf16 [n, q_heads, head_dim], k_cache, v_cache bf16, block_tables I32 [n, entries],
 *       seq_lens I32 [n] ; out bf16 [n, q_heads, head_dim]
 *   libifk_paged_decode_gqa_c8   "inferfabric.paged_decode.gqa.c8.v2"
 *       q, k_cache I8, v_cache I8, k_scale F32, v_scale F32, block_tables, seq_lens ; out
 *   libifk_varlen_prefill_bf16   "inferfabric.varlen_prefill.bf16.v2"
 *       q bf16 [total_q, q_heads, head_dim], k_cache, v_cache bf16, block_tables I32,
 *       cu_seqlens_q I32 [n+1], kv_lens I32 [n] ; out bf16 [total_q, q_heads, head_dim]
 *   libifk_mla_decode_bf16       "inferfabric.mla_decode.bf16.v2"
 *       q bf16 [n, heads, 576], cache bf16 [blocks, block_size, 576], block_tables, seq_lens ;
 *       out bf16 [n, heads, 512]
 *   libifk_mla_decode_c8         "inferfabric.mla_decode.c8.v2"
 *       q, cache I8 [blocks, block_size, 656], block_tables, seq_lens ; out
 *   libifk_mla_cache_write_c8    "inferfabric.mla_cache_write.c8.v2"
 *       rows bf16 [rows, 576], slot_mapping ; cache I8 [blocks, block_size, 656] (access 3)
 *   libifk_mla_norm_rope_cache_bf16 "inferfabric.mla_norm_rope_cache.bf16.v2"
 *       x bf16 [rows <= 4096, 576], gamma bf16 [512], cos, sin bf16 [rows, 64], slot_mapping ;
 *       cache bf16 [blocks, block_size, 576] (access 3); eps 1e-5
 *   libifk_mla_norm_rope_cache_c8   "inferfabric.mla_norm_rope_cache.c8.v2"
 *       same inputs ; cache I8 [blocks, block_size, 656] (access 3)
 *   libifk_mla_window_attention_w512_bf16  "inferfabric.mla_window_attention.w512.bf16.v2"
 *   libifk_mla_window_attention_w2048_bf16 "inferfabric.mla_window_attention.w2048.bf16.v2"
 *       q bf16 [rows, heads, 576], cache bf16 [blocks, block_size, 576], block_tables I32
 *       [seqs, entries], cu_seqlens_q I32 [seqs+1], kv_lens I32 [seqs], sink_keys bf16
 *       [n <= 128, 576], sink_values bf16 [n, 512] ; out bf16 [rows, heads, 512]
 *       (window 512 or 2048 keys, the two windows of examples/openpangu/92b-tp8-ep8.inferfabric:97)
 *   libifk_mla_sparse_attention_c8 "inferfabric.mla_sparse_attention.c8.v2"
 *       q, cache I8 [blocks, block_size, 656], indices I32 [rows, topk], block_tables,
 *       cu_seqlens_q, kv_lens, sink_keys, sink_values ; out bf16 [rows, heads, 512]
 *   libifk_paged_attention_qwen_gated_bf16 "inferfabric.paged_attention.qwen_gated.bf16.v2"
 *       q bf16 [batch <= 64, 8, 256], k, v bf16 [batch, 512], gate bf16 [batch, 8, 256],
 *       append I64 [batch], table I64 [batch, context], mask F32 [batch, context] ;
 *       keys, values bf16 [slots, 512] (access 3), out bf16 [batch, 8, 256]
 *       (inferfabric_acl_paged_attention_prepare, native/src/inferfabric_acl.cpp:1343-1430)
 * Every contract above except the gated attention also answers version 1
 * under the same name with ".v1" (integer ports as I8 byte views).
 * Attention contracts use scale 1/sqrt(192) for MLA and 1/sqrt(head_dim) for GQA.
 * max_context is entries * block_size of the block-table descriptor.
 */

/* Lookup by contract name ("...v1" with version 1, "...v2" with version 2)
 * inside libifattn_hip.so. NULL for unknown contracts or unsupported versions. */
const IFKernelV1 *ifattn_kernel_v1_contract(const char *contract, uint32_t requested_version);
/* Lookup by operator index (the per-operator libraries forward here). */
const IFKernelV1 *ifattn_kernel_v1_operator(int32_t index, uint32_t requested_version);

#ifdef __cplusplus
}
#endif
#endif /* INFERFABRIC_KERNEL_V1_H */
