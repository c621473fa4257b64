/* Operator plug-in ABI for the attention-path kernels.
 *
 * Same POD layout and calling contract as the reference's
 * native/include/inferfabric_kernel_v1.h:8-34 (the loader is
 * native/src/compiled_kernel.cpp:39-128), so an existing CompiledKernel loader
 * can dlopen these libraries unchanged. Interface declarations have to match
 * field for field; the text here is this project's own.
 *
 * Additive extension, reported as abi_version 2 (the same struct):
 *   dtype  4 = I32, 5 = I64   (block tables, slot mappings, cu_seqlens)
 *   access 3 = read + write   (caches updated in place by the write operators)
 * Every operator here needs at least one of these, so
 * inferfabric_kernel_v1(1) returns NULL and inferfabric_kernel_v1(2) returns the
 * table. The contract string fixes the semantics, including the softmax scale
 * (1/sqrt(head_dim) for GQA, 1/sqrt(192) for MLA) since the ABI carries no
 * scalars. target is "gfx950". stream is a hipStream_t passed as void*.
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
 * Attention contracts use scale 1/sqrt(192) for MLA and 1/sqrt(head_dim) for GQA.
 * max_context is entries * block_size of the block-table descriptor.
 */

/* Lookup by contract name inside libifattn_hip.so (the per-operator libraries
 * forward to it). NULL for unknown contracts or unsupported versions. */
const IFKernelV1 *ifattn_kernel_v1_contract(const char *contract, uint32_t requested_version);

#ifdef __cplusplus
}
#endif
#endif /* INFERFABRIC_KERNEL_V1_H */
