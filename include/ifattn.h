/* ifattn — MI355X (gfx950) continuous-batching attention path, C ABI.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed
 * as void*. Nothing here allocates device memory, synchronizes, or changes the
 * caller's stream; calls are asynchronous on `stream` and safe to record into a
 * HIP graph (all control data is read on the device). Functions return an
 * int32 status (0 = OK, negative = error) and leave a thread-local message in
 * ifattn_last_error(), the boundary convention of the reference
 * (native/src/inferfabric_acl.cpp:46-58, native/src/program_engine.cpp:274-278).
 *
 * Layouts (row-major, contiguous):
 *   GQA caches     K, V : [num_blocks * block_size, kv_heads, head_dim]  (bf16 or int8)
 *                  this is the reference's flattened slot-row cache [slots, kv_heads*head_dim]
 *                  (native/src/inferfabric_acl.cpp:1359-1362); slot = block*block_size + offset.
 *   C8 scales           : [num_blocks * block_size, kv_heads] fp32
 *   MLA cache (bf16)    : [num_blocks * block_size, 576]       (token_executor.h:749)
 *   MLA cache (C8)      : [num_blocks * block_size, 656] bytes (docs/packed-mla-cache.md:27-43)
 *   block tables        : [num_seqs, table_stride] int32        (page_binding.h:132-160)
 *   q / out (decode)    : [num_seqs, q_heads, head_dim] bf16
 *   q / out (prefill)   : [total_q_rows, q_heads, head_dim] bf16, packed by cu_seqlens_q
 */
#ifndef IFATTN_H
#define IFATTN_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define IFATTN_OK 0
#define IFATTN_EINVAL (-1)  /* argument / contract violation, nothing launched */
#define IFATTN_ELAUNCH (-2) /* HIP launch error */
#define IFATTN_EWORKSPACE (-3)

/* Dtype codes: 1..3 are the reference's IFKernelTensorV1 codes
 * (native/include/inferfabric_kernel_v1.h:7); 4 and 5 are additive. */
#define IFATTN_DTYPE_I8 1
#define IFATTN_DTYPE_BF16 2
#define IFATTN_DTYPE_F32 3
#define IFATTN_DTYPE_I32 4
#define IFATTN_DTYPE_I64 5

/* Version of this direct ifattn_* C ABI (functions, argument lists, status
 * codes). It is raised only by an incompatible change; added entry points keep
 * it. It is unrelated to the IFKernelV1 plug-in table's abi_version (1 or 2,
 * chosen per call by requested_version; see inferfabric_kernel_v1.h). */
#define IFATTN_ABI_VERSION 1

int32_t ifattn_abi_version(void);
const char *ifattn_last_error(void);

/* ---- slot-mapped cache writes ------------------------------------------------ */

/* cache[slot_mapping[r]] = rows[r] for K and (optionally) V. Rows are row_bytes
 * each (a multiple of 16: 1024 B for 2 kv heads x 128 bf16, 1152 B for an MLA
 * latent row). slot_mapping holds int32 or int64 physical slots; negative or
 * >= num_slots entries are skipped. Bit copy.
 * Replaces aclnnScatterNdUpdate x2 in inferfabric_acl_paged_attention_prepare
 * (native/src/inferfabric_acl.cpp:1364-1376) and aclnnInplaceIndexCopy of the
 * MLA cache (native/src/token_executor.h:733-757). */
int32_t ifattn_kv_cache_write(const void *k_rows, const void *v_rows, void *k_cache,
                              void *v_cache, const void *slot_mapping, int32_t slot_dtype,
                              int64_t rows, int64_t row_bytes, int64_t num_slots, void *stream);

/* Quantizing write, int8 with one fp32 scale per (token, kv head):
 * scale = max|x|/127 (1.0 for an all-zero row), q = round-half-even(x/scale)
 * clamped to +-127. Rows bf16 [rows, kv_heads, head_dim].
 * Replaces the row-quantized cache write (native/kernels/cache_quantization.cpp:12-38,
 * token_executor.h:795-810) at the per_token_head granularity of
 * crates/inferfabric-authoring/src/execution.rs:65-66. */
int32_t ifattn_kv_cache_write_c8(const void *k_rows, const void *v_rows, void *k_cache,
                                 void *v_cache, void *k_scale, void *v_scale,
                                 const void *slot_mapping, int32_t slot_dtype, int64_t rows,
                                 int32_t kv_heads, int32_t head_dim, int64_t num_slots,
                                 void *stream);

/* Packed C8 MLA latent write: 576 bf16 (512 latent + 64 rope) per row ->
 * 656-byte row {int8[512], bf16 rope[64], f32 scale[4]}, scale per 128-value
 * tile = max/127 (0 for a zero tile), nearest-even codes. Replaces the cache
 * storage half of aclnnAiInfraKvRmsNormRopeCache pertile128
 * (native/src/resident_cache_writer.h:5-20; docs/packed-mla-cache.md:27-43). */
int32_t ifattn_mla_cache_write_c8(const void *rows, void *cache, const void *slot_mapping,
                                  int32_t slot_dtype, int64_t rows_count, int64_t num_slots,
                                  void *stream);

/* Fused MLA cache writer: for each of `rows` (1..4096) rows x [rows, 576] bf16
 * (512 latent + 64 rope): y = x[0:512] * rsqrt(mean(x[0:512]^2) + eps) * gamma,
 * rope[d] = bf16(x[512+d]*cos[r,d] + (d < 32 ? -x[544+d] : x[480+d])*sin[r,d]),
 * stored at cache row slot_mapping[r] as either a bf16 576-wide row
 * {bf16(y), rope} (packed = 0) or the packed C8 656-byte row
 * {int8 y/scale[t], rope, f32 scale[4]} (packed = 1; scale = tile max/127, 0
 * for a zero tile, nearest-even codes). gamma [512] bf16, cos/sin [rows, 64]
 * bf16. Slots < 0 or >= num_slots are skipped. fp32 arithmetic in a fixed
 * order (bit-identical to the CPU oracle).
 * Replaces aclnnAiInfraKvRmsNormRopeCache (mode "PA", rotary "half", quant
 * "pertile128"/"none") behind resident::normalized_cache_append
 * (native/src/resident_cache_writer.h:5-20); acceptance rules
 * native/probes/prefill_cache_writer_probe.cpp:38-61. */
int32_t ifattn_mla_norm_rope_cache_write(const void *x, const void *gamma, const void *cos,
                                         const void *sin, const void *slot_mapping,
                                         int32_t slot_dtype, int64_t rows, float eps, void *cache,
                                         int32_t packed, int64_t num_slots, void *stream);

/* ---- paged decode (one query row per sequence) --------------------------------- */

/* Workspace bytes for the split-K partials of the decode kernels. */
uint64_t ifattn_paged_decode_workspace_size(int32_t num_seqs, int32_t q_heads, int32_t head_dim,
                                            int32_t max_context);

/* Ragged paged GQA decode, bf16 caches. For each sequence b and q head h
 * (kv head h / (q_heads/kv_heads)): softmax(scale * q.K[0..len_b)) . V with fp32
 * accumulation; len_b = seq_lens[b] (>= 1, clamped to max_context).
 * head_dim 64/128/256, q_heads/kv_heads <= 16, block_size a multiple of 32,
 * table_stride*block_size >= max_context.
 * Replaces the gather + matmul + fp32 softmax + matmul sequence of
 * inferfabric_acl_paged_attention_prepare (native/src/inferfabric_acl.cpp:1377-1428)
 * without the gather copy; CPU oracle crates/inferfabric-cli/src/npu_probe/attention.rs:221-253. */
int32_t ifattn_paged_decode_bf16(const void *q, const void *k_cache, const void *v_cache,
                                 const int32_t *block_tables, int32_t table_stride,
                                 const int32_t *seq_lens, void *out, int32_t num_seqs,
                                 int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                 int32_t block_size, int64_t num_blocks, int32_t max_context,
                                 float scale, void *workspace, uint64_t workspace_bytes,
                                 void *stream);

/* One decode step as the reference's paged attention operator runs it
 * (native/src/inferfabric_acl.cpp:1343-1430): the slot-mapped write of `rows`
 * new K/V rows (as ifattn_kv_cache_write, row = kv_heads*head_dim bf16) followed
 * by ifattn_paged_decode_bf16 over the updated caches. The write is folded into
 * the decode prologue launch, so the step is two kernel launches. */
int32_t ifattn_paged_decode_step_bf16(const void *q, const void *k_rows, const void *v_rows,
                                      void *k_cache, void *v_cache, const void *slot_mapping,
                                      int32_t slot_dtype, int64_t rows,
                                      const int32_t *block_tables, int32_t table_stride,
                                      const int32_t *seq_lens, void *out, int32_t num_seqs,
                                      int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                      int32_t block_size, int64_t num_blocks, int32_t max_context,
                                      float scale, void *workspace, uint64_t workspace_bytes,
                                      void *stream);

/* The Qwen-shape paged attention of the reference session ABI
 * (inferfabric_acl_paged_attention_prepare, native/include/inferfabric_acl.h:103-113;
 * body native/src/inferfabric_acl.cpp:1343-1430), with device pointers in place
 * of the session's buffer ids and the same argument order and meaning:
 *   q [batch, 8, 256] bf16 (kv head major: head h reads kv head h / 4);
 *   k, v [batch, 512] bf16 rows appended at keys/values[append[b]] (int64);
 *   keys, values [slots, 512] bf16 caches (2 kv heads x 256);
 *   table [batch, context] int64: the physical row of every context position;
 *   mask [batch, context] fp32, added to the scaled scores (-inf drops the
 *   position, and such positions are never read from the caches);
 *   gate [batch, 8, 256] bf16, multiplied into the attention output;
 *   out [batch, 8, 256] bf16.
 * Scale 1/16 (inferfabric_acl.cpp:1400). Limits as the reference: batch 1..64,
 * slots 1..2^20, context 1..262144. A request whose positions are all masked
 * gets a zero output. Workspace: ifattn_gated_paged_attention_workspace_size. */
uint64_t ifattn_gated_paged_attention_workspace_size(int64_t batch, int64_t context);
int32_t ifattn_gated_paged_attention_bf16(const void *q, const void *k, const void *v,
                                          const void *gate, void *keys, void *values,
                                          const int64_t *append, const int64_t *table,
                                          const float *mask, void *out, int64_t batch,
                                          int64_t slots, int64_t context, void *workspace,
                                          uint64_t workspace_bytes, void *stream);

/* The producer of the Qwen attention's q, k and gate: per-head zero-centred RMS
 * norm (eps 1e-6, fp32 gamma = 1 + checkpoint weight), partial RoPE on the first
 * 64 of 256 channels (theta 1e7, cos/sin rounded to bf16) and the sigmoid gate,
 * in one launch. Replaces inferfabric_acl_attention_qk_prepare's ACLNN steps
 * (native/src/inferfabric_acl.cpp:1236-1341; CPU statement
 * crates/inferfabric-cli/src/npu_probe/attention.rs:35-64), same operands:
 *   packed_q [batch, 8, 512] bf16 (256 query then 256 gate channels per head);
 *   k [batch, 2, 256] bf16; q_gamma, k_gamma [256] fp32; positions [batch] int64;
 *   q_out [batch, 8, 256], k_out [batch, 2, 256], gate [batch, 8, 256] bf16.
 * batch 1..64 as the reference. */
int32_t ifattn_qk_norm_rope_gate_bf16(const void *packed_q, const void *k, const float *q_gamma,
                                      const float *k_gamma, const int64_t *positions, void *q_out,
                                      void *k_out, void *gate, int64_t batch, void *stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ifattn_paged_decode_step_bf16 without a workspace. The
 * call's scratch (split-K plan and partials) lives in a static
 * device array of IFATTN_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends; calls needing more (ifattn_paged_decode_workspace_size above it) fail
 * with IFATTN_EINVAL. The entry point allocates nothing. All calls on one GPU
 * share that GPU's array: calls that overlap on one GPU (concurrent streams,
 * threads) race and must be serialized by the caller. */
#define IFATTN_NOALLOC_SCRATCH_BYTES (32ull << 20)
int32_t ifattn_paged_decode_step_bf16_noalloc(
    const void *q, const void *k_rows, const void *v_rows, void *k_cache, void *v_cache,
    const void *slot_mapping, int32_t slot_dtype, int64_t rows, const int32_t *block_tables,
    int32_t table_stride, const int32_t *seq_lens, void *out, int32_t num_seqs, int32_t q_heads,
    int32_t kv_heads, int32_t head_dim, int32_t block_size, int64_t num_blocks,
    int32_t max_context, float scale, void *stream);

/* Same over an int8 cache with fp32 scales per (token, kv head), dequantized in
 * registers (replaces cache_dequantize + bf16 attention, token_executor.h:812-822). */
int32_t ifattn_paged_decode_c8(const void *q, const void *k_cache, const void *v_cache,
                               const void *k_scale, const void *v_scale,
                               const int32_t *block_tables, int32_t table_stride,
                               const int32_t *seq_lens, void *out, int32_t num_seqs,
                               int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                               int32_t block_size, int64_t num_blocks, int32_t max_context,
                               float scale, void *workspace, uint64_t workspace_bytes,
                               void *stream);

/* ---- packed varlen chunked prefill -------------------------------------------- */

uint64_t ifattn_varlen_prefill_workspace_size(int32_t num_seqs, int32_t total_q, int32_t q_heads,
                                              int32_t head_dim, int32_t max_kv_len);

/* Packed TND batch: sequence s owns query rows [cu_seqlens_q[s], cu_seqlens_q[s+1])
 * and kv_lens[s] cached keys (prior context + this chunk, already written).
 * Row t of a chunk of `count` rows sees keys [0, kv_len - count + t]
 * (causal rule of native/src/openpangu_attention_metadata.h:20-22; writes precede
 * queries, native/include/sliding_window_layout.h:7). Sequences with one row are
 * decode rows. Replaces the TND attention call of token_executor.h:863-906 /
 * resident_window_attention.h:17-31 (without window/sinks). */
int32_t ifattn_varlen_prefill_bf16(const void *q, const void *k_cache, const void *v_cache,
                                   const int32_t *block_tables, int32_t table_stride,
                                   const int32_t *cu_seqlens_q, const int32_t *kv_lens, void *out,
                                   int32_t num_seqs, int32_t total_q, int32_t max_q_len,
                                   int32_t max_kv_len, int32_t q_heads, int32_t kv_heads,
                                   int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                   float scale, void *workspace, uint64_t workspace_bytes,
                                   void *stream);

/* ---- packed MLA latent decode -------------------------------------------------- */

uint64_t ifattn_mla_decode_workspace_size(int32_t num_seqs, int32_t heads, int32_t max_context,
                                          int32_t block_size);

/* q [num_seqs, heads, 576] bf16 (512 absorbed latent + 64 rope); cache rows of
 * 576 bf16; s_j = scale * q.row_j, o = softmax(s) . row_j[0:512];
 * out [num_seqs, heads, 512] bf16. heads <= 16 per call; block_size a power of
 * two >= 16 (bf16 rows) or >= 32 (C8 rows).
 * Replaces the BF16 latent attention (token_executor.h:863-906); CPU oracle
 * native/probes/sliding_window_probe.cpp:144-163 without sinks/window. */
int32_t ifattn_mla_decode_bf16(const void *q, const void *cache, const int32_t *block_tables,
                               int32_t table_stride, const int32_t *seq_lens, void *out,
                               int32_t num_seqs, int32_t heads, int32_t block_size,
                               int64_t num_blocks, int32_t max_context, float scale,
                               void *workspace, uint64_t workspace_bytes, void *stream);

/* Same over the packed 656-byte C8 rows: latent = int8 * scale[d/128], rope bf16
 * (native/probes/packed_cache_probe.cpp:57); replaces
 * aclnnAiInfraKvQuantSparseFlashAttention on dense causal candidates
 * (token_executor.h:841-852) without learned sinks. */
int32_t ifattn_mla_decode_c8(const void *q, const void *cache, const int32_t *block_tables,
                             int32_t table_stride, const int32_t *seq_lens, void *out,
                             int32_t num_seqs, int32_t heads, int32_t block_size,
                             int64_t num_blocks, int32_t max_context, float scale,
                             void *workspace, uint64_t workspace_bytes, void *stream);

/* ---- resident slot reuse: page reset and state copy --------------------------- */

/* Zero the {offset, bytes} spans (uint64 pairs in DEVICE memory, as produced by
 * ifattn_page_spans) of a device state field of field_bytes bytes: the reset of
 * a resident's owned pages before reuse (native/src/page_binding.h:19-35).
 * Spans outside the field are skipped. */
int32_t ifattn_page_reset(void *field, uint64_t field_bytes, const uint64_t *spans,
                          uint64_t count, void *stream);
/* Copy the {source, destination, bytes} ranges (uint64 triples in DEVICE
 * memory, as produced by ifattn_pages_copy_plan) inside one device state field:
 * a resident's completed pages to another slot (page_binding.h:161-187).
 * Ranges must not overlap one another or themselves (the plan guarantees it);
 * ranges outside the field are skipped. */
int32_t ifattn_state_copy(void *field, uint64_t field_bytes, const uint64_t *ranges,
                          uint64_t count, void *stream);
/* Checked forms: the whole plan is validated on the device first, with the
 * reference's rule for every span (native/src/prepared_execution.h:346-354: not
 * empty, inside the field, and for copies source and destination apart). An
 * invalid plan moves no byte. *status (device int32) receives 0, or 1 + the
 * index of the first invalid span; read it after the stream completes. */
int32_t ifattn_page_reset_checked(void *field, uint64_t field_bytes, const uint64_t *spans,
                                  uint64_t count, int32_t *status, void *stream);
int32_t ifattn_state_copy_checked(void *field, uint64_t field_bytes, const uint64_t *ranges,
                                  uint64_t count, int32_t *status, void *stream);

/* The fused MLA decode step: the cache writer of ifattn_mla_norm_rope_cache_write
 * and the decode attention of ifattn_mla_decode_bf16 (packed = 0, bf16 rows) or
 * ifattn_mla_decode_c8 (packed = 1, 656-byte rows) in one launch. For each
 * sequence s the step's latent row x_new[s] ([num_seqs, 576] bf16: 512 latent +
 * 64 rope, with cos/sin [num_seqs, 64] bf16 and gamma [512] bf16) is normalized,
 * roped and stored at the sequence's last position seq_lens[s] - 1 (the slot
 * block_tables[s][(len-1)/block_size] * block_size + (len-1) % block_size;
 * sequences with seq_lens[s] = 0 write nothing), then attended over with the
 * other cached keys. Rows and outputs are bit-identical to the writer followed
 * by the decode entry point (the same code writes the row); the writer's
 * separate launch disappears. Replaces resident::normalized_cache_append
 * followed by attend_packed / attend (native/src/resident_cache_writer.h:5-20,
 * token_executor.h:841-906) for a decode step. The block holding a sequence's
 * last position must belong to that sequence alone in this call (as a decode
 * step's tail block does): only the workgroup that reads a sequence's last tile
 * waits for its row, so another sequence reading the same block could see the
 * row before or after the write. Workspace as ifattn_mla_decode_workspace_size. */
int32_t ifattn_mla_decode_step(const void *q, const void *x_new, const void *gamma,
                               const void *cos, const void *sin, float eps, void *cache,
                               int32_t packed, const int32_t *block_tables, int32_t table_stride,
                               const int32_t *seq_lens, void *out, int32_t num_seqs, int32_t heads,
                               int32_t block_size, int64_t num_blocks, int32_t max_context,
                               float scale, void *workspace, uint64_t workspace_bytes,
                               void *stream);

/* ---- packed-MLA attention over query rows (windows, sparse lists, sinks) ----- */

/* Rows: sequence s owns query rows [cu_seqlens_q[s], cu_seqlens_q[s+1]) (NULL:
 * one row per sequence, num_rows = num_seqs) and kv_lens[s] cached keys
 * (writes precede queries); row t of a sequence with `count` rows sees
 * causal = kv_len - count + t + 1 keys (openpangu_attention_metadata.h:20-22).
 * Learned sink rows (keys [n_sinks, 576], values [n_sinks, 512] bf16,
 * n_sinks <= 128) join every row's softmax. q [num_rows, heads, 576] bf16,
 * out [num_rows, heads, 512] bf16, heads <= 16, scale multiplies q.k. */
uint64_t ifattn_mla_attention_workspace_size(int32_t num_rows, int32_t heads, int32_t max_context,
                                             int32_t window, int32_t topk, int32_t n_sinks,
                                             int32_t block_size);

/* BF16 latent rows (576 wide) over the window of each row: positions
 * [max(0, causal - window), causal) (window 0 = all) read through the block
 * table, which may be a ring of physical pages (sliding_window_layout.h:9-33:
 * only the window must be resident). Replaces aclnnAiInfraFusedInferAttentionSink
 * (TND, pre_tokens = window - 1, next_tokens = 0, learned sinks) of
 * token_executor.h:863-906 / resident_window_attention.h:17-31; CPU oracle
 * native/probes/sliding_window_probe.cpp:144-163. */
int32_t ifattn_mla_window_attention_bf16(const void *q, const void *cache,
                                         const int32_t *block_tables, int32_t table_stride,
                                         const int32_t *cu_seqlens_q, const int32_t *kv_lens,
                                         int32_t num_seqs, int32_t num_rows, int32_t window,
                                         const void *sink_keys, const void *sink_values,
                                         int32_t n_sinks, void *out, int32_t heads,
                                         int32_t block_size, int64_t num_blocks,
                                         int32_t max_context, float scale, void *workspace,
                                         uint64_t workspace_bytes, void *stream);

/* The same window attention over row-quantized latent rows, as if_cache_quantize
 * writes them (native/kernels/cache_quantization.cpp:12-38): row i of the cache
 * is 576 int8 codes (bits 8, 576 bytes) or 576 int4 codes (bits 4, 288 bytes,
 * two's complement, element 2b in the low nibble of byte b), with one fp32 scale
 * row_scales[i]; value = code * scale. The codes are dequantized in registers,
 * so the cache is read once as stored. Replaces the reference's integer-cache
 * path, which dequantizes the whole cache to bf16 (if_cache_dequantize,
 * token_executor.h:806-822) before the window attention (:863-906). The cache
 * must be below 4 GiB; block_size a power of two >= 16. Workspace as
 * ifattn_mla_attention_workspace_size (topk 0). */
int32_t ifattn_mla_window_attention_rowq(const void *q, const void *cache, const float *row_scales,
                                         int32_t bits, const int32_t *block_tables,
                                         int32_t table_stride, const int32_t *cu_seqlens_q,
                                         const int32_t *kv_lens, int32_t num_seqs, int32_t num_rows,
                                         int32_t window, const void *sink_keys,
                                         const void *sink_values, int32_t n_sinks, void *out,
                                         int32_t heads, int32_t block_size, int64_t num_blocks,
                                         int32_t max_context, float scale, void *workspace,
                                         uint64_t workspace_bytes, void *stream);

/* Packed C8 rows (656 bytes) over each row's candidate list indices[row][0..topk):
 * logical positions of its sequence, the first min(causal, topk) distinct and
 * < causal, then -1 (openpangu_attention_metadata.h:10-37); -1 or out-of-table
 * entries are skipped. The cache must be below 4 GiB (32-bit row offsets).
 * Replaces aclnnAiInfraKvQuantSparseFlashAttention (quant modes 2, tile 128, rope
 * 64, learned sinks; token_executor.h:841-852, docs/packed-mla-cache.md:50-60);
 * CPU oracle native/probes/packed_cache_probe.cpp:47-66. */
int32_t ifattn_mla_sparse_attention_c8(const void *q, const void *cache, const int32_t *indices,
                                       int32_t topk, const int32_t *block_tables,
                                       int32_t table_stride, const int32_t *cu_seqlens_q,
                                       const int32_t *kv_lens, int32_t num_seqs, int32_t num_rows,
                                       const void *sink_keys, const void *sink_values,
                                       int32_t n_sinks, void *out, int32_t heads,
                                       int32_t block_size, int64_t num_blocks,
                                       int32_t max_context, float scale, void *workspace,
                                       uint64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* IFATTN_H */
