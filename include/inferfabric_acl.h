/* inferfabric_acl — the reference's session ABI, served on one MI355X by
 * libinferfabric_acl.so (ironpangu_amd/session/inferfabric_acl.cpp).
 *
 * Every declaration below has the name, argument list and return type of
 * native/include/inferfabric_acl.h (the reference header, lines cited per
 * group), so a caller that binds that header by name — the Rust loader
 * crates/inferfabric-native/src/ffi.rs:36-70, the probes under
 * crates/inferfabric-cli/src/npu_probe/ — binds this library unchanged.
 *
 * Conventions (the reference's, inferfabric_acl.h:7-10 and
 * native/src/inferfabric_acl.cpp:46-58): 0 = OK, -1 = error with a message in
 * the calling thread's inferfabric_acl_last_error(); buffers, operations and
 * graphs are u64 ids (from 1) owned by the session; a session is used only on
 * the thread that opened it; every operation runs on the session's one HIP
 * stream and execute / replay / read / write return after it completes.
 *
 * Served here: the session itself (open, close, memory and allocation stats,
 * budget, allocate, buffer views, read, write, region copy, captured copies,
 * replay, device count), composite sequences, execute / capture of operations,
 * and the two operations of the Qwen attention path: attention_qk_prepare
 * (q/k norm, partial RoPE, gate) and paged_attention_prepare (row append +
 * paged GQA attention + gate). Every other prepare entry exists so that
 * by-name loaders resolve it, and fails with "not in this library". */
#ifndef INFERFABRIC_ACL_H
#define INFERFABRIC_ACL_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct inferfabric_acl_session inferfabric_acl_session;

/* Session (inferfabric_acl.h:11-14, :134). ABI version 2, as ffi.rs:44 checks. */
uint32_t inferfabric_acl_abi_version(void);
const char *inferfabric_acl_last_error(void);
int32_t inferfabric_acl_open(int32_t device, inferfabric_acl_session **out);
int32_t inferfabric_acl_close(inferfabric_acl_session *);

/* Memory accounting (inferfabric_acl.h:15-33). HBM figures come from
 * hipMemGetInfo; workspaces are dedicated per operation. */
typedef struct inferfabric_acl_memory_stats {
  uint64_t total_bytes, free_bytes, observed_peak_bytes, buffer_bytes;
  uint64_t temporary_bytes, workspace_bytes, graphs, budget_bytes;
} inferfabric_acl_memory_stats;
int32_t inferfabric_acl_memory_snapshot(inferfabric_acl_session *, inferfabric_acl_memory_stats *);
typedef struct inferfabric_acl_allocation_stats {
  uint64_t scratch_pool_bytes, layer_pool_bytes, snapshot_pool_bytes;
  uint64_t owned_temporary_bytes, logical_scratch_bytes, logical_workspace_bytes;
  uint64_t workspace_blocks, owned_buffers, buffer_views;
  uint64_t dedicated_activations, dedicated_workspaces;
} inferfabric_acl_allocation_stats;
int32_t inferfabric_acl_allocation_snapshot(inferfabric_acl_session *,
                                            inferfabric_acl_allocation_stats *);
int32_t inferfabric_acl_set_memory_budget(inferfabric_acl_session *, uint64_t bytes,
                                          uint64_t reserve);

/* Buffers (inferfabric_acl.h:34-45). Views: offset a multiple of 512. */
int32_t inferfabric_acl_allocate(inferfabric_acl_session *, uint64_t bytes, uint64_t *handle);
int32_t inferfabric_acl_buffer_view(inferfabric_acl_session *, uint64_t parent, uint64_t offset,
                                    uint64_t bytes, uint64_t *handle);
int32_t inferfabric_acl_write(inferfabric_acl_session *, uint64_t handle, uint64_t offset,
                              const void *, uint64_t bytes);
int32_t inferfabric_acl_read(inferfabric_acl_session *, uint64_t handle, uint64_t offset, void *,
                             uint64_t bytes);
int32_t inferfabric_acl_copy_region(inferfabric_acl_session *, uint64_t, uint64_t, uint64_t,
                                    uint64_t, uint64_t);

/* Graphs (inferfabric_acl.h:46-50, :64-66): capture records one run of the
 * operation into a HIP graph after an eager warm-up run; replay launches it
 * and waits. */
int32_t inferfabric_acl_capture_copy(inferfabric_acl_session *, uint64_t source,
                                     uint64_t destination, uint64_t bytes, uint64_t *graph);
int32_t inferfabric_acl_replay(inferfabric_acl_session *, uint64_t graph);
int32_t inferfabric_acl_operation_execute(inferfabric_acl_session *, uint64_t operation);
int32_t inferfabric_acl_operation_capture(inferfabric_acl_session *, uint64_t operation,
                                          uint64_t *graph);
int32_t inferfabric_acl_sequence_prepare(inferfabric_acl_session *, const uint64_t *,
                                         uint64_t count, uint64_t *operation);

/* The Qwen attention path (inferfabric_acl.h:94-113). */
int32_t inferfabric_acl_attention_qk_prepare(inferfabric_acl_session *, uint64_t packed_q,
                                             uint64_t k, uint64_t qgamma, uint64_t kgamma,
                                             uint64_t positions, uint64_t qout, uint64_t kout,
                                             uint64_t gate, int64_t batch, uint64_t *operation);
int32_t inferfabric_acl_paged_attention_prepare(inferfabric_acl_session *, uint64_t q, uint64_t k,
                                                uint64_t v, uint64_t gate, uint64_t keys,
                                                uint64_t values, uint64_t append, uint64_t table,
                                                uint64_t mask, uint64_t out, int64_t batch,
                                                int64_t slots, int64_t context,
                                                uint64_t *operation);

/* Resolvable but not served: each fails with "not in this library"
 * (inferfabric_acl.h:51-63, :67-93, :114-133, :135-153). */
int32_t inferfabric_acl_linear_prepare(inferfabric_acl_session *, uint64_t x, uint64_t weight,
                                       uint64_t y, int64_t m, int64_t n, int64_t k,
                                       uint64_t *operation);
int32_t inferfabric_acl_linear_execute(inferfabric_acl_session *, uint64_t operation);
int32_t inferfabric_acl_linear_capture(inferfabric_acl_session *, uint64_t operation,
                                       uint64_t *graph);
int32_t inferfabric_acl_rms_prepare(inferfabric_acl_session *, uint64_t x, uint64_t gamma,
                                    uint64_t y, int64_t m, int64_t k, uint64_t *operation);
int32_t inferfabric_acl_delta_prepare(inferfabric_acl_session *, uint64_t q, uint64_t k,
                                      uint64_t v, uint64_t g, uint64_t beta, uint64_t state,
                                      uint64_t out, int64_t bh, int64_t dk, int64_t dv,
                                      uint64_t *operation);
int32_t inferfabric_acl_conv_prepare(inferfabric_acl_session *, uint64_t x, uint64_t weight,
                                     uint64_t history, uint64_t out, int64_t batch,
                                     int64_t channels, uint64_t *operation);
int32_t inferfabric_acl_pointwise_prepare(inferfabric_acl_session *, uint64_t a, uint64_t b,
                                          uint64_t out, int64_t count, int32_t kind,
                                          uint64_t *operation);
int32_t inferfabric_acl_delta_transforms_prepare(inferfabric_acl_session *, uint64_t conv,
                                                 uint64_t a, uint64_t b, uint64_t a_log,
                                                 uint64_t dt_bias, uint64_t q, uint64_t k,
                                                 uint64_t v, uint64_t g, uint64_t beta,
                                                 int64_t batch, uint64_t *operation);
int32_t inferfabric_acl_gated_rms_prepare(inferfabric_acl_session *, uint64_t x, uint64_t z,
                                          uint64_t weight, uint64_t out, int64_t bh,
                                          int64_t width, uint64_t *operation);
int32_t inferfabric_acl_embedding_prepare(inferfabric_acl_session *, uint64_t weight,
                                          uint64_t ids, uint64_t out, int64_t vocab,
                                          int64_t width, uint64_t *operation);
int32_t inferfabric_acl_model_layer_prepare(inferfabric_acl_session *, int32_t kind,
                                            const uint64_t *weights, uint64_t count,
                                            uint64_t input, uint64_t output, uint64_t positions,
                                            uint64_t append, uint64_t table, uint64_t mask,
                                            int64_t slots, int64_t context, uint64_t *state_a,
                                            uint64_t *state_b, uint64_t *operation);
int32_t inferfabric_acl_embedding_batch_prepare(inferfabric_acl_session *, uint64_t, uint64_t,
                                                int64_t, int64_t, int64_t, uint64_t *);
int32_t inferfabric_acl_model_layer_batch_prepare(inferfabric_acl_session *, int32_t,
                                                  const uint64_t *, uint64_t, uint64_t, uint64_t,
                                                  uint64_t, uint64_t, uint64_t, uint64_t, int64_t,
                                                  int64_t, int64_t, uint64_t, uint64_t *,
                                                  uint64_t *, uint64_t *);
int32_t inferfabric_acl_sampler_prepare(inferfabric_acl_session *, uint64_t logits,
                                        uint64_t params, uint64_t counts, uint64_t seen,
                                        uint64_t mask, uint64_t controls, uint64_t random,
                                        uint64_t output, uint64_t probabilities, int64_t vocab,
                                        int64_t random_count, int32_t greedy,
                                        uint64_t *operation);
int32_t inferfabric_acl_random_fill(inferfabric_acl_session *, uint64_t buffer, int64_t count,
                                    uint64_t seed);

/* Tensor parallelism (inferfabric_acl.h:129-133): one GPU here. device_count
 * reports HIP devices; tp_root_size is 0 and tp_root / tp_init fail. */
int32_t inferfabric_acl_device_count(uint32_t *);
uint64_t inferfabric_acl_tp_root_size(void);
int32_t inferfabric_acl_tp_root(void *, uint64_t);
int32_t inferfabric_acl_tp_init(inferfabric_acl_session *, uint32_t, uint32_t, const void *,
                                uint64_t);

#ifdef __cplusplus
}
#endif
#endif
