/*
 * triton_mla C ABI: MI355X (gfx950) kernels for weight-absorbed MLA decode
 * over a paged latent KV cache.
 *
 * Plain C types only: device pointers, element strides and sizes. No torch
 * or HIP types appear in the signatures; `stream` is a hipStream_t passed as
 * void* (NULL = the legacy default stream). All launches are asynchronous on
 * that stream; no entry point synchronises the host or allocates memory.
 * Every entry point returns a tmla_status (0 = success).
 *
 * Element codes (`dtype`): TMLA_BF16, TMLA_FP16. q, kv and out share it.
 *
 * Work partition. Stage 1 runs a grid of workers; each worker owns a
 * contiguous range of 64-token KV tiles and, for every sequence that range
 * touches, writes either the final output (when it covers the whole sequence)
 * or a partial (in the input dtype) plus a base-2 log-sum-exp into a workspace slot.
 * Stage 2 merges the partials of every sequence that was split.
 *   num_splits > 0 : every sequence is cut into num_splits tile-aligned
 *                    pieces, one worker each (the reference's uniform
 *                    split-KV scheme; grid = batch * num_splits workers).
 *   num_splits == 0: the total tile count is spread evenly over
 *                    num_workers workers regardless of sequence boundaries
 *                    (balanced for ragged lengths; computed on the device
 *                    from cache_seqlens, so no host synchronisation).
 */
#ifndef TRITON_MLA_H
#define TRITON_MLA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TMLA_OK = 0,
    TMLA_ERR_INVALID_ARGUMENT = 1,
    TMLA_ERR_UNSUPPORTED = 2,
    TMLA_ERR_WORKSPACE_TOO_SMALL = 3,
    TMLA_ERR_HIP = 4
} tmla_status;

enum { TMLA_BF16 = 0, TMLA_FP16 = 1 };

/* Human-readable text for a status returned by the last failing call on this
 * thread (includes the HIP error string for TMLA_ERR_HIP). */
const char* tmla_last_error(void);

/* ABI version: major * 10000 + minor * 100 + patch. */
int tmla_version(void);

/*
 * Bytes of device workspace tmla_mla_decode / _partial / _combine need:
 * partial outputs (input dtype [slots, H, head_dim_v]) and base-2 log-sum-exps
 * (float32 [slots, H]); slots = batch * num_splits (uniform) or
 * num_workers + batch (balanced).
 */
size_t tmla_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim_v,
                            int32_t num_splits, int32_t num_workers);

/*
 * Stage 1: split-KV partial attention.
 * Replaces the reference's `_mla_decode_stage1` launch
 * (src/triton_mla/kernel.py:276-302; kernel body kernel.py:43-138).
 *
 *   q          [batch, num_heads, head_dim_v + rope_dim], element strides
 *              (q_stride_b, q_stride_h, 1).
 *   kv         paged: [num_blocks, page_size, head_dim_v + rope_dim] with
 *              strides (kv_stride_0, kv_stride_1, 1); dense (block_table ==
 *              NULL): [batch, num_blocks (= capacity), D] and page_size must
 *              be 1.
 *   block_table[batch, bt_cols] int32 page ids, row stride bt_stride_b.
 *   seqlens    [batch] int32 valid tokens per sequence.
 *   softmax_scale  multiplies q.k before the softmax (natural-exp domain).
 *   out        [batch, num_heads, head_dim_v] dtype, strides
 *              (out_stride_b, out_stride_h, 1); written for sequences that one
 *              worker completes. lse [batch, num_heads] float32 natural log.
 * Page ids are clamped to [0, num_blocks) and page slots to [0, bt_cols) so a
 * malformed table cannot address memory outside the cache.
 */
int tmla_mla_decode_partial(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            const void* kv, int64_t kv_stride_0, int64_t kv_stride_1,
                            int64_t num_blocks, int32_t page_size,
                            const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                            const int32_t* seqlens, int32_t batch, int32_t num_heads,
                            int32_t head_dim_v, int32_t rope_dim, int32_t dtype,
                            float softmax_scale, int32_t num_splits, int32_t num_workers,
                            void* out, int64_t out_stride_b, int64_t out_stride_h, float* lse,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Stage 2: log-sum-exp merge of the partials of every split sequence, and
 * out = 0 / lse = -inf for empty sequences.
 * Replaces the reference's `_mla_decode_stage2` launch
 * (src/triton_mla/kernel.py:303-320; kernel body kernel.py:141-181).
 * Arguments mean what they mean for tmla_mla_decode_partial, which must have
 * run before on the same stream with the same partition arguments.
 */
int tmla_mla_decode_combine(const int32_t* seqlens, int32_t batch, int32_t num_heads,
                            int32_t head_dim_v, int32_t dtype, int32_t num_splits,
                            int32_t num_workers, void* out, int64_t out_stride_b,
                            int64_t out_stride_h, float* lse, const void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Both stages back to back: the whole of the reference's `mla_decode`
 * device work (src/triton_mla/kernel.py:264-320) for one call.
 */
int tmla_mla_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                    int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                    int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                    int32_t bt_cols, const int32_t* seqlens, int32_t batch, int32_t num_heads,
                    int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                    int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                    int64_t out_stride_h, float* lse, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Number of compute units of `device` (0 on error); the default worker count. */
int32_t tmla_device_cu_count(int32_t device);

#ifdef __cplusplus
}
#endif

#endif /* TRITON_MLA_H */
