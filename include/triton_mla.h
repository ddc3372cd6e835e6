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
 * Element codes (`dtype`): TMLA_BF16, TMLA_FP16 (every decode entry point),
 * TMLA_FP32 (tmla_mla_decode_generic only). q, kv and out share it.
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

enum { TMLA_BF16 = 0, TMLA_FP16 = 1, TMLA_FP32 = 2 };

/* Human-readable text for a status returned by the last failing call on this
 * thread (includes the HIP error string for TMLA_ERR_HIP). */
const char* tmla_last_error(void);

/* ABI version: major * 10000 + minor * 100 + patch. */
int tmla_version(void);

/*
 * Bytes of device workspace tmla_mla_decode / _partial / _combine / _fused
 * need: partial outputs (input dtype [slots, H, head_dim_v]) and their
 * base-2 log-sum-exps (float32 [slots, H]) from the start of the buffer, and
 * a block of fixed size (256 KiB) at the END of the buffer (its size rounded
 * down to 256 bytes) for the int32 counters of the single launch's merge;
 * slots = batch * num_splits (uniform) or num_workers + batch (balanced).
 * The two-kernel entry points need no initialisation. A workspace may be
 * reused by any later call whose tmla_workspace_bytes is no larger, of any
 * shape, one call at a time.
 */
size_t tmla_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim_v,
                            int32_t num_splits, int32_t num_workers);

/*
 * Bytes at the end of the workspace that must be zero before its first use
 * by tmla_mla_decode_fused (or tmla_mla_decode_causal with single_launch):
 * zero the last min(tmla_workspace_zero_bytes(...), workspace_bytes) bytes
 * once (the counter block and the rounding slack; the same for every call).
 * Every single launch leaves its counters at zero again, and the partials of
 * no call reach that suffix, so later calls of any shape whose
 * tmla_workspace_bytes fits the buffer need nothing. The counters are
 * (2 * batch + slots) int32 per workgroup along the heads of the launched
 * grid, whose workgroups take 32, 64 or 128 heads (fewer heads per workgroup
 * when the call would leave compute units idle); a call whose counters
 * would not fit the block (more than 65536) or whose workgroups would not
 * all fit the device at once runs as two kernels:
 * tmla_mla_decode_fused_is_single tells which. No counterpart in the
 * reference (its two launches need no counters).
 */
size_t tmla_workspace_zero_bytes(int32_t batch, int32_t num_heads, int32_t head_dim_v,
                                 int32_t num_splits, int32_t num_workers);

/*
 * The balanced partition (num_splits == 0) shares the T = sum cdiv(seqlen,
 * 64) tiles of a call among num_workers workers. With c = cdiv(T,
 * num_workers): if the sequences cut into pieces of at most c tiles give no
 * more than num_workers pieces, worker w takes piece w (the pieces of each
 * sequence in order). Otherwise the tiles are laid out in order on a line on
 * which every non-empty sequence starts with tmla_partition_segment_tiles()
 * extra positions (the cost of a worker's start-up and finalize on a further
 * sequence, in tiles), and worker w takes positions [w v, (w + 1) v),
 * v = cdiv(line length, num_workers). No counterpart in the reference (its
 * splits are uniform); for callers that predict the partition, e.g. its
 * split counts.
 */
int32_t tmla_partition_segment_tiles(void);

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
 *              worker completes. lse [batch, num_heads] float32 natural log,
 *              or NULL when the caller does not need it (then not written;
 *              the same holds for every entry point below that takes lse).
 * Page ids are clamped to [0, num_blocks) and page slots to [0, bt_cols) so a
 * malformed table cannot address memory outside the cache. seqlens[b] must
 * not exceed the table's capacity bt_cols * page_size (dense: num_blocks), as
 * in the reference; the launch is sized from that capacity, so larger lengths
 * give undefined results (still without out-of-bounds accesses).
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
 * Both stages back to back: the whole of the reference's `mla_decode` device
 * work (src/triton_mla/kernel.py:264-320) for one call.
 */
int tmla_mla_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                    int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                    int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                    int32_t bt_cols, const int32_t* seqlens, int32_t batch, int32_t num_heads,
                    int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                    int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                    int64_t out_stride_h, float* lse, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * The same call as ONE launch (no counterpart in the reference, which always
 * launches two kernels): when every workgroup of stage 1 fits on the device
 * at once (workers times head blocks at most the CU count: blocks of up to
 * 128 heads, of 16 heads for calls of at most 16 heads;
 * tmla_mla_decode_fused_is_single tells), the workers of a split
 * sequence merge its partials themselves, each a share of the heads, once
 * all of them have stored theirs (a bounded wait of spin_limit polls, about
 * 2^7 clocks apart; < 0 selects the default, 16384; 0 makes every worker
 * that does not complete the count hand its share over at once). A worker
 * that stops waiting hands its share to the one whose arrival completes the
 * count. Otherwise it runs both stages like tmla_mla_decode. Results equal
 * tmla_mla_decode's bit for bit. The workspace's counter suffix must be
 * zero before its first use (tmla_workspace_zero_bytes).
 */
int tmla_mla_decode_fused(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                          int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                          int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                          int32_t bt_cols, const int32_t* seqlens, int32_t batch, int32_t num_heads,
                          int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                          int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                          int64_t out_stride_h, float* lse, void* workspace, size_t workspace_bytes,
                          int32_t spin_limit, void* stream);

/*
 * tmla_mla_decode without a caller-owned workspace: no counterpart in the
 * reference (whose launches take buffers torch allocates per call,
 * kernel.py:268-271). For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The partials live in a 64 MiB device array built into the
 * library, one per device, held until the process ends; no call allocates or
 * frees anything. Calls whose tmla_workspace_bytes exceed 64 MiB return
 * TMLA_ERR_WORKSPACE_TOO_SMALL before touching the device. Every call on a
 * device shares that device's array: calls that overlap on one device (other
 * streams, other threads) race and must be serialised by the caller. The
 * stream must belong to the current device. Results equal tmla_mla_decode's
 * bit for bit.
 */
int tmla_mla_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                            int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                            int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                            int32_t bt_cols, const int32_t* seqlens, int32_t batch, int32_t num_heads,
                            int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                            int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                            int64_t out_stride_h, float* lse, void* stream);

/*
 * 1 when tmla_mla_decode_fused with these arguments runs as a single launch
 * on `device`, 0 when it runs both stages. capacity_tokens = bt_cols *
 * page_size for a paged cache, the dense capacity otherwise (the launch
 * trims its grid to the tiles that capacity allows).
 */
int32_t tmla_mla_decode_fused_is_single(int32_t batch, int32_t num_heads, int32_t head_dim_v,
                                        int32_t num_splits, int32_t num_workers,
                                        int64_t capacity_tokens, int32_t device);

/*
 * Multi-token (causal) decode, no counterpart in the reference (its
 * `mla_decode` takes one query token per sequence: kernel.py:238 asserts a
 * 3-D q, README.md:32 "single-token decode only"). For speculative decoding
 * and chunked prefill onto the cache: each sequence b has q_len query tokens,
 * the last q_len of its cache_seqlens[b] tokens, and query token t sees the
 * first cache_seqlens[b] - (q_len - 1 - t) tokens (none when that is <= 0:
 * out = 0, lse = -inf).
 *   q    [batch, q_len * num_heads, head_dim_v + rope_dim]: row t * num_heads
 *        + h of sequence b at q + b * q_stride_b + (t * num_heads + h) *
 *        q_stride_h (a [batch, q_len, num_heads, D] tensor whose token and
 *        head dims are packed).
 *   out  [batch, q_len * num_heads, head_dim_v] the same way; lse [batch,
 *        q_len * num_heads] float32 natural log.
 * The workspace is tmla_workspace_bytes(batch, q_len * num_heads, ...).
 * single_launch != 0 runs like tmla_mla_decode_fused (default spin limit),
 * else like tmla_mla_decode. q_len = 1 gives tmla_mla_decode's results bit for bit.
 */
int tmla_mla_decode_causal(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                           int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                           int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                           int32_t bt_cols, const int32_t* seqlens, int32_t batch, int32_t q_len,
                           int32_t num_heads, int32_t head_dim_v, int32_t rope_dim, int32_t dtype,
                           float softmax_scale, int32_t num_splits, int32_t num_workers, void* out,
                           int64_t out_stride_b, int64_t out_stride_h, float* lse, void* workspace,
                           size_t workspace_bytes, int32_t single_launch, void* stream);
/*
 * Decode over an fp8 latent cache, no counterpart in the reference (its
 * README.md:32-33 lists "no FP8 cache" among the limitations). Both stages,
 * like tmla_mla_decode_causal (q_len = 1: single-token decode), with:
 *   kv       one byte per element, OCP FP8 E4M3 ("e4m3fn": bias 7, no
 *            infinities, 0x7f/0xff NaN), same layout as the 16-bit cache with
 *            strides in elements (= bytes); page_size a multiple of 16 when
 *            paged; strides multiples of 16.
 *   kv_scale float32; cache row t of sequence b stands for
 *            e4m3(byte) * kv_scale[page * scale_stride_0 + (t % page_size) *
 *            scale_stride_1] (dense: kv_scale[b * scale_stride_0 + t *
 *            scale_stride_1]): one scale per page (stride_1 = 0), per token,
 *            or per tensor (both 0). The array must hold every index a page
 *            id < num_blocks and a row < page_size can form.
 *   dtype    the element type of q and out (TMLA_BF16 or TMLA_FP16).
 * The attention is the reference's over the dequantised cache: scores of
 * the widened (exact) fp8 values times the row's scale, probabilities times
 * the row's scale rounded to dtype for the value product, float32
 * accumulation. The workspace is tmla_workspace_bytes(batch, q_len *
 * num_heads, ...); the partials use tmla_mla_decode_combine's format.
 * With more than 16 (virtual) heads, one scale per page or per tensor
 * (scale_stride_1 = 0) and pages of a power-of-two multiple of 32 tokens, the
 * cache is widened once per workgroup into the 16-bit kernel's ring; other
 * calls run groups of 16 heads that each stream the cache.
 */
int tmla_mla_decode_fp8(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                        int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                        const float* kv_scale, int64_t scale_stride_0, int64_t scale_stride_1,
                        const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                        const int32_t* seqlens, int32_t batch, int32_t q_len, int32_t num_heads,
                        int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                        int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                        int64_t out_stride_h, float* lse, void* workspace, size_t workspace_bytes,
                        void* stream);
/*
 * Stage 1 of tmla_mla_decode_fp8 alone (q_len = 1); stage 2 is
 * tmla_mla_decode_combine with the same partition arguments.
 */
int tmla_mla_decode_fp8_partial(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                                int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                                int32_t page_size, const float* kv_scale, int64_t scale_stride_0,
                                int64_t scale_stride_1, const int32_t* block_table, int64_t bt_stride_b,
                                int32_t bt_cols, const int32_t* seqlens, int32_t batch,
                                int32_t num_heads, int32_t head_dim_v, int32_t rope_dim, int32_t dtype,
                                float softmax_scale, int32_t num_splits, int32_t num_workers, void* out,
                                int64_t out_stride_b, int64_t out_stride_h, float* lse, void* workspace,
                                size_t workspace_bytes, void* stream);
/*
 * Decode for the head dims and element types the kernels above are not built
 * for. The reference's kernels take any power-of-two head_dim_v and rope_dim
 * (src/triton_mla/kernel.py:243-244) and any element type shared by q and
 * the cache (kernel.py:245); this entry point takes head_dim_v a power of
 * two in [16, 1024], rope_dim a power of two in [16, 256] and dtype
 * TMLA_BF16, TMLA_FP16 or TMLA_FP32, and runs both of the reference's
 * stages the reference's way: sequence b is cut into num_splits pieces of
 * cdiv(seqlens[b], num_splits) tokens (kernel.py:84-86), one workgroup per
 * (16 heads, piece, sequence), each writing a float32 partial and its base-2
 * log-sum-exp (kernel.py:43-138, launch kernel.py:276-302), which a second
 * kernel merges (kernel.py:141-181, launch kernel.py:303-320). Scores and
 * sums in float32, probabilities rounded to dtype for the value product
 * (kernel.py:123). bf16 / fp16 calls with head_dim_v <= 512 and
 * head_dim_v + rope_dim <= 576 run on matrix cores (v_mfma_f32_16x16x32,
 * 64 heads per workgroup), the others on the vector ALU (16 heads per
 * workgroup): for unusual dims, not at the speed of the kernels above. Arguments mean what they mean for tmla_mla_decode;
 * num_splits in [1, 65535]; batch and num_heads at most 65535; the
 * workspace is tmla_generic_workspace_bytes(batch, num_heads, head_dim_v,
 * num_splits) bytes and needs no initialisation. Sequence lengths above the
 * cache's capacity are cut to it.
 */
size_t tmla_generic_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim_v, int32_t num_splits);
/*
 * Heads per workgroup of tmla_mla_decode_generic's stage 1 for these dims and
 * element type (64: the matrix-core form, for bf16 / fp16 with head_dim_v <=
 * 512 and head_dim_v + rope_dim <= 576; 16: the vector-ALU form; 0: not
 * accepted), for callers that size num_splits to the device. No counterpart
 * in the reference (its autotune picks BLOCK_H, kernel.py:32-46).
 */
int32_t tmla_generic_heads_per_workgroup(int32_t head_dim_v, int32_t rope_dim, int32_t dtype);
int tmla_mla_decode_generic(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                            int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                            const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                            const int32_t* seqlens, int32_t batch, int32_t num_heads, int32_t head_dim_v,
                            int32_t rope_dim, int32_t dtype, float softmax_scale, int32_t num_splits, void* out,
                            int64_t out_stride_b, int64_t out_stride_h, float* lse, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Profiling hook, no counterpart in the reference: copies the partial
 * kernel's phase stamps of the last launch into `host` (up to `bytes`):
 * 4096 workers x 9 slots x {100 MHz wall clock, shader clock} uint64 (slot
 * meanings in mla_decode.hip, phase_stamp). Synchronous. Only a library
 * built with TMLA_STAMPS=1 records stamps; any other build returns
 * TMLA_ERR_UNSUPPORTED.
 */
int tmla_debug_stamps(void* host, size_t bytes);

/* Number of compute units of `device` (0 on error); the default worker count. */
int32_t tmla_device_cu_count(int32_t device);

/*
 * MLA layer glue: the absorbed-projection steps on either side of
 * tmla_mla_decode in one decode step of the DeepSeek MLA layer, and the
 * dense projections (wq_a, wq_b, wkv_a, wo) of a step's few rows. wkv_b is the
 * layer's [num_heads * (qk_nope_dim + v_head_dim), kv_lora_rank] weight with
 * row stride wkv_b_stride_0: rows h*(nope+v) .. +nope are W_UK[h], the next v
 * rows W_UV[h] (the reference's view, src/triton_mla/model.py:96-99).
 */

/*
 * Query side of the absorbed step: for every (b, h)
 *   q_out[b, h, :rank]  = q_proj[b, h*(nope+rope) : +nope] . W_UK[h]
 *   q_out[b, h, rank:]  = RoPE(q_proj[b, h*(nope+rope)+nope : +rope], positions[b])
 * Replaces the q_pe RoPE of `MLA._project` (src/triton_mla/model.py:74-83,
 * apply_rope model.py:44-50: rotate-half, theta ** (2i/rope), float32) and the
 * W_UK einsum + concatenation of `MLA.forward` (model.py:108-109).
 * q_proj is wq_b's output [batch, num_heads*(nope+rope)] (row stride
 * q_proj_stride_b); q_out [batch, num_heads, rank+rope] with element strides
 * (q_out_stride_b, q_out_stride_h, 1). Built for qk_nope_dim 128,
 * qk_rope_dim 64 and kv_lora_rank a multiple of 128.
 */
int tmla_mla_absorb_q(const void* q_proj, int64_t q_proj_stride_b, const void* wkv_b,
                      int64_t wkv_b_stride_0, const int32_t* positions, int32_t batch,
                      int32_t num_heads, int32_t qk_nope_dim, int32_t qk_rope_dim,
                      int32_t kv_lora_rank, int32_t v_head_dim, float rope_theta, int32_t dtype,
                      void* q_out, int64_t q_out_stride_b, int64_t q_out_stride_h, void* stream);

/*
 * Output side of the absorbed step:
 *   out[b, h*v_head_dim + v] = o_latent[b, h, :] . W_UV[h][v, :]
 * Replaces the W_UV einsum of `MLA.forward` (src/triton_mla/model.py:120-124);
 * out [batch, num_heads*v_head_dim] (row stride out_stride_b) is the input of
 * the wo projection. o_latent is mla_decode's output [batch, num_heads,
 * kv_lora_rank], element strides (o_stride_b, o_stride_h, 1). Built for
 * v_head_dim a multiple of 32 and kv_lora_rank a multiple of 512.
 */
int tmla_mla_absorb_out(const void* o_latent, int64_t o_stride_b, int64_t o_stride_h,
                        const void* wkv_b, int64_t wkv_b_stride_0, int32_t batch,
                        int32_t num_heads, int32_t qk_nope_dim, int32_t kv_lora_rank,
                        int32_t v_head_dim, int32_t dtype, void* out, int64_t out_stride_b,
                        void* stream);

/*
 * Cache append of the new token: for every sequence b
 *   row = [RMSNorm(kv_proj[b, :rank]) * norm_weight, RoPE(kv_proj[b, rank:rank+rope])]
 * written at position positions[b] (= cache_seqlens before the step) of
 * sequence b: page block_table[b, pos / page_size], row pos % page_size, or
 * row pos of sequence b when block_table is NULL (dense [batch, capacity, D],
 * page_size 1, num_blocks = capacity). Replaces the kv half of `MLA._project`
 * (src/triton_mla/model.py:80-83; RMSNorm model.py:34-41) and
 * `MLA._append_kv` (model.py:86-94). RMSNorm in float32 (normalised value
 * times the weight, rounded once to the cache dtype). A position
 * whose page slot or page id lies outside the table or the cache is not
 * written. norm_weight may be NULL (weight 1). Built for rope_dim 64 and
 * kv_lora_rank a multiple of 64 up to 1024.
 */
int tmla_mla_kv_append(const void* kv_proj, int64_t kv_proj_stride_b, const void* norm_weight,
                       float eps, float rope_theta, const int32_t* positions, int32_t batch,
                       int32_t kv_lora_rank, int32_t rope_dim, int32_t dtype, void* kv_cache,
                       int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                       int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                       int32_t bt_cols, void* stream);

/*
 * RMSNorm of rows: y[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * weight
 * in float32 (the normalised value times the weight), rounded once to the
 * dtype. Replaces `RMSNorm.forward` (src/triton_mla/model.py:34-41) on the
 * query latent of `MLA._project` (model.py:76). weight [dim] may be NULL
 * (weight 1). Row strides in elements, multiples of 8; x, weight and y
 * 16-byte aligned; built for dim a multiple of 8.
 */
int tmla_mla_rms_norm(const void* x, int64_t x_stride, const void* weight, float eps, int32_t rows,
                      int32_t dim, int32_t dtype, void* y, int64_t y_stride, void* stream);

/*
 * The query latent's RMSNorm (tmla_mla_rms_norm on batch rows of q_dim) and
 * the cache append of the new token (tmla_mla_kv_append) in one launch, with
 * the same arithmetic and bits as the two calls, plus next_positions[b] =
 * positions[b] + 1 (the sequence lengths after the step, which the step's
 * decode reads). The two read different rows of the step's first projection
 * and do not depend on each other. Replaces `q_norm` (src/triton_mla/
 * model.py:76), the kv half of `MLA._project` and `MLA._append_kv`
 * (model.py:80-94) and `cache_seqlens + 1` (model.py:109) of one step.
 */
int tmla_mla_norm_append(const void* q_lat, int64_t q_lat_stride, const void* q_norm_weight,
                         float q_eps, int32_t q_dim, void* q_out, int64_t q_out_stride,
                         const void* kv_proj, int64_t kv_proj_stride_b, const void* kv_norm_weight,
                         float kv_eps, float rope_theta, const int32_t* positions,
                         int32_t* next_positions, int32_t batch, int32_t kv_lora_rank,
                         int32_t rope_dim, int32_t dtype, void* kv_cache, int64_t kv_stride_0,
                         int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                         const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                         void* stream);

/*
 * Dense projection of a decode step's rows: y[m, n] = x[m, :] . w[n, :]
 * (float32 accumulation, rounded once to the dtype), i.e. nn.Linear without
 * bias with w in its [out_features, in_features] layout. Replaces the
 * library GEMMs of the four projections of `MLA.forward` / `MLA._project`
 * (src/triton_mla/model.py:66-72 define them; model.py:74-82, 124 apply
 * them) for batches of at most 64 rows, where a GEMM library's tiles leave
 * most compute units idle: every weight row is read once, by workgroups of
 * 64 (or 16) output columns, and the contraction is split over the waves of
 * a workgroup and, when there are few column groups, over several
 * workgroups, whose tiles are summed in a fixed order, so the result does
 * not depend on timing. Row strides in elements; x and w 16-byte aligned
 * with row strides a multiple of 8. Built for m <= 64, n a multiple of 16
 * and k a multiple of 64 (TMLA_ERR_UNSUPPORTED otherwise).
 *
 * workspace: tmla_mla_project_workspace_bytes(m, n, k) bytes, 256-byte
 * aligned (may be NULL when that is 0), zero-filled before its first use:
 * a fixed 64 KiB block of arrival counters, then the partial tiles of a
 * split contraction. Every call leaves its counters at zero again, so one
 * buffer at least as large as each call's need serves calls of any shapes
 * in turn. Calls that share a workspace must not run concurrently.
 */
size_t tmla_mla_project_workspace_bytes(int32_t m, int32_t n, int32_t k);
int tmla_mla_project(const void* x, int64_t x_stride, const void* w, int64_t w_stride, int32_t m,
                     int32_t n, int32_t k, int32_t dtype, void* y, int64_t y_stride, void* workspace,
                     size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRITON_MLA_H */
