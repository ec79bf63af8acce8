/*
 * tritiercache_amd.h -- C ABI of the MI355X (gfx950) TriTierCache decode path.
 *
 * Drop-in replacement for the compute surface of the reference's `tri_tier._C`
 * extension (csrc/bindings.cpp). Every entry point takes plain pointers and
 * sizes. Tensor pointers are DEVICE pointers (HBM) unless stated otherwise;
 * `stream` is a hipStream_t passed as void* (NULL = the default stream). All
 * work is enqueued on `stream`; no entry point synchronises the host unless its
 * comment says so.
 *
 * Return value: TT_OK (0) or one of the TT_ERR_* codes; tt_last_error() then
 * returns a message for the calling thread. The codes map onto the Python
 * exceptions the reference's exception translator raises
 * (bindings.cpp:321-337): INVALID_ARGUMENT -> ValueError, OUT_OF_RANGE ->
 * IndexError, NO_MEMORY -> MemoryError, RUNTIME / HIP -> RuntimeError.
 *
 * Metadata dtype: meta_fp16 = 0 selects FP32 scale/zero arrays (float*),
 * meta_fp16 = 1 selects IEEE binary16 stored as uint16_t, as in the reference
 * (pbs_metadata_dtype "fp32" / "fp16").
 */
#ifndef TRITIERCACHE_AMD_H
#define TRITIERCACHE_AMD_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define TT_API __attribute__((visibility("default")))
#else
#define TT_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define TT_OK 0
#define TT_ERR_INVALID_ARGUMENT 1
#define TT_ERR_OUT_OF_RANGE 2
#define TT_ERR_NO_MEMORY 3
#define TT_ERR_RUNTIME 4
#define TT_ERR_HIP 5

/* Message for the last failing call on this thread ("" if none). */
TT_API const char* tt_last_error(void);

/* Library version string, e.g. "tritiercache_amd 0.1.0 gfx950". */
TT_API const char* tt_version(void);

/* Number of visible HIP devices (0 when no GPU or no driver). Never fails. */
TT_API int tt_device_count(void);

/* Classifies an address: 0 = not known to HIP (pageable host memory),
 * 1 = device memory, 2 = host memory registered with / allocated by HIP.
 * Lets the Python layer accept the reference's raw integer addresses. */
TT_API int tt_pointer_kind(const void* ptr);

/* ---------------------------------------------------------------------------
 * Stateless kernels
 * ------------------------------------------------------------------------- */

/* Replaces _C.quantize_k_block (bindings.cpp:180-212, kernel
 * csrc/cpu/quantize_k_avx2.cpp:26-110), batched over `num_blocks` consecutive
 * blocks. K: [num_blocks * k_group_size, num_heads, head_dim] f32.
 * packed: [num_blocks * k_group_size/16, num_heads, head_dim] u32.
 * scale, zero: [num_blocks, num_heads, head_dim]. Bit-exact with the reference. */
TT_API int tt_quantize_k_block(const float* K, uint32_t* packed, void* scale, void* zero, int num_blocks,
                        int num_heads, int head_dim, int k_group_size, int meta_fp16, void* stream);

/* Replaces _C.quantize_v_block (bindings.cpp:214-246, kernel
 * csrc/cpu/quantize_v_avx2.cpp:44-108). V: [tokens, num_heads, head_dim] f32,
 * packed: [tokens, num_heads, head_dim/16] i32, scale/zero: [tokens, num_heads].
 * head_dim must be a multiple of 16. Bit-exact with the reference. */
TT_API int tt_quantize_v_block(const float* V, int32_t* packed, void* scale, void* zero, int tokens,
                        int num_heads, int head_dim, int meta_fp16, void* stream);

/* Replaces _C.dequantize_k (bindings.cpp:248-281, csrc/cpu/dequantize_avx2.cpp:24-110).
 * out: [num_blocks * k_group_size, num_heads, head_dim] f32. */
TT_API int tt_dequantize_k(const int32_t* packed, const void* scale, const void* zero, float* out,
                    int num_blocks, int num_heads, int head_dim, int k_group_size, int meta_fp16,
                    void* stream);

/* Replaces _C.dequantize_v (bindings.cpp:283-315, csrc/cpu/dequantize_avx2.cpp:138-204).
 * head_dim must be a multiple of 16. */
TT_API int tt_dequantize_v(const int32_t* packed, const void* scale, const void* zero, float* out,
                    int total_tokens, int num_heads, int head_dim, int meta_fp16, void* stream);

/* Replaces _C.fused_attention_decode (bindings.cpp:99-178, 340-363; kernel
 * csrc/cpu/fused_attn_avx2.cpp:145-301). Single-pass split-K decode attention
 * over the FP32 dense tiers and the 2-bit packed blocks, GQA head grouping,
 * -1 token ids masked, optional mean attention weights
 * [dense_count + num_blocks*k_group_size].
 * Requirements beyond the reference's: num_q_heads % num_kv_heads == 0,
 * head_dim a multiple of 16 of at most 256, and, with mean weights,
 * num_q_heads x tokens x 4 bytes of logits within 4 GiB (the same bound
 * holds for every attention entry point and for tt_engine_create's
 * max_seq_len).
 * Uses a library-owned device workspace (grown on demand, one per device);
 * concurrent calls on one device race on it -- use the _ws variant for that.
 * Growing it synchronises the device and frees the previous buffer, so a HIP
 * graph captured around an earlier call must not be replayed after a call
 * with a larger workspace (capture the _ws or _noalloc variant instead). */
TT_API int tt_fused_attention_decode(const float* Q, const float* dense_K, const float* dense_V,
                              int dense_count, const int32_t* PBS_K_Packed,
                              const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                              const int32_t* PBS_V_Packed, const void* PBS_V_Scales,
                              const void* PBS_V_Zeroes, const int64_t* PBS_token_ids,
                              int num_blocks, int num_q_heads, int num_kv_heads, int head_dim,
                              float* attn_output, float* mean_attn_weights, int k_group_size,
                              int meta_fp16, void* stream);

/* Same computation with a caller-provided device workspace of at least
 * tt_fused_attention_workspace_bytes(...) bytes. No allocation. The size
 * query validates its arguments as the entry points do and returns 0 (with
 * tt_last_error set) for arguments they would reject. */
TT_API size_t tt_fused_attention_workspace_bytes(int dense_count, int num_blocks, int num_q_heads,
                                          int num_kv_heads, int head_dim, int k_group_size,
                                          int want_mean_weights);
TT_API int tt_fused_attention_decode_ws(const float* Q, const float* dense_K, const float* dense_V,
                                 int dense_count, const int32_t* PBS_K_Packed,
                                 const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                                 const int32_t* PBS_V_Packed, const void* PBS_V_Scales,
                                 const void* PBS_V_Zeroes, const int64_t* PBS_token_ids,
                                 int num_blocks, int num_q_heads, int num_kv_heads, int head_dim,
                                 float* attn_output, float* mean_attn_weights, int k_group_size,
                                 int meta_fp16, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the computation of tt_fused_attention_decode, with its
 * scratch in a static device array of the library (32 MiB, held by every GPU
 * the library runs on until the process ends) instead of an allocated
 * workspace. Calls no hipMalloc/hipFree. A call whose workspace would exceed
 * 32 MiB (tt_fused_attention_workspace_bytes) fails with
 * TT_ERR_INVALID_ARGUMENT and enqueues nothing. All calls on one GPU share that
 * GPU's array: calls that overlap on one GPU (other streams, other host
 * threads) race on it. */
TT_API int tt_fused_attention_decode_noalloc(const float* Q, const float* dense_K, const float* dense_V,
                                             int dense_count, const int32_t* PBS_K_Packed,
                                             const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                                             const int32_t* PBS_V_Packed, const void* PBS_V_Scales,
                                             const void* PBS_V_Zeroes, const int64_t* PBS_token_ids,
                                             int num_blocks, int num_q_heads, int num_kv_heads, int head_dim,
                                             float* attn_output, float* mean_attn_weights, int k_group_size,
                                             int meta_fp16, void* stream);

/* The two phases of tt_fused_attention_decode_ws, for callers that merge
 * split-K partials themselves or overlap the phases:
 *   tt_attention_partials  the single-pass split kernel: per (query head,
 *                          split) running max, sum and weighted V accumulator
 *                          (+ per-token logits when want_mean_weights) into
 *                          `workspace`;
 *   tt_attention_finalize  what reads them. With both attn_output and
 *                          mean_attn_weights: the log-sum-exp merge and the mean
 *                          attention weights in one launch. With attn_output
 *                          only: the merge alone, which also leaves each query
 *                          head's softmax statistics in the workspace. With
 *                          mean_attn_weights only: the mean weights from those
 *                          statistics; it must follow a merge-only call on the
 *                          same workspace and partials (in stream order, or
 *                          after an event when called on another stream: the
 *                          mean weights then overlap later work on the first
 *                          stream, e.g. the next layer's partials).
 * All calls of one decode step take the same shape arguments and
 * want_mean_weights. No counterpart in the reference, which has a single entry
 * point (bindings.cpp:99-178). */
TT_API int tt_attention_partials(const float* Q, const float* dense_K, const float* dense_V,
                                 int dense_count, const int32_t* PBS_K_Packed,
                                 const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                                 const int32_t* PBS_V_Packed, const void* PBS_V_Scales,
                                 const void* PBS_V_Zeroes, const int64_t* PBS_token_ids,
                                 int num_blocks, int num_q_heads, int num_kv_heads, int head_dim,
                                 int k_group_size, int meta_fp16, int want_mean_weights,
                                 void* workspace, size_t workspace_bytes, void* stream);
TT_API int tt_attention_finalize(const float* Q, int dense_count, int num_blocks, int num_q_heads,
                                 int num_kv_heads, int head_dim, float* attn_output,
                                 float* mean_attn_weights, int k_group_size, int meta_fp16,
                                 int want_mean_weights, void* workspace, size_t workspace_bytes,
                                 void* stream);
/* For callers that run layers back to back: the merge of this call's
 * partials into attn_output (as tt_attention_finalize with mean_attn_weights
 * NULL, leaving the softmax statistics in `workspace`) and, in the same launch,
 * the mean attention weights of an earlier call that merged that way, whose
 * partials are still in `prev_workspace` (planned with want_mean_weights = 1,
 * prev_dense_count tokens and prev_num_blocks blocks, the same shape
 * arguments), into prev_mean_attn_weights. The two workspaces must not
 * overlap. A layer's mean weights then ride in the next layer's finalize
 * launch, and only the last layer's need a launch of their own
 * (tt_attention_finalize with attn_output NULL). No counterpart in the
 * reference (bindings.cpp:99-178 returns both from one call). */
TT_API int tt_attention_finalize_deferred(const float* Q, int dense_count, int num_blocks,
                                          int num_q_heads, int num_kv_heads, int head_dim,
                                          float* attn_output, int k_group_size, int meta_fp16,
                                          void* workspace, size_t workspace_bytes,
                                          int prev_dense_count, int prev_num_blocks,
                                          float* prev_mean_attn_weights, void* prev_workspace,
                                          size_t prev_workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Batched ragged decode: one decode step of many sequences, each with its own
 * tier tables and lengths, in one split-K launch plus one merge launch (head_dim
 * 128; other head dims run the sequences one after another). No counterpart
 * in the reference, whose callers run fused_attention_decode (bindings.cpp:
 * 99-178) once per sequence; each sequence's result is that call's result.
 *
 * One tt_decode_seq holds the arguments of tt_fused_attention_decode for one
 * sequence (all device pointers; mean_attn_weights may be NULL, the PBS
 * pointers are unused when num_blocks == 0 and the dense ones when
 * dense_count == 0). */
typedef struct tt_decode_seq {
    const float* Q;                  /* [Hq, D] */
    const float* dense_K;            /* [dense_count, Hkv, D] */
    const float* dense_V;            /* [dense_count, Hkv, D] */
    const int32_t* PBS_K_Packed;     /* [num_blocks * k_group_size / 16, Hkv, D] */
    const void* PBS_K_Scales;        /* [num_blocks, Hkv, D] */
    const void* PBS_K_Zeroes;        /* [num_blocks, Hkv, D] */
    const int32_t* PBS_V_Packed;     /* [num_blocks * k_group_size, Hkv, D / 16] */
    const void* PBS_V_Scales;        /* [num_blocks * k_group_size, Hkv] */
    const void* PBS_V_Zeroes;        /* [num_blocks * k_group_size, Hkv] */
    const int64_t* PBS_token_ids;    /* [num_blocks * k_group_size], -1 = masked slot */
    float* attn_output;              /* [Hq, D] */
    float* mean_attn_weights;        /* [dense_count + num_blocks * k_group_size] or NULL */
    int32_t dense_count;
    int32_t num_blocks;
} tt_decode_seq;

/* Device workspace bytes for tt_fused_attention_decode_batched over `seqs`
 * (host array; only the counts and the mean_attn_weights pointers are read).
 * 0 on invalid arguments. */
TT_API size_t tt_batched_decode_workspace_bytes(const tt_decode_seq* seqs, int num_seqs, int num_q_heads,
                                                int num_kv_heads, int head_dim, int k_group_size);

/* `seqs` (host memory) is read by the call to plan the launch; the kernels
 * read `seqs_device`, a device copy of the same array, which must stay valid
 * and unchanged until the work enqueued on `stream` has run. All sequences
 * share the head counts, head_dim, k_group_size and metadata dtype. The
 * workspace must hold tt_batched_decode_workspace_bytes(...) bytes. No
 * allocation. */
TT_API int tt_fused_attention_decode_batched(const tt_decode_seq* seqs, const tt_decode_seq* seqs_device,
                                             int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                             int k_group_size, int meta_fp16, void* workspace,
                                             size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Engine: replaces _C.TriTierCacheEngine (bindings.cpp:384-626, class
 * csrc/include/cache_engine.h:10-123, csrc/cache_engine.cpp). All tier buffers
 * and counters live in device memory; a step enqueues its kernels without a
 * host synchronisation.
 * ------------------------------------------------------------------------- */
typedef struct tt_engine tt_engine;

/* cache_engine.cpp:8-82. pbs_metadata_dtype: "fp16" selects FP16 metadata,
 * anything else FP32; k_group_size 32 selects 32, anything else 16. The
 * engine lives on the current HIP device. */
TT_API int tt_engine_create(tt_engine** out, int num_q_heads, int num_kv_heads, int head_dim,
                     int max_seq_len, int sink_size, int rw_size, float h_ratio, float score_decay,
                     int update_interval, int k_group_size, const char* pbs_metadata_dtype,
                     void* stream);
TT_API int tt_engine_destroy(tt_engine* e);

/* cache_engine.cpp:397-541: ingest (ring eviction, routing, waiting-room
 * flush), attention over sinks + heavy hitters + recent window + packed
 * blocks, decayed score feedback. Q [Hq*D], K_new/V_new [Hkv*D],
 * attn_output [Hq*D]: device f32. */
TT_API int tt_engine_step(tt_engine* e, const float* Q, const float* K_new, const float* V_new,
                   float* attn_output, void* stream);

/* step() plus the per-head softmax weights of this step, written as
 * [num_q_heads, visible] f32 in the engine's visible order (sinks, heavy-hitter
 * slots, recent window oldest first, packed slots). `visible_out` (host int)
 * receives the visible count; this call synchronises `stream`.
 * `head_weights_capacity` (columns per head row): the visible count before the
 * step plus max(1, chunk_size) always suffices, as one step adds at most one
 * visible token or one flushed block. A capacity that the step's visible count
 * could exceed (by the engine's host-side tier bounds and by that count)
 * returns TT_ERR_OUT_OF_RANGE before the step is enqueued, with the engine
 * unchanged. */
TT_API int tt_engine_step_weights(tt_engine* e, const float* Q, const float* K_new, const float* V_new,
                           float* attn_output, float* head_weights, int head_weights_capacity,
                           int* visible_out, void* stream);

/* cache_engine.cpp:271-395. K_all/V_all [q_len, Hkv, D] device f32. */
/* tt_engine_step for callers that step the engines of a model's layers one
 * after another: this engine's step runs up to its merged attention output,
 * and its mean attention weights and score feedback are left pending; the
 * pending feedback of `prev` (another engine on the same device, NULL for the
 * first layer) runs in the same launch as this engine's merge. Each engine's
 * pending feedback must run before its next step: it does so in the finalize
 * launch of the next engine stepped this way, in tt_engine_flush_feedback, or
 * at the start of any later call on that engine (step, prefill, feedback,
 * counters, buffers) on that call's stream, which must be ordered after the
 * stream of the step that left it (the same stream, or the caller's events).
 * A call that fails to launch the pending feedback leaves it pending. The
 * state after the feedback is
 * the state tt_engine_step leaves (the mean weights from the merge's softmax
 * statistics, within 1e-6 of those it rebuilds). No counterpart in the
 * reference, whose step (cache_engine.cpp:397-541) runs its feedback last. */
TT_API int tt_engine_step_deferred(tt_engine* e, const float* Q, const float* K_new,
                                   const float* V_new, float* attn_output, tt_engine* prev,
                                   void* stream);
TT_API int tt_engine_flush_feedback(tt_engine* e, void* stream);
TT_API int tt_engine_prefill(tt_engine* e, const float* K_all, const float* V_all, int q_len, void* stream);

/* The two halves of step() around the attention, for tier maintenance in
 * isolation: ingest (cache_engine.cpp:405-431) and the score feedback
 * (:511-540) with caller-supplied mean weights [visible] (device f32). */
TT_API int tt_engine_ingest(tt_engine* e, const float* K_new, const float* V_new, void* stream);
TT_API int tt_engine_feedback(tt_engine* e, const float* mean_attn_weights, void* stream);

/* Counters (synchronises `stream`), in the order of tt_engine_counter_names(). */
#define TT_ENGINE_N_COUNTERS 23
TT_API int tt_engine_counters(tt_engine* e, int64_t* out, void* stream);
TT_API const char* tt_engine_counter_names(void);

/* get_buffer_bytes (cache_engine.cpp:543-568): the reference's accounting of
 * allocated tier bytes, with the PBS sized by pbs_allocated_blocks
 * (synchronises `stream`). */
TT_API int tt_engine_buffer_bytes(tt_engine* e, size_t* out, void* stream);

/* Device pointer and logical element count of a tier buffer, for the
 * zero-copy getters (bindings.cpp:461-626). which: 0 S_K 1 S_V 2 RW_K 3 RW_V
 * 4 HH_K 5 HH_V 6 HH_token_ids 7 HH_scores 8 WR_K 9 WR_V 10 WR_token_ids
 * 11 PBS_K_Packed 12 PBS_K_Scales 13 PBS_K_Zeroes 14 PBS_V_Packed 15 PBS_V_Scales
 * 16 PBS_V_Zeroes 17 PBS_token_ids 18 global_attn_scores 19 mean attention
 * weights of the last step [visible] (no reference getter). PBS buffers are sized
 * by pbs_allocated_blocks (synchronises `stream`). The pointers stay valid
 * until the physical PBS capacity grows (only past max_seq_len tokens). */
TT_API int tt_engine_buffer(tt_engine* e, int which, void** dev_ptr, int64_t* numel, int* elem_size,
                     void* stream);

/* Visible token count after the last enqueued call (synchronises `stream`). */
TT_API int tt_engine_visible(tt_engine* e, int* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
