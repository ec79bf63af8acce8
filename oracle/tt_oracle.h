/*
 * tt_oracle.h -- CPU restatement of TriTierCache's fused decode step.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle for the HIP
 * implementation in tritiercache_amd/. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and only to check or to time
 * the CPU side. The product path never calls into it.
 *
 * Every function restates the reference algorithm in plain, single-threaded
 * C11 (compiled with -ffp-contract=off; every fused multiply-add the reference
 * performs is written as an explicit fmaf). Citations are to the reference
 * repository (RahulGPi/TriTierCache).
 *
 * Parity pins (how each function is checked, see tests/test_oracle.py):
 *   orc_quantize_v_block   reference KAT vectors (tests/test_quantize_v.cpp,
 *                          tests/tie_test_v.cpp) + bit-exact vs compiled reference
 *   orc_quantize_k_block   bit-exact vs compiled reference + closed-form brute force
 *   orc_dequantize_k/v     bit-exact vs compiled reference + closed form
 *   orc_fused_attention_decode   bit-exact vs compiled reference on this host
 *                          (same glibc expf), float64 brute force within 1e-5
 *   orc_engine_*           bit-exact state vs the compiled reference engine,
 *                          step by step (fixtures + live)
 */
#ifndef TT_ORACLE_H
#define TT_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 conversions with the semantics of F16C vcvtps2ph imm8=0
 * (round to nearest even, denormals kept, NaN quieted) and vcvtph2ps. */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);

/* quantize_k_avx2.cpp:26-110. K [kgs, H, D] token-major; packed [(kgs/16), H, D];
 * scale/zero [H, D] as float (meta_fp16=0) or uint16 half bits (meta_fp16=1). */
void orc_quantize_k_block(const float* K, uint32_t* packed, void* scale_out, void* zero_out,
                          int num_heads, int head_dim, int k_group_size, int meta_fp16);

/* quantize_v_avx2.cpp:44-108. V [chunk, H, D]; packed [chunk, H, ceil(D/16)];
 * scale/zero [chunk, H]. head_dim must be a multiple of 16 (the reference
 * reads 16 channels per group unconditionally, :91-92). */
void orc_quantize_v_block(const float* V, int32_t* packed, void* scale_out, void* zero_out,
                          int num_heads, int head_dim, int chunk_size, int meta_fp16);

/* dequantize_avx2.cpp:24-110 (K) and :138-204 (V). */
void orc_dequantize_k(const int32_t* packed, const void* scale, const void* zero, float* out,
                      int num_blocks, int num_heads, int head_dim, int k_group_size, int meta_fp16);
void orc_dequantize_v(const int32_t* packed, const void* scale, const void* zero, float* out,
                      int total_tokens, int num_heads, int head_dim, int meta_fp16);

/* fused_attn_avx2.cpp:145-301: dequantise every block, two-pass softmax,
 * GQA kv_h = h / (Hq/Hkv), -1 token ids masked, optional mean weights. */
void orc_fused_attention_decode(const float* Q, const float* dense_K, const float* dense_V,
                                int dense_count, const int32_t* PBS_K_Packed,
                                const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                                const int32_t* PBS_V_Packed, const void* PBS_V_Scales,
                                const void* PBS_V_Zeroes, const int64_t* PBS_token_ids,
                                int num_blocks, int num_q_heads, int num_kv_heads, int head_dim,
                                float* attn_output, float* mean_attn_weights, int k_group_size,
                                int meta_fp16);

/* ---- Engine: cache_engine.h:10-123 / cache_engine.cpp ---- */
typedef struct orc_engine orc_engine;

orc_engine* orc_engine_create(int num_q_heads, int num_kv_heads, int head_dim, int max_seq_len,
                              int sink_size, int rw_size, float h_ratio, float score_decay,
                              int update_interval, int k_group_size, int meta_fp16);
void orc_engine_destroy(orc_engine* e);
/* cache_engine.cpp:397-541 */
void orc_engine_step(orc_engine* e, const float* Q, const float* K_new, const float* V_new,
                     float* attn_output);
/* cache_engine.cpp:271-395 */
void orc_engine_prefill(orc_engine* e, const float* K_all, const float* V_all, int q_len);
/* The two halves of step() around the attention call: ingest (:405-431) and
 * score feedback (:511-540) with caller-supplied mean weights, for lockstep
 * runs where the weights come from elsewhere. */
void orc_engine_ingest(orc_engine* e, const float* K_new, const float* V_new);
void orc_engine_feedback(orc_engine* e, const float* mean_attn_weights);
/* Attention over the current visible set (:433-509) without feedback. */
void orc_engine_attend(orc_engine* e, const float* Q, float* attn_output, float* mean_weights);
/* Number of visible tokens: s_count + hh_count + rw_count + blocks_used*chunk. */
int orc_engine_visible(const orc_engine* e);
size_t orc_engine_buffer_bytes(const orc_engine* e);

/* Counters, in this order: num_q_heads num_kv_heads head_dim max_seq_len sink_size
 * rw_size update_interval k_group_size chunk_size quant_head_dim max_hh use_fp16_meta
 * s_count rw_count rw_head_index hh_count wr_count pbs_allocated_blocks pbs_blocks_used
 * pbs_count total_processed_tokens last_calc_pos total_evictions */
#define ORC_N_COUNTERS 23
void orc_engine_counters(const orc_engine* e, int64_t* out);
float orc_engine_cached_threshold(const orc_engine* e);

/* Raw buffer access (host memory owned by the engine). which:
 * 0 S_K 1 S_V 2 RW_K 3 RW_V 4 HH_K 5 HH_V 6 HH_token_ids 7 HH_scores 8 WR_K 9 WR_V
 * 10 WR_token_ids 11 PBS_K_Packed 12 PBS_K_Scales 13 PBS_K_Zeroes 14 PBS_V_Packed
 * 15 PBS_V_Scales 16 PBS_V_Zeroes 17 PBS_token_ids 18 global_attn_scores
 * Returns the pointer and writes the element count and element size. */
void* orc_engine_buffer(orc_engine* e, int which, int64_t* numel, int* elem_size);

#ifdef __cplusplus
}
#endif
#endif
