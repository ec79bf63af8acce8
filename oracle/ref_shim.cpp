// ref_shim.cpp -- C entry points over the reference's own compiled C++ sources.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with
// the reference's csrc/cache_engine.cpp and csrc/cpu/*_avx2.cpp, taken from
// where they lie in the reference checkout, with the reference's own flags
// (setup.py:37-40: -O3 -fopenmp -mavx2 -mbmi2 -mfma -mf16c, C++17). The output
// goes to oracle/_ref/libttref.so. It is used to pin the C restatement in
// tt_oracle.c bit for bit, to write the golden fixtures under tests/golden/,
// and as the CPU baseline that bench.py times.
//
// Only the two entry points ttref_engine_ingest / ttref_engine_feedback restate
// reference code: they are the ring-ingest block (cache_engine.cpp:405-431) and
// the score-feedback block (:511-540) of TriTierCacheEngine::step written out
// separately, so a run can inject mean weights between them. They are compiled
// with the reference's flags, so `decay * g + w` contracts exactly as there.
#include "cache_engine.h"
#include "fused_attn_avx2.h"
#include "quantize_k_avx2.h"
#include "quantize_v_avx2.h"
#include "dequant_avx2.h"

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

extern "C" {

void ttref_quantize_k_block(const float* K, uint32_t* packed, void* scale, void* zero, int H, int D,
                            int kgs, int fp16) {
    if (fp16)
        quantize_k_block_avx2(K, packed, (uint16_t*)scale, (uint16_t*)zero, H, D, kgs);
    else
        quantize_k_block_avx2(K, packed, (float*)scale, (float*)zero, H, D, kgs);
}

void ttref_quantize_v_block(const float* V, int32_t* packed, void* scale, void* zero, int H, int D,
                            int chunk, int fp16) {
    if (fp16)
        quantize_v_block_avx2(V, packed, (uint16_t*)scale, (uint16_t*)zero, H, D, chunk);
    else
        quantize_v_block_avx2(V, packed, (float*)scale, (float*)zero, H, D, chunk);
}

void ttref_dequantize_k(const int32_t* packed, const void* scale, const void* zero, float* out, int nb,
                        int H, int D, int kgs, int fp16) {
    if (fp16)
        dequantize_k_avx2(packed, (const uint16_t*)scale, (const uint16_t*)zero, out, nb, H, D, kgs);
    else
        dequantize_k_avx2(packed, (const float*)scale, (const float*)zero, out, nb, H, D, kgs);
}

void ttref_dequantize_v(const int32_t* packed, const void* scale, const void* zero, float* out, int nt,
                        int H, int D, int fp16) {
    if (fp16)
        dequantize_v_avx2(packed, (const uint16_t*)scale, (const uint16_t*)zero, out, nt, H, D);
    else
        dequantize_v_avx2(packed, (const float*)scale, (const float*)zero, out, nt, H, D);
}

void ttref_fused_attention_decode(const float* Q, const float* dK, const float* dV, int dense_count,
                                  const int32_t* KP, const void* KS, const void* KZ, const int32_t* VP,
                                  const void* VS, const void* VZ, const int64_t* ids, int nb, int Hq,
                                  int Hkv, int D, float* out, float* mw, int kgs, int fp16) {
    if (fp16)
        fused_attention_decode_avx2(Q, dK, dV, dense_count, KP, (const uint16_t*)KS, (const uint16_t*)KZ, VP,
                                    (const uint16_t*)VS, (const uint16_t*)VZ, ids, nb, Hq, Hkv, D, out, mw,
                                    kgs);
    else
        fused_attention_decode_avx2(Q, dK, dV, dense_count, KP, (const float*)KS, (const float*)KZ, VP,
                                    (const float*)VS, (const float*)VZ, ids, nb, Hq, Hkv, D, out, mw, kgs);
}

void* ttref_engine_create(int Hq, int Hkv, int D, int max_seq_len, int sink, int rw, float h_ratio,
                          float decay, int update_interval, int kgs, int fp16) {
    return new TriTierCacheEngine(Hq, Hkv, D, max_seq_len, sink, rw, h_ratio, decay, update_interval, kgs,
                                  fp16 ? "fp16" : "fp32");
}

void ttref_engine_destroy(void* e) { delete (TriTierCacheEngine*)e; }

void ttref_engine_step(void* ev, const float* Q, const float* K, const float* V, float* out) {
    ((TriTierCacheEngine*)ev)->step(Q, K, V, out);
}

void ttref_engine_prefill(void* ev, const float* K, const float* V, int q_len) {
    ((TriTierCacheEngine*)ev)->prefill(K, V, q_len);
}

void ttref_engine_ingest(void* ev, const float* K_new, const float* V_new) {
    TriTierCacheEngine& e = *(TriTierCacheEngine*)ev;
    size_t kv_stride = static_cast<size_t>(e.num_kv_heads) * e.head_dim;
    if (e.s_count < e.sink_size) {
        std::memcpy(e.S_K.data() + static_cast<size_t>(e.s_count) * kv_stride, K_new, kv_stride * sizeof(float));
        std::memcpy(e.S_V.data() + static_cast<size_t>(e.s_count) * kv_stride, V_new, kv_stride * sizeof(float));
        e.s_count++;
    } else if (e.rw_count < e.rw_size) {
        std::memcpy(e.RW_K.data() + static_cast<size_t>(e.rw_count) * kv_stride, K_new, kv_stride * sizeof(float));
        std::memcpy(e.RW_V.data() + static_cast<size_t>(e.rw_count) * kv_stride, V_new, kv_stride * sizeof(float));
        e.rw_count++;
    } else {
        int slot = e.rw_head_index;
        int64_t evicted_id = static_cast<int64_t>(e.total_processed_tokens) - e.rw_size;
        std::vector<float> ek(kv_stride), evv(kv_stride);
        std::memcpy(ek.data(), e.RW_K.data() + static_cast<size_t>(slot) * kv_stride, kv_stride * sizeof(float));
        std::memcpy(evv.data(), e.RW_V.data() + static_cast<size_t>(slot) * kv_stride, kv_stride * sizeof(float));
        std::memcpy(e.RW_K.data() + static_cast<size_t>(slot) * kv_stride, K_new, kv_stride * sizeof(float));
        std::memcpy(e.RW_V.data() + static_cast<size_t>(slot) * kv_stride, V_new, kv_stride * sizeof(float));
        e.rw_head_index = (e.rw_head_index + 1) % e.rw_size;
        e.route_evicted_token(ek.data(), evv.data(), evicted_id);
    }
    e.total_processed_tokens++;
}

void ttref_engine_feedback(void* ev, const float* mean_attn_weights) {
    TriTierCacheEngine& e = *(TriTierCacheEngine*)ev;
    int dense_count = e.s_count + e.hh_count + e.rw_count;
    for (int i = 0; i < e.s_count; ++i)
        if (i < e.max_seq_len)
            e.global_attn_scores[i] = e.score_decay * e.global_attn_scores[i] + mean_attn_weights[i];
    for (int i = 0; i < e.hh_count; ++i) {
        int64_t tid = e.HH_token_ids[i];
        if (tid >= 0 && tid < e.max_seq_len) {
            e.global_attn_scores[tid] = e.score_decay * e.global_attn_scores[tid] + mean_attn_weights[e.s_count + i];
            e.HH_scores[i] = e.global_attn_scores[tid];
        }
    }
    int rw_base_id = e.total_processed_tokens - e.rw_count;
    for (int i = 0; i < e.rw_count; ++i) {
        int tid = rw_base_id + i;
        if (tid >= 0 && tid < e.max_seq_len)
            e.global_attn_scores[tid] =
                e.score_decay * e.global_attn_scores[tid] + mean_attn_weights[e.s_count + e.hh_count + i];
    }
    for (int i = 0; i < e.pbs_blocks_used * e.chunk_size; ++i) {
        int64_t tid = e.PBS_token_ids[i];
        if (tid >= 0 && tid < e.max_seq_len)
            e.global_attn_scores[tid] = e.score_decay * e.global_attn_scores[tid] + mean_attn_weights[dense_count + i];
    }
}

int ttref_engine_visible(void* ev) {
    TriTierCacheEngine& e = *(TriTierCacheEngine*)ev;
    return e.s_count + e.hh_count + e.rw_count + e.pbs_blocks_used * e.chunk_size;
}

size_t ttref_engine_buffer_bytes(void* ev) { return ((TriTierCacheEngine*)ev)->get_buffer_bytes(); }

float ttref_engine_cached_threshold(void* ev) { return ((TriTierCacheEngine*)ev)->cached_threshold; }

// Same 23 counters, same order, as orc_engine_counters in tt_oracle.h.
void ttref_engine_counters(void* ev, int64_t* o) {
    TriTierCacheEngine& e = *(TriTierCacheEngine*)ev;
    int64_t v[23] = {e.num_q_heads, e.num_kv_heads, e.head_dim, e.max_seq_len, e.sink_size, e.rw_size,
                     e.update_interval, e.k_group_size, e.chunk_size, e.quant_head_dim, e.max_hh,
                     e.use_fp16_meta ? 1 : 0, e.s_count, e.rw_count, e.rw_head_index, e.hh_count, e.wr_count,
                     e.pbs_allocated_blocks, e.pbs_blocks_used, e.pbs_count, e.total_processed_tokens,
                     e.last_calc_pos, e.total_evictions};
    std::memcpy(o, v, sizeof(v));
}

// Same buffer numbering as orc_engine_buffer in tt_oracle.h.
void* ttref_engine_buffer(void* ev, int which, int64_t* numel, int* es) {
    TriTierCacheEngine& e = *(TriTierCacheEngine*)ev;
    bool f16 = e.use_fp16_meta;
    switch (which) {
    case 0: *numel = e.S_K.size(); *es = 4; return e.S_K.data();
    case 1: *numel = e.S_V.size(); *es = 4; return e.S_V.data();
    case 2: *numel = e.RW_K.size(); *es = 4; return e.RW_K.data();
    case 3: *numel = e.RW_V.size(); *es = 4; return e.RW_V.data();
    case 4: *numel = e.HH_K.size(); *es = 4; return e.HH_K.data();
    case 5: *numel = e.HH_V.size(); *es = 4; return e.HH_V.data();
    case 6: *numel = e.HH_token_ids.size(); *es = 8; return e.HH_token_ids.data();
    case 7: *numel = e.HH_scores.size(); *es = 4; return e.HH_scores.data();
    case 8: *numel = e.WR_K.size(); *es = 4; return e.WR_K.data();
    case 9: *numel = e.WR_V.size(); *es = 4; return e.WR_V.data();
    case 10: *numel = e.WR_token_ids.size(); *es = 8; return e.WR_token_ids.data();
    case 11: *numel = e.PBS_K_Packed.size(); *es = 4; return e.PBS_K_Packed.data();
    case 12:
        *numel = f16 ? e.PBS_K_Scales_fp16.size() : e.PBS_K_Scales_fp32.size(); *es = f16 ? 2 : 4;
        return f16 ? (void*)e.PBS_K_Scales_fp16.data() : (void*)e.PBS_K_Scales_fp32.data();
    case 13:
        *numel = f16 ? e.PBS_K_Zeroes_fp16.size() : e.PBS_K_Zeroes_fp32.size(); *es = f16 ? 2 : 4;
        return f16 ? (void*)e.PBS_K_Zeroes_fp16.data() : (void*)e.PBS_K_Zeroes_fp32.data();
    case 14: *numel = e.PBS_V_Packed.size(); *es = 4; return e.PBS_V_Packed.data();
    case 15:
        *numel = f16 ? e.PBS_V_Scales_fp16.size() : e.PBS_V_Scales_fp32.size(); *es = f16 ? 2 : 4;
        return f16 ? (void*)e.PBS_V_Scales_fp16.data() : (void*)e.PBS_V_Scales_fp32.data();
    case 16:
        *numel = f16 ? e.PBS_V_Zeroes_fp16.size() : e.PBS_V_Zeroes_fp32.size(); *es = f16 ? 2 : 4;
        return f16 ? (void*)e.PBS_V_Zeroes_fp16.data() : (void*)e.PBS_V_Zeroes_fp32.data();
    case 17: *numel = e.PBS_token_ids.size(); *es = 8; return e.PBS_token_ids.data();
    case 18: *numel = e.global_attn_scores.size(); *es = 4; return e.global_attn_scores.data();
    default: *numel = 0; *es = 0; return nullptr;
    }
}

}  // extern "C"
