/*
 * tt_oracle.c -- CPU restatement of TriTierCache's fused decode step.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle, never the product). See tt_oracle.h
 * for which callers may load it and how each function is pinned.
 *
 * Build: oracle/Makefile, gcc -std=c11 -O2 -ffp-contract=off. The reference's
 * compiled AVX2 code fuses exactly where it uses _mm256_fmadd_ps or where GCC's
 * default -ffp-contract=fast contracts a scalar a*b+c; both are written here as
 * explicit fmaf() and nothing else is fused.
 */
#include "tt_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <limits.h>

/* ------------------------------------------------------------------------- */
/* Scalar models of the x86 vector primitives the reference uses.            */
/* ------------------------------------------------------------------------- */

/* MINPS/MAXPS (vminps/vmaxps): dest = (a < b) ? a : b, i.e. the second
 * operand is returned on equality (+0/-0) and on NaN. */
static inline float minps(float a, float b) { return (a < b) ? a : b; }
static inline float maxps(float a, float b) { return (a > b) ? a : b; }
/* std::min(a,b) = (b < a) ? b : a ; std::max(a,b) = (a < b) ? b : a */
static inline float std_min(float a, float b) { return (b < a) ? b : a; }
static inline float std_max(float a, float b) { return (a < b) ? b : a; }

/* vcvtps2dq under the default MXCSR (round to nearest even); NaN and
 * out-of-range inputs give the "integer indefinite" 0x80000000. */
static inline int32_t cvtps2dq(float x) {
    if (!(x >= -2147483648.0f && x < 2147483648.0f)) return INT32_MIN;
    return (int32_t)nearbyintf(x);
}

uint16_t orc_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t mant = u & 0x7fffffu;
    if (exp == 0xffu) {
        if (mant == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7c00u | 0x200u | (mant >> 13));
    }
    if (exp == 0) return (uint16_t)sign; /* fp32 denormals are far below half range */
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* half denormal: m = round(|x| * 2^24) */
        uint32_t full = mant | 0x800000u;
        int shift = 126 - (int)exp; /* >= 14 */
        if (shift > 24) return (uint16_t)sign;
        uint32_t m = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (m & 1u))) m++;
        return (uint16_t)(sign | m);
    }
    uint32_t m = mant >> 13, rem = mant & 0x1fffu;
    uint32_t h = sign | ((uint32_t)e << 10) | m;
    if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    uint32_t u;
    if (exp == 0) {
        if (mant == 0) {
            u = sign;
        } else {
            int e = -1;
            do { mant <<= 1; e++; } while (!(mant & 0x400u));
            mant &= 0x3ffu;
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 0x1fu) {
        u = sign | 0x7f800000u | (mant << 13);
    } else {
        u = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline void store_meta(void* base, size_t idx, float v, int fp16) {
    if (fp16) ((uint16_t*)base)[idx] = orc_f32_to_f16(v);
    else ((float*)base)[idx] = v;
}
static inline float load_meta(const void* base, size_t idx, int fp16) {
    return fp16 ? orc_f16_to_f32(((const uint16_t*)base)[idx]) : ((const float*)base)[idx];
}

/* ------------------------------------------------------------------------- */
/* Quantisers                                                                */
/* ------------------------------------------------------------------------- */

/* quantize_k_avx2.cpp:26-110. Per (head, channel): min/max over the block's
 * k_group_size tokens, scale = max((max-min)/3, 1e-9), q = clamp(rne((x-min)/scale),0,3),
 * token t = 16w + sub_t stored at bits 2*sub_t of word w (:65-77). The 8-wide
 * vector body covers channels [0, 8*floor(D/8)); the scalar tail (:84-108)
 * differs only in its min/max operand order (NaN / signed-zero behaviour). */
void orc_quantize_k_block(const float* K, uint32_t* packed, void* scale_out, void* zero_out,
                          int num_heads, int head_dim, int k_group_size, int meta_fp16) {
    const int row_stride = num_heads * head_dim;
    const int c_vec_end = (head_dim / 8) * 8;
    const int num_words = k_group_size / 16;
    for (int h = 0; h < num_heads; ++h) {
        const float* hb = K + (size_t)h * head_dim;
        for (int c = 0; c < head_dim; ++c) {
            const int vec = c < c_vec_end;
            float mn = INFINITY, mx = -INFINITY;
            for (int t = 0; t < k_group_size; ++t) {
                float x = hb[(size_t)t * row_stride + c];
                if (vec) { mn = minps(mn, x); mx = maxps(mx, x); }
                else { mn = std_min(mn, x); mx = std_max(mx, x); }
            }
            float d3 = (mx - mn) / 3.0f;
            float scale = vec ? maxps(d3, 1e-9f) : std_max(d3, 1e-9f);
            store_meta(scale_out, (size_t)h * head_dim + c, scale, meta_fp16);
            store_meta(zero_out, (size_t)h * head_dim + c, mn, meta_fp16);
            for (int w = 0; w < num_words; ++w) {
                uint32_t bits = 0;
                for (int sub_t = 0; sub_t < 16; ++sub_t) {
                    int t = w * 16 + sub_t;
                    float x = hb[(size_t)t * row_stride + c];
                    float norm = (x - mn) / scale;
                    int32_t q = cvtps2dq(norm);
                    if (vec) { q = q > 0 ? q : 0; q = q < 3 ? q : 3; }
                    else { q = q < 3 ? q : 3; q = q > 0 ? q : 0; }
                    bits |= ((uint32_t)q) << (2 * sub_t);
                }
                packed[((size_t)w * num_heads + h) * head_dim + c] = bits;
            }
        }
    }
}

/* hmin8/hmax8 reduction trees (quantize_v_avx2.cpp:7-23): lanes (i, i+4), then
 * (i, i+2), then (0, 1), each with MINPS/MAXPS operand order. */
static float hmin8(const float* x) {
    float m0 = minps(x[0], x[4]), m1 = minps(x[1], x[5]), m2 = minps(x[2], x[6]), m3 = minps(x[3], x[7]);
    float n0 = minps(m0, m2), n1 = minps(m1, m3);
    return minps(n0, n1);
}
static float hmax8(const float* x) {
    float m0 = maxps(x[0], x[4]), m1 = maxps(x[1], x[5]), m2 = maxps(x[2], x[6]), m3 = maxps(x[3], x[7]);
    float n0 = maxps(m0, m2), n1 = maxps(m1, m3);
    return maxps(n0, n1);
}

/* quantize_v_avx2.cpp:44-108. Per (token, head): min/max over D channels,
 * same scale formula, channel 16g+i stored at bits 2i of word g. */
void orc_quantize_v_block(const float* V, int32_t* packed, void* scale_out, void* zero_out,
                          int num_heads, int head_dim, int chunk_size, int meta_fp16) {
    const int qhd = (head_dim + 15) / 16;
    const int row_stride = num_heads * head_dim;
    for (int t = 0; t < chunk_size; ++t) {
        for (int h = 0; h < num_heads; ++h) {
            const float* v = V + (size_t)t * row_stride + (size_t)h * head_dim;
            float mn = INFINITY, mx = -INFINITY;
            int c = 0;
            for (; c + 8 <= head_dim; c += 8) {
                mn = std_min(mn, hmin8(v + c));
                mx = std_max(mx, hmax8(v + c));
            }
            for (; c < head_dim; ++c) {
                mn = std_min(mn, v[c]);
                mx = std_max(mx, v[c]);
            }
            float scale = std_max((mx - mn) / 3.0f, 1e-9f);
            store_meta(scale_out, (size_t)t * num_heads + h, scale, meta_fp16);
            store_meta(zero_out, (size_t)t * num_heads + h, mn, meta_fp16);
            for (int g = 0; g < qhd; ++g) {
                uint32_t bits = 0;
                for (int i = 0; i < 16; ++i) {
                    float x = v[g * 16 + i];
                    int32_t q = cvtps2dq((x - mn) / scale);
                    q = q < 3 ? q : 3;
                    q = q > 0 ? q : 0;
                    bits |= ((uint32_t)q) << (2 * i);
                }
                packed[((size_t)t * num_heads + h) * qhd + g] = (int32_t)bits;
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Dequantisers: x = fmaf((float)q, scale, zero)                             */
/* ------------------------------------------------------------------------- */

/* dequantize_avx2.cpp:24-110 */
void orc_dequantize_k(const int32_t* packed, const void* scale, const void* zero, float* out,
                      int num_blocks, int num_heads, int head_dim, int k_group_size, int meta_fp16) {
    const int wpb = k_group_size / 16;
    const size_t bps = (size_t)wpb * num_heads * head_dim;
    const size_t bms = (size_t)num_heads * head_dim;
    const size_t ors = (size_t)num_heads * head_dim;
    for (int b = 0; b < num_blocks; ++b)
        for (int h = 0; h < num_heads; ++h)
            for (int c = 0; c < head_dim; ++c) {
                float s = load_meta(scale, b * bms + (size_t)h * head_dim + c, meta_fp16);
                float z = load_meta(zero, b * bms + (size_t)h * head_dim + c, meta_fp16);
                for (int w = 0; w < wpb; ++w) {
                    uint32_t p = (uint32_t)packed[b * bps + ((size_t)w * num_heads + h) * head_dim + c];
                    for (int sub_t = 0; sub_t < 16; ++sub_t) {
                        int q = (int)((p >> (2 * sub_t)) & 3u);
                        size_t tok = (size_t)b * k_group_size + w * 16 + sub_t;
                        out[tok * ors + (size_t)h * head_dim + c] = fmaf((float)q, s, z);
                    }
                }
            }
}

/* dequantize_avx2.cpp:138-204 */
void orc_dequantize_v(const int32_t* packed, const void* scale, const void* zero, float* out,
                      int total_tokens, int num_heads, int head_dim, int meta_fp16) {
    const int qhd = (head_dim + 15) / 16;
    for (int tok = 0; tok < total_tokens; ++tok)
        for (int h = 0; h < num_heads; ++h) {
            float s = load_meta(scale, (size_t)tok * num_heads + h, meta_fp16);
            float z = load_meta(zero, (size_t)tok * num_heads + h, meta_fp16);
            const int32_t* hp = packed + ((size_t)tok * num_heads + h) * qhd;
            float* o = out + (size_t)tok * num_heads * head_dim + (size_t)h * head_dim;
            for (int g = 0; g < qhd; ++g) {
                uint32_t p = (uint32_t)hp[g];
                for (int i = 0; i < 16; ++i) o[g * 16 + i] = fmaf((float)((p >> (2 * i)) & 3u), s, z);
            }
        }
}

/* ------------------------------------------------------------------------- */
/* Fused decode attention (faithful: dequantise-all, two-pass softmax)       */
/* ------------------------------------------------------------------------- */

/* dot_avx2 (fused_attn_avx2.cpp:21-61): eight 8-lane FMA accumulators over
 * 64-element chunks, then 32-element chunks on the first four, then 8-element
 * chunks on the first, a pairwise tree and hsum8 (:11-18). */
static float dot_ref(const float* a, const float* b, int n) {
    float acc[8][8];
    memset(acc, 0, sizeof(acc));
    int i = 0;
    for (; i + 64 <= n; i += 64)
        for (int j = 0; j < 8; ++j)
            for (int l = 0; l < 8; ++l) acc[j][l] = fmaf(a[i + 8 * j + l], b[i + 8 * j + l], acc[j][l]);
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l) acc[j][l] = fmaf(a[i + 8 * j + l], b[i + 8 * j + l], acc[j][l]);
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
    float r0[8], r2[8], r4[8], r6[8];
    for (int l = 0; l < 8; ++l) {
        r0[l] = acc[0][l] + acc[1][l];
        r2[l] = acc[2][l] + acc[3][l];
        r4[l] = acc[4][l] + acc[5][l];
        r6[l] = acc[6][l] + acc[7][l];
    }
    for (int l = 0; l < 8; ++l) { r0[l] = r0[l] + r2[l]; r4[l] = r4[l] + r6[l]; }
    for (int l = 0; l < 8; ++l) r0[l] = r0[l] + r4[l];
    float s0 = r0[0] + r0[4], s1 = r0[1] + r0[5], s2 = r0[2] + r0[6], s3 = r0[3] + r0[7];
    float t0 = s0 + s2, t1 = s1 + s3;
    float sum = t0 + t1;
    for (; i < n; ++i) sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* axpy_avx2 (:64-136): out += scale * x, one fused rounding per element. */
static void axpy_ref(float* out, const float* x, float scale, int n) {
    for (int i = 0; i < n; ++i) out[i] = fmaf(x[i], scale, out[i]);
}

void orc_fused_attention_decode(const float* Q, const float* dense_K, const float* dense_V,
                                int dense_count, const int32_t* PBS_K_Packed,
                                const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                                const int32_t* PBS_V_Packed, const void* PBS_V_Scales,
                                const void* PBS_V_Zeroes, const int64_t* PBS_token_ids,
                                int num_blocks, int num_q_heads, int num_kv_heads, int head_dim,
                                float* attn_output, float* mean_attn_weights, int k_group_size,
                                int meta_fp16) {
    const float inv_sqrt_hd = 1.0f / sqrtf((float)head_dim);
    const int total_pbs = num_blocks * k_group_size;
    const int total_tokens = dense_count + total_pbs;
    const int gqa = (num_kv_heads > 0) ? (num_q_heads / num_kv_heads) : 1;
    const int wpb = k_group_size / 16;
    const int qhd = (head_dim + 15) / 16;
    const size_t kvs = (size_t)num_kv_heads * head_dim;

    float* scores = (float*)malloc(sizeof(float) * ((size_t)num_q_heads * total_tokens + 1));
    float* kdq = NULL;
    float* vdq = NULL;
    if (num_blocks > 0) {
        kdq = (float*)malloc(sizeof(float) * (size_t)total_pbs * kvs);
        vdq = (float*)malloc(sizeof(float) * (size_t)total_pbs * kvs);
        const size_t msz = meta_fp16 ? 2 : 4;
        for (int b = 0; b < num_blocks; ++b) {
            orc_dequantize_k(PBS_K_Packed + (size_t)b * wpb * kvs,
                             (const char*)PBS_K_Scales + (size_t)b * kvs * msz,
                             (const char*)PBS_K_Zeroes + (size_t)b * kvs * msz,
                             kdq + (size_t)b * k_group_size * kvs, 1, num_kv_heads, head_dim,
                             k_group_size, meta_fp16);
            orc_dequantize_v(PBS_V_Packed + (size_t)b * k_group_size * num_kv_heads * qhd,
                             (const char*)PBS_V_Scales + (size_t)b * k_group_size * num_kv_heads * msz,
                             (const char*)PBS_V_Zeroes + (size_t)b * k_group_size * num_kv_heads * msz,
                             vdq + (size_t)b * k_group_size * kvs, k_group_size, num_kv_heads,
                             head_dim, meta_fp16);
        }
    }
    float* row_max = (float*)malloc(sizeof(float) * (size_t)(num_q_heads > 0 ? num_q_heads : 1));
    float* row_sum = (float*)malloc(sizeof(float) * (size_t)(num_q_heads > 0 ? num_q_heads : 1));

    for (int h = 0; h < num_q_heads; ++h) {
        const int kv_h = (gqa > 1) ? (h / gqa) : h;
        const float* q = Q + (size_t)h * head_dim;
        float* hs = scores + (size_t)h * total_tokens;
        for (int i = 0; i < dense_count; ++i)
            hs[i] = dot_ref(q, dense_K + ((size_t)i * num_kv_heads + kv_h) * head_dim, head_dim) * inv_sqrt_hd;
        for (int b = 0; b < num_blocks; ++b)
            for (int t = 0; t < k_group_size; ++t) {
                int gi = dense_count + b * k_group_size + t;
                if (PBS_token_ids[b * k_group_size + t] == -1) hs[gi] = -INFINITY;
                else hs[gi] = dot_ref(q, kdq + ((size_t)(b * k_group_size + t) * num_kv_heads + kv_h) * head_dim,
                                      head_dim) * inv_sqrt_hd;
            }
        float mx = -INFINITY;
        for (int i = 0; i < total_tokens; ++i) mx = std_max(mx, hs[i]);
        row_max[h] = mx;
        float sum_exp = 0.0f;
        for (int i = 0; i < total_tokens; ++i)
            if (hs[i] != -INFINITY) sum_exp += expf(hs[i] - mx);
        float inv_sum = sum_exp > 0.0f ? (1.0f / sum_exp) : 1.0f;
        row_sum[h] = sum_exp > 0.0f ? sum_exp : 1.0f;
        float* out_h = attn_output + (size_t)h * head_dim;
        for (int c = 0; c < head_dim; ++c) out_h[c] = 0.0f;
        for (int i = 0; i < dense_count; ++i) {
            float w = expf(hs[i] - mx) * inv_sum;
            axpy_ref(out_h, dense_V + ((size_t)i * num_kv_heads + kv_h) * head_dim, w, head_dim);
        }
        for (int b = 0; b < num_blocks; ++b)
            for (int t = 0; t < k_group_size; ++t) {
                if (PBS_token_ids[b * k_group_size + t] == -1) continue;
                int gi = dense_count + b * k_group_size + t;
                float w = expf(hs[gi] - mx) * inv_sum;
                axpy_ref(out_h, vdq + ((size_t)(b * k_group_size + t) * num_kv_heads + kv_h) * head_dim, w,
                         head_dim);
            }
    }
    if (mean_attn_weights) {
        for (int i = 0; i < total_tokens; ++i) {
            float sum_w = 0.0f;
            for (int h = 0; h < num_q_heads; ++h) {
                float sc = scores[(size_t)h * total_tokens + i];
                if (sc != -INFINITY) sum_w += expf(sc - row_max[h]) / row_sum[h];
            }
            mean_attn_weights[i] = sum_w / (float)num_q_heads;
        }
    }
    free(scores);
    free(kdq);
    free(vdq);
    free(row_max);
    free(row_sum);
}

/* ------------------------------------------------------------------------- */
/* Engine (cache_engine.h / cache_engine.cpp)                                */
/* ------------------------------------------------------------------------- */

struct orc_engine {
    int num_q_heads, num_kv_heads, head_dim, max_seq_len, sink_size, rw_size;
    float h_ratio, score_decay;
    int update_interval, k_group_size, use_fp16_meta, chunk_size, quant_head_dim, max_hh;
    int s_count, rw_count, rw_head_index, hh_count, wr_count;
    int pbs_allocated_blocks, pbs_blocks_used, pbs_count;
    int total_processed_tokens, last_calc_pos, total_evictions;
    float cached_threshold;
    float *S_K, *S_V, *RW_K, *RW_V, *HH_K, *HH_V, *HH_scores, *WR_K, *WR_V;
    int64_t *HH_token_ids, *WR_token_ids, *PBS_token_ids;
    int32_t *PBS_K_Packed, *PBS_V_Packed;
    void *PBS_K_Scales, *PBS_K_Zeroes, *PBS_V_Scales, *PBS_V_Zeroes;
    float* global_attn_scores;
    float *dense_K, *dense_V, *mean_attn_weights;
    size_t mw_cap;
};

static void* zalloc(size_t n) { return calloc(n ? n : 1, 1); }

/* cache_engine.cpp:8-82 */
orc_engine* orc_engine_create(int num_q_heads, int num_kv_heads, int head_dim, int max_seq_len,
                              int sink_size, int rw_size, float h_ratio, float score_decay,
                              int update_interval, int k_group_size, int meta_fp16) {
    orc_engine* e = (orc_engine*)zalloc(sizeof(orc_engine));
    e->num_q_heads = num_q_heads;
    e->num_kv_heads = num_kv_heads;
    e->head_dim = head_dim;
    e->max_seq_len = max_seq_len;
    e->sink_size = sink_size;
    e->rw_size = rw_size;
    e->h_ratio = h_ratio;
    e->score_decay = score_decay;
    e->update_interval = update_interval;
    e->k_group_size = (k_group_size == 32) ? 32 : 16;
    e->use_fp16_meta = meta_fp16 ? 1 : 0;
    e->chunk_size = e->k_group_size;
    e->quant_head_dim = (head_dim + 15) / 16;
    e->max_hh = (int)ceilf((float)max_seq_len * h_ratio);
    if (e->max_hh < 1) e->max_hh = 1;
    e->last_calc_pos = -1;
    e->cached_threshold = 0.0f;
    size_t kvs = (size_t)num_kv_heads * head_dim;
    e->S_K = (float*)zalloc(sizeof(float) * sink_size * kvs);
    e->S_V = (float*)zalloc(sizeof(float) * sink_size * kvs);
    e->RW_K = (float*)zalloc(sizeof(float) * rw_size * kvs);
    e->RW_V = (float*)zalloc(sizeof(float) * rw_size * kvs);
    e->HH_K = (float*)zalloc(sizeof(float) * e->max_hh * kvs);
    e->HH_V = (float*)zalloc(sizeof(float) * e->max_hh * kvs);
    e->HH_token_ids = (int64_t*)zalloc(sizeof(int64_t) * e->max_hh);
    for (int i = 0; i < e->max_hh; ++i) e->HH_token_ids[i] = -1;
    e->HH_scores = (float*)zalloc(sizeof(float) * e->max_hh);
    e->WR_K = (float*)zalloc(sizeof(float) * e->chunk_size * kvs);
    e->WR_V = (float*)zalloc(sizeof(float) * e->chunk_size * kvs);
    e->WR_token_ids = (int64_t*)zalloc(sizeof(int64_t) * e->chunk_size);
    for (int i = 0; i < e->chunk_size; ++i) e->WR_token_ids[i] = -1;
    e->global_attn_scores = (float*)zalloc(sizeof(float) * (size_t)max_seq_len);
    size_t max_dense = (size_t)(sink_size + e->max_hh + rw_size);
    e->dense_K = (float*)zalloc(sizeof(float) * max_dense * kvs);
    e->dense_V = (float*)zalloc(sizeof(float) * max_dense * kvs);
    e->mw_cap = max_dense + 1024;
    e->mean_attn_weights = (float*)zalloc(sizeof(float) * e->mw_cap);
    return e;
}

void orc_engine_destroy(orc_engine* e) {
    if (!e) return;
    free(e->S_K); free(e->S_V); free(e->RW_K); free(e->RW_V); free(e->HH_K); free(e->HH_V);
    free(e->HH_token_ids); free(e->HH_scores); free(e->WR_K); free(e->WR_V); free(e->WR_token_ids);
    free(e->PBS_K_Packed); free(e->PBS_V_Packed); free(e->PBS_K_Scales); free(e->PBS_K_Zeroes);
    free(e->PBS_V_Scales); free(e->PBS_V_Zeroes); free(e->PBS_token_ids);
    free(e->global_attn_scores); free(e->dense_K); free(e->dense_V); free(e->mean_attn_weights);
    free(e);
}

static void* grow(void* p, size_t old_bytes, size_t new_bytes) {
    void* n = zalloc(new_bytes);
    if (p) memcpy(n, p, old_bytes);
    free(p);
    return n;
}

/* cache_engine.cpp:84-116: grow in chunks of 64 blocks, new token ids = -1. */
static void ensure_pbs_capacity(orc_engine* e, int min_blocks) {
    if (min_blocks <= e->pbs_allocated_blocks) return;
    int nb = e->pbs_allocated_blocks + 64;
    if (nb < min_blocks) nb = min_blocks;
    int ob = e->pbs_allocated_blocks;
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    size_t wpb = (size_t)(e->k_group_size / 16);
    size_t msz = e->use_fp16_meta ? 2 : 4;
    size_t ch = (size_t)e->chunk_size;
    size_t vps = (size_t)e->num_kv_heads * e->quant_head_dim;
    e->PBS_K_Packed = (int32_t*)grow(e->PBS_K_Packed, ob * wpb * kvs * 4, nb * wpb * kvs * 4);
    e->PBS_K_Scales = grow(e->PBS_K_Scales, ob * kvs * msz, nb * kvs * msz);
    e->PBS_K_Zeroes = grow(e->PBS_K_Zeroes, ob * kvs * msz, nb * kvs * msz);
    e->PBS_V_Scales = grow(e->PBS_V_Scales, ob * ch * e->num_kv_heads * msz, nb * ch * e->num_kv_heads * msz);
    e->PBS_V_Zeroes = grow(e->PBS_V_Zeroes, ob * ch * e->num_kv_heads * msz, nb * ch * e->num_kv_heads * msz);
    e->PBS_V_Packed = (int32_t*)grow(e->PBS_V_Packed, ob * ch * vps * 4, nb * ch * vps * 4);
    e->PBS_token_ids = (int64_t*)grow(e->PBS_token_ids, ob * ch * 8, nb * ch * 8);
    for (size_t i = ob * ch; i < nb * ch; ++i) e->PBS_token_ids[i] = -1;
    e->pbs_allocated_blocks = nb;
}

static int cmp_float(const void* a, const void* b) {
    float x = *(const float*)a, y = *(const float*)b;
    return (x < y) ? -1 : ((y < x) ? 1 : 0);
}

/* cache_engine.cpp:118-146. The k-th smallest candidate with
 * k = (size_t)(q * (float)(n-1)) computed in float32 (q = clamp(1-h_ratio)).
 * Where total - rw_size exceeds max_seq_len the reference reads past the end
 * of global_attn_scores (undefined behaviour); this restatement, like the HIP
 * engine, clamps the candidate range to the score array instead. */
static float fetch_or_calc_threshold(orc_engine* e) {
    int cs = e->sink_size;
    int ce = e->total_processed_tokens - e->rw_size;
    if (ce > e->max_seq_len) ce = e->max_seq_len;
    if (ce <= cs) {
        e->cached_threshold = 0.0f;
        return e->cached_threshold;
    }
    if (e->last_calc_pos == -1 || (e->total_processed_tokens - e->last_calc_pos >= e->update_interval)) {
        size_t n = (size_t)(ce - cs);
        float* v = (float*)malloc(sizeof(float) * n);
        for (size_t i = 0; i < n; ++i) v[i] = e->global_attn_scores[cs + i];
        float q = 1.0f - e->h_ratio;
        if (q < 0.0f) q = 0.0f;
        if (q > 1.0f) q = 1.0f;
        size_t k = (size_t)(q * (float)(n - 1));
        qsort(v, n, sizeof(float), cmp_float);
        e->cached_threshold = v[k];
        free(v);
        e->last_calc_pos = e->total_processed_tokens;
    }
    return e->cached_threshold;
}

/* cache_engine.cpp:148-207 */
static void flush_waiting_room(orc_engine* e) {
    ensure_pbs_capacity(e, e->pbs_blocks_used + 1);
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    size_t wpb = (size_t)(e->k_group_size / 16);
    size_t vps = (size_t)e->num_kv_heads * e->quant_head_dim;
    size_t msz = e->use_fp16_meta ? 2 : 4;
    size_t b = (size_t)e->pbs_blocks_used;
    size_t ch = (size_t)e->chunk_size;
    orc_quantize_k_block(e->WR_K, (uint32_t*)(e->PBS_K_Packed + b * wpb * kvs),
                         (char*)e->PBS_K_Scales + b * kvs * msz, (char*)e->PBS_K_Zeroes + b * kvs * msz,
                         e->num_kv_heads, e->head_dim, e->k_group_size, e->use_fp16_meta);
    orc_quantize_v_block(e->WR_V, e->PBS_V_Packed + b * ch * vps,
                         (char*)e->PBS_V_Scales + b * ch * e->num_kv_heads * msz,
                         (char*)e->PBS_V_Zeroes + b * ch * e->num_kv_heads * msz, e->num_kv_heads,
                         e->head_dim, e->chunk_size, e->use_fp16_meta);
    for (size_t t = 0; t < ch; ++t) e->PBS_token_ids[b * ch + t] = e->WR_token_ids[t];
    e->pbs_blocks_used++;
    e->pbs_count += e->chunk_size;
    e->wr_count = 0;
}

/* cache_engine.cpp:209-269 */
static void route_evicted_token(orc_engine* e, const float* k, const float* v, int64_t token_id) {
    e->total_evictions++;
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    size_t rb = kvs * sizeof(float);
    float score = (token_id >= 0 && token_id < (int64_t)e->max_seq_len) ? e->global_attn_scores[token_id] : 0.0f;
    float thresh = fetch_or_calc_threshold(e);
    if (score >= thresh) {
        if (e->hh_count < e->max_hh) {
            memcpy(e->HH_K + (size_t)e->hh_count * kvs, k, rb);
            memcpy(e->HH_V + (size_t)e->hh_count * kvs, v, rb);
            e->HH_token_ids[e->hh_count] = token_id;
            e->HH_scores[e->hh_count] = score;
            e->hh_count++;
            return;
        }
        int min_idx = 0;
        float min_score = e->HH_scores[0];
        for (int i = 1; i < e->hh_count; ++i)
            if (e->HH_scores[i] < min_score) { min_score = e->HH_scores[i]; min_idx = i; }
        if (score > min_score) {
            memcpy(e->WR_K + (size_t)e->wr_count * kvs, e->HH_K + (size_t)min_idx * kvs, rb);
            memcpy(e->WR_V + (size_t)e->wr_count * kvs, e->HH_V + (size_t)min_idx * kvs, rb);
            e->WR_token_ids[e->wr_count] = e->HH_token_ids[min_idx];
            e->wr_count++;
            memcpy(e->HH_K + (size_t)min_idx * kvs, k, rb);
            memcpy(e->HH_V + (size_t)min_idx * kvs, v, rb);
            e->HH_token_ids[min_idx] = token_id;
            e->HH_scores[min_idx] = score;
            if (e->wr_count == e->chunk_size) flush_waiting_room(e);
            return;
        }
    }
    memcpy(e->WR_K + (size_t)e->wr_count * kvs, k, rb);
    memcpy(e->WR_V + (size_t)e->wr_count * kvs, v, rb);
    e->WR_token_ids[e->wr_count] = token_id;
    e->wr_count++;
    if (e->wr_count == e->chunk_size) flush_waiting_room(e);
}

/* cache_engine.cpp:271-395 */
void orc_engine_prefill(orc_engine* e, const float* K_all, const float* V_all, int q_len) {
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    if (q_len <= e->sink_size + e->rw_size) {
        int s = e->sink_size < q_len ? e->sink_size : q_len;
        if (s > 0) {
            memcpy(e->S_K, K_all, (size_t)s * kvs * 4);
            memcpy(e->S_V, V_all, (size_t)s * kvs * 4);
            e->s_count = s;
        }
        int r = q_len - s;
        if (r > 0) {
            memcpy(e->RW_K, K_all + (size_t)s * kvs, (size_t)r * kvs * 4);
            memcpy(e->RW_V, V_all + (size_t)s * kvs, (size_t)r * kvs * 4);
            e->rw_count = r;
            e->rw_head_index = 0;
        }
        e->total_processed_tokens = q_len;
        return;
    }
    memcpy(e->S_K, K_all, (size_t)e->sink_size * kvs * 4);
    memcpy(e->S_V, V_all, (size_t)e->sink_size * kvs * 4);
    e->s_count = e->sink_size;
    int rw_start = q_len - e->rw_size;
    memcpy(e->RW_K, K_all + (size_t)rw_start * kvs, (size_t)e->rw_size * kvs * 4);
    memcpy(e->RW_V, V_all + (size_t)rw_start * kvs, (size_t)e->rw_size * kvs * 4);
    e->rw_count = e->rw_size;
    e->rw_head_index = 0;
    int n_inter = rw_start - e->sink_size;
    int nbq = n_inter / e->chunk_size;
    int rem = n_inter % e->chunk_size;
    if (nbq > 0) {
        ensure_pbs_capacity(e, e->pbs_blocks_used + nbq);
        size_t wpb = (size_t)(e->k_group_size / 16);
        size_t vps = (size_t)e->num_kv_heads * e->quant_head_dim;
        size_t msz = e->use_fp16_meta ? 2 : 4;
        size_t ch = (size_t)e->chunk_size;
        for (int b = 0; b < nbq; ++b) {
            size_t dst = (size_t)(e->pbs_blocks_used + b);
            int src = e->sink_size + b * e->chunk_size;
            orc_quantize_k_block(K_all + (size_t)src * kvs, (uint32_t*)(e->PBS_K_Packed + dst * wpb * kvs),
                                 (char*)e->PBS_K_Scales + dst * kvs * msz, (char*)e->PBS_K_Zeroes + dst * kvs * msz,
                                 e->num_kv_heads, e->head_dim, e->k_group_size, e->use_fp16_meta);
            orc_quantize_v_block(V_all + (size_t)src * kvs, e->PBS_V_Packed + dst * ch * vps,
                                 (char*)e->PBS_V_Scales + dst * ch * e->num_kv_heads * msz,
                                 (char*)e->PBS_V_Zeroes + dst * ch * e->num_kv_heads * msz, e->num_kv_heads,
                                 e->head_dim, e->chunk_size, e->use_fp16_meta);
            for (size_t t = 0; t < ch; ++t) e->PBS_token_ids[dst * ch + t] = src + (int64_t)t;
        }
        e->pbs_blocks_used += nbq;
        e->pbs_count += nbq * e->chunk_size;
        e->total_evictions += nbq * e->chunk_size;
    }
    if (rem > 0) {
        int rs = e->sink_size + nbq * e->chunk_size;
        memcpy(e->WR_K, K_all + (size_t)rs * kvs, (size_t)rem * kvs * 4);
        memcpy(e->WR_V, V_all + (size_t)rs * kvs, (size_t)rem * kvs * 4);
        for (int t = 0; t < rem; ++t) e->WR_token_ids[t] = rs + t;
        e->wr_count = rem;
    } else {
        e->wr_count = 0;
    }
    e->total_processed_tokens = q_len;
}

/* cache_engine.cpp:405-431 */
void orc_engine_ingest(orc_engine* e, const float* K_new, const float* V_new) {
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    size_t rb = kvs * sizeof(float);
    if (e->s_count < e->sink_size) {
        memcpy(e->S_K + (size_t)e->s_count * kvs, K_new, rb);
        memcpy(e->S_V + (size_t)e->s_count * kvs, V_new, rb);
        e->s_count++;
    } else if (e->rw_count < e->rw_size) {
        memcpy(e->RW_K + (size_t)e->rw_count * kvs, K_new, rb);
        memcpy(e->RW_V + (size_t)e->rw_count * kvs, V_new, rb);
        e->rw_count++;
    } else {
        int slot = e->rw_head_index;
        int64_t evicted_id = (int64_t)e->total_processed_tokens - e->rw_size;
        float* ek = (float*)malloc(rb);
        float* ev = (float*)malloc(rb);
        memcpy(ek, e->RW_K + (size_t)slot * kvs, rb);
        memcpy(ev, e->RW_V + (size_t)slot * kvs, rb);
        memcpy(e->RW_K + (size_t)slot * kvs, K_new, rb);
        memcpy(e->RW_V + (size_t)slot * kvs, V_new, rb);
        e->rw_head_index = (e->rw_head_index + 1) % e->rw_size;
        route_evicted_token(e, ek, ev, evicted_id);
        free(ek);
        free(ev);
    }
    e->total_processed_tokens++;
}

int orc_engine_visible(const orc_engine* e) {
    return e->s_count + e->hh_count + e->rw_count + e->pbs_blocks_used * e->chunk_size;
}

/* cache_engine.cpp:433-509: dense set = sinks, HH slots, RW oldest->newest;
 * then every used PBS block. The waiting room is not attended. */
void orc_engine_attend(orc_engine* e, const float* Q, float* attn_output, float* mean_weights) {
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    int dc = 0;
    if (e->s_count > 0) {
        memcpy(e->dense_K, e->S_K, (size_t)e->s_count * kvs * 4);
        memcpy(e->dense_V, e->S_V, (size_t)e->s_count * kvs * 4);
        dc += e->s_count;
    }
    if (e->hh_count > 0) {
        memcpy(e->dense_K + (size_t)dc * kvs, e->HH_K, (size_t)e->hh_count * kvs * 4);
        memcpy(e->dense_V + (size_t)dc * kvs, e->HH_V, (size_t)e->hh_count * kvs * 4);
        dc += e->hh_count;
    }
    for (int i = 0; i < e->rw_count; ++i) {
        int ri = (e->rw_head_index + i) % e->rw_size;
        memcpy(e->dense_K + (size_t)dc * kvs, e->RW_K + (size_t)ri * kvs, kvs * 4);
        memcpy(e->dense_V + (size_t)dc * kvs, e->RW_V + (size_t)ri * kvs, kvs * 4);
        dc++;
    }
    orc_fused_attention_decode(Q, e->dense_K, e->dense_V, dc, e->PBS_K_Packed, e->PBS_K_Scales,
                               e->PBS_K_Zeroes, e->PBS_V_Packed, e->PBS_V_Scales, e->PBS_V_Zeroes,
                               e->PBS_token_ids, e->pbs_blocks_used, e->num_q_heads, e->num_kv_heads,
                               e->head_dim, attn_output, mean_weights, e->k_group_size, e->use_fp16_meta);
}

/* cache_engine.cpp:511-540. The reference's `decay * g + w` is compiled to a
 * single FMA (GCC -O3 -mfma, default -ffp-contract=fast). */
void orc_engine_feedback(orc_engine* e, const float* mw) {
    const float d = e->score_decay;
    float* g = e->global_attn_scores;
    for (int i = 0; i < e->s_count; ++i)
        if (i < e->max_seq_len) g[i] = fmaf(d, g[i], mw[i]);
    for (int i = 0; i < e->hh_count; ++i) {
        int64_t tid = e->HH_token_ids[i];
        if (tid >= 0 && tid < e->max_seq_len) {
            g[tid] = fmaf(d, g[tid], mw[e->s_count + i]);
            e->HH_scores[i] = g[tid];
        }
    }
    int rw_base = e->total_processed_tokens - e->rw_count;
    for (int i = 0; i < e->rw_count; ++i) {
        int tid = rw_base + i;
        if (tid >= 0 && tid < e->max_seq_len) g[tid] = fmaf(d, g[tid], mw[e->s_count + e->hh_count + i]);
    }
    int dc = e->s_count + e->hh_count + e->rw_count;
    for (int i = 0; i < e->pbs_blocks_used * e->chunk_size; ++i) {
        int64_t tid = e->PBS_token_ids[i];
        if (tid >= 0 && tid < e->max_seq_len) g[tid] = fmaf(d, g[tid], mw[dc + i]);
    }
}

/* cache_engine.cpp:397-541 */
void orc_engine_step(orc_engine* e, const float* Q, const float* K_new, const float* V_new,
                     float* attn_output) {
    orc_engine_ingest(e, K_new, V_new);
    size_t need = (size_t)orc_engine_visible(e);
    if (e->mw_cap < need) {
        e->mean_attn_weights = (float*)grow(e->mean_attn_weights, e->mw_cap * 4, need * 4);
        e->mw_cap = need;
    }
    orc_engine_attend(e, Q, attn_output, e->mean_attn_weights);
    orc_engine_feedback(e, e->mean_attn_weights);
}

/* cache_engine.cpp:543-568 */
size_t orc_engine_buffer_bytes(const orc_engine* e) {
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    size_t b = 0;
    b += 2 * (size_t)e->sink_size * kvs * 4;
    b += 2 * (size_t)e->rw_size * kvs * 4;
    b += 2 * (size_t)e->max_hh * kvs * 4;
    b += (size_t)e->max_hh * 8 + (size_t)e->max_hh * 4;
    b += 2 * (size_t)e->chunk_size * kvs * 4;
    b += (size_t)e->chunk_size * 8;
    size_t nb = (size_t)e->pbs_allocated_blocks;
    size_t msz = e->use_fp16_meta ? 2 : 4;
    b += nb * (size_t)(e->k_group_size / 16) * kvs * 4;
    b += 2 * nb * kvs * msz;
    b += 2 * nb * (size_t)e->chunk_size * e->num_kv_heads * msz;
    b += nb * (size_t)e->chunk_size * e->num_kv_heads * e->quant_head_dim * 4;
    b += nb * (size_t)e->chunk_size * 8;
    b += (size_t)e->max_seq_len * 4;
    return b;
}

void orc_engine_counters(const orc_engine* e, int64_t* o) {
    int64_t v[ORC_N_COUNTERS] = {
        e->num_q_heads, e->num_kv_heads, e->head_dim, e->max_seq_len, e->sink_size, e->rw_size,
        e->update_interval, e->k_group_size, e->chunk_size, e->quant_head_dim, e->max_hh,
        e->use_fp16_meta, e->s_count, e->rw_count, e->rw_head_index, e->hh_count, e->wr_count,
        e->pbs_allocated_blocks, e->pbs_blocks_used, e->pbs_count, e->total_processed_tokens,
        e->last_calc_pos, e->total_evictions};
    memcpy(o, v, sizeof(v));
}

float orc_engine_cached_threshold(const orc_engine* e) { return e->cached_threshold; }

void* orc_engine_buffer(orc_engine* e, int which, int64_t* numel, int* es) {
    size_t kvs = (size_t)e->num_kv_heads * e->head_dim;
    size_t nb = (size_t)e->pbs_allocated_blocks;
    size_t ch = (size_t)e->chunk_size;
    int msz = e->use_fp16_meta ? 2 : 4;
    switch (which) {
    case 0: *numel = (int64_t)(e->sink_size * kvs); *es = 4; return e->S_K;
    case 1: *numel = (int64_t)(e->sink_size * kvs); *es = 4; return e->S_V;
    case 2: *numel = (int64_t)(e->rw_size * kvs); *es = 4; return e->RW_K;
    case 3: *numel = (int64_t)(e->rw_size * kvs); *es = 4; return e->RW_V;
    case 4: *numel = (int64_t)(e->max_hh * kvs); *es = 4; return e->HH_K;
    case 5: *numel = (int64_t)(e->max_hh * kvs); *es = 4; return e->HH_V;
    case 6: *numel = e->max_hh; *es = 8; return e->HH_token_ids;
    case 7: *numel = e->max_hh; *es = 4; return e->HH_scores;
    case 8: *numel = (int64_t)(ch * kvs); *es = 4; return e->WR_K;
    case 9: *numel = (int64_t)(ch * kvs); *es = 4; return e->WR_V;
    case 10: *numel = (int64_t)ch; *es = 8; return e->WR_token_ids;
    case 11: *numel = (int64_t)(nb * (e->k_group_size / 16) * kvs); *es = 4; return e->PBS_K_Packed;
    case 12: *numel = (int64_t)(nb * kvs); *es = msz; return e->PBS_K_Scales;
    case 13: *numel = (int64_t)(nb * kvs); *es = msz; return e->PBS_K_Zeroes;
    case 14: *numel = (int64_t)(nb * ch * e->num_kv_heads * e->quant_head_dim); *es = 4; return e->PBS_V_Packed;
    case 15: *numel = (int64_t)(nb * ch * e->num_kv_heads); *es = msz; return e->PBS_V_Scales;
    case 16: *numel = (int64_t)(nb * ch * e->num_kv_heads); *es = msz; return e->PBS_V_Zeroes;
    case 17: *numel = (int64_t)(nb * ch); *es = 8; return e->PBS_token_ids;
    case 18: *numel = e->max_seq_len; *es = 4; return e->global_attn_scores;
    default: *numel = 0; *es = 0; return NULL;
    }
}
