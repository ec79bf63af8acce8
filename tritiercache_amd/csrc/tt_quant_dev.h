// tt_quant_dev.h -- device functions for the bit-exact 2-bit quantisers.
// Used by the standalone kernels (tt_quant.hip) and by the engine's
// waiting-room flush (tt_engine.hip).
#pragma once
#include "tt_common.h"

namespace tt {

// K, one channel of one block (quantize_k_avx2.cpp:26-110). `src` points at
// token 0 of the channel, tokens `tok_stride` floats apart. `vec` selects the
// 8-wide vector body semantics (channel < 8*floor(D/8)) versus the scalar tail.
// Writes scale/zero and kgs/16 words spaced `word_stride` apart.
// KGS tokens known at compile time: every load is issued before the first
// use and each value is read once (the runtime-length loop waits for each
// load in turn, twice).
template <typename MetaT, int KGS>
__device__ __forceinline__ void quant_k_channel_n(const float* __restrict__ src, size_t tok_stride, bool vec,
                                                  MetaT* scale_dst, MetaT* zero_dst, uint32_t* packed_dst,
                                                  size_t word_stride) {
    float x[KGS];
#pragma unroll
    for (int t = 0; t < KGS; ++t) x[t] = src[t * tok_stride];
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
    for (int t = 0; t < KGS; ++t) {
        if (vec) {
            mn = x86_minps(mn, x[t]);
            mx = x86_maxps(mx, x[t]);
        } else {
            mn = std_min(mn, x[t]);
            mx = std_max(mx, x[t]);
        }
    }
    const float d3 = (mx - mn) / 3.0f;
    const float s = vec ? x86_maxps(d3, 1e-9f) : std_max(d3, 1e-9f);
    Meta<MetaT>::store(scale_dst, 0, s);
    Meta<MetaT>::store(zero_dst, 0, mn);
#pragma unroll
    for (int w = 0; w < KGS / 16; ++w) {
        uint32_t bits = 0;
#pragma unroll
        for (int st = 0; st < 16; ++st) {
            int q = cvt_rne_i32((x[w * 16 + st] - mn) / s);
            if (vec) {
                q = q > 0 ? q : 0;
                q = q < 3 ? q : 3;
            } else {
                q = q < 3 ? q : 3;
                q = q > 0 ? q : 0;
            }
            bits |= static_cast<uint32_t>(q) << (2 * st);
        }
        packed_dst[w * word_stride] = bits;
    }
}

template <typename MetaT>
__device__ __forceinline__ void quant_k_channel(const float* __restrict__ src, size_t tok_stride, int kgs, bool vec,
                                                MetaT* scale_dst, MetaT* zero_dst, uint32_t* packed_dst,
                                                size_t word_stride) {
    if (kgs == 16) {
        quant_k_channel_n<MetaT, 16>(src, tok_stride, vec, scale_dst, zero_dst, packed_dst, word_stride);
        return;
    }
    if (kgs == 32) {
        quant_k_channel_n<MetaT, 32>(src, tok_stride, vec, scale_dst, zero_dst, packed_dst, word_stride);
        return;
    }
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    for (int t = 0; t < kgs; ++t) {
        const float x = src[t * tok_stride];
        if (vec) {
            mn = x86_minps(mn, x);
            mx = x86_maxps(mx, x);
        } else {
            mn = std_min(mn, x);
            mx = std_max(mx, x);
        }
    }
    const float d3 = (mx - mn) / 3.0f;
    const float s = vec ? x86_maxps(d3, 1e-9f) : std_max(d3, 1e-9f);
    Meta<MetaT>::store(scale_dst, 0, s);
    Meta<MetaT>::store(zero_dst, 0, mn);
    const int words = kgs / 16;
    for (int w = 0; w < words; ++w) {
        uint32_t bits = 0;
        for (int st = 0; st < 16; ++st) {
            const float x = src[(w * 16 + st) * tok_stride];
            int q = cvt_rne_i32((x - mn) / s);
            if (vec) {
                q = q > 0 ? q : 0;
                q = q < 3 ? q : 3;
            } else {
                q = q < 3 ? q : 3;
                q = q > 0 ? q : 0;
            }
            bits |= static_cast<uint32_t>(q) << (2 * st);
        }
        packed_dst[w * word_stride] = bits;
    }
}

// hmin8 / hmax8 reduction trees (quantize_v_avx2.cpp:7-23).
__device__ __forceinline__ float hmin8(const float* x) {
    const float m0 = x86_minps(x[0], x[4]), m1 = x86_minps(x[1], x[5]);
    const float m2 = x86_minps(x[2], x[6]), m3 = x86_minps(x[3], x[7]);
    return x86_minps(x86_minps(m0, m2), x86_minps(m1, m3));
}
__device__ __forceinline__ float hmax8(const float* x) {
    const float m0 = x86_maxps(x[0], x[4]), m1 = x86_maxps(x[1], x[5]);
    const float m2 = x86_maxps(x[2], x[6]), m3 = x86_maxps(x[3], x[7]);
    return x86_maxps(x86_maxps(m0, m2), x86_maxps(m1, m3));
}

// V, one (token, head) row of D channels, D % 16 == 0
// (quantize_v_avx2.cpp:44-108): channel 16g+i lands in bits 2i of word g.
// The row's D/16 words are spread over `wpr` = D/16 consecutive lanes of one
// wave (lane w of the aligned group computes word w). The reference
// folds the 8-channel chunk minima (maxima) in channel order with a strict
// compare, so a NaN chunk result never replaces the running value and the
// first of equal values (a signed zero) stays. Each lane folds its two
// chunks the same way (never NaN), then the lanes combine in a tree whose
// kept operand on ties is always the lower channels': the same value as the
// reference's fold, bit for bit.
template <typename MetaT>
__device__ __forceinline__ void quant_v_row_lanes(const float* __restrict__ v, int w, int wpr, MetaT* scale_dst,
                                                  MetaT* zero_dst, int32_t* packed_dst) {
    float x[16];
    if ((reinterpret_cast<uintptr_t>(v) & 15) == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 f = reinterpret_cast<const float4*>(v + 16 * w)[j];
            x[4 * j] = f.x;
            x[4 * j + 1] = f.y;
            x[4 * j + 2] = f.z;
            x[4 * j + 3] = f.w;
        }
    } else {  // a caller's row that is only 4-byte aligned
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = v[16 * w + i];
    }
    float mn = std_min(std_min(__builtin_huge_valf(), hmin8(x)), hmin8(x + 8));
    float mx = std_max(std_max(-__builtin_huge_valf(), hmax8(x)), hmax8(x + 8));
    for (int m = 1; m < wpr; m <<= 1) {
        const float on = __shfl_xor(mn, m, 64), ox = __shfl_xor(mx, m, 64);
        const bool up = (w & m) != 0;
        mn = up ? std_min(on, mn) : std_min(mn, on);
        mx = up ? std_max(ox, mx) : std_max(mx, ox);
    }
    const float s = std_max((mx - mn) / 3.0f, 1e-9f);
    if (w == 0) {
        Meta<MetaT>::store(scale_dst, 0, s);
        Meta<MetaT>::store(zero_dst, 0, mn);
    }
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int q = cvt_rne_i32((x[i] - mn) / s);
        q = q < 3 ? q : 3;
        q = q > 0 ? q : 0;
        bits |= static_cast<uint32_t>(q) << (2 * i);
    }
    packed_dst[w] = static_cast<int32_t>(bits);
}

}  // namespace tt
