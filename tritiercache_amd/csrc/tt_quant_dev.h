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

// Packs 16 channels (x[i] -> bits 2i) against the row's (mn, s).
__device__ __forceinline__ uint32_t quant_v_word(const float* x, float mn, float s) {
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int q = cvt_rne_i32((x[i] - mn) / s);
        q = q < 3 ? q : 3;
        q = q > 0 ? q : 0;
        bits |= static_cast<uint32_t>(q) << (2 * i);
    }
    return bits;
}

// V, one (token, head) row of D channels, D % 16 == 0
// (quantize_v_avx2.cpp:44-108): channel 16g+i lands in bits 2i of word g.
// The row's wpr = D/16 words are spread over a group of `group` consecutive
// lanes of one wave (group: a power of two, wpr <= group <= 64, so a group
// never straddles waves); lane w < wpr of the aligned group computes word w,
// lanes w >= wpr only pad the reduction tree. The reference folds the
// 8-channel chunk minima (maxima) in channel order with a strict compare, so
// a NaN chunk result never replaces the running value and the first of equal
// values (a signed zero) stays. Each lane folds its two chunks the same way
// (never NaN), then the lanes combine in a tree whose kept operand on ties is
// always the lower channels': the same value as the reference's fold, bit
// for bit. Padding lanes hold +inf / -inf, which a real lane's value always
// keeps (a tie with +inf keeps the lower lane's +inf, the same value).
template <typename MetaT>
__device__ __forceinline__ void quant_v_row_lanes(const float* __restrict__ v, int w, int wpr, int group,
                                                  MetaT* scale_dst, MetaT* zero_dst, int32_t* packed_dst) {
    const bool real = w < wpr;
    float x[16];
    if (!real) {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = 0.0f;
    } else if ((reinterpret_cast<uintptr_t>(v) & 15) == 0) {
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
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    if (real) {
        mn = std_min(std_min(mn, hmin8(x)), hmin8(x + 8));
        mx = std_max(std_max(mx, hmax8(x)), hmax8(x + 8));
    }
    for (int m = 1; m < group; m <<= 1) {
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
    if (real) packed_dst[w] = static_cast<int32_t>(quant_v_word(x, mn, s));
}

// The same row on one thread, for rows of more than 64 words: the
// reference's sequential fold over the 8-channel chunks, then every word.
template <typename MetaT>
__device__ __forceinline__ void quant_v_row_serial(const float* __restrict__ v, int wpr, MetaT* scale_dst,
                                                   MetaT* zero_dst, int32_t* packed_dst) {
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    for (int c = 0; c < 16 * wpr; c += 8) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = v[c + i];
        mn = std_min(mn, hmin8(x));
        mx = std_max(mx, hmax8(x));
    }
    const float s = std_max((mx - mn) / 3.0f, 1e-9f);
    Meta<MetaT>::store(scale_dst, 0, s);
    Meta<MetaT>::store(zero_dst, 0, mn);
    for (int w = 0; w < wpr; ++w) {
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = v[16 * w + i];
        packed_dst[w] = static_cast<int32_t>(quant_v_word(x, mn, s));
    }
}

// Lanes per row for quant_v_row_lanes: the next power of two >= wpr, or 0
// when that exceeds a wave (use quant_v_row_serial).
__host__ __device__ inline int quant_v_group(int wpr) {
    int g = 1;
    while (g < wpr) g <<= 1;
    return g <= 64 ? g : 0;
}

}  // namespace tt
