// tt_attn.hip -- single-pass split-K decode attention over the tiered cache (gfx950).
//
// Replaces the reference's fused_attention_decode_impl
// (csrc/cpu/fused_attn_avx2.cpp:145-301), which dequantises every packed block
// into a scratch buffer, stores a [Hq, N] score matrix and makes three passes.
// Here each token's K/V bytes are read from HBM once:
//
//   attn_split_kernel   grid (splits, Hkv, head-chunks), 256 threads = 4 waves.
//                       A workgroup owns one KV head and a contiguous, cost-
//                       balanced range of 16-token tiles (FP32 dense tiles
//                       first, then 2-bit packed tiles). Each wave streams its
//                       tiles with coalesced vector loads, unpacks the 2-bit
//                       words in registers (fmaf(q, scale, zero), the
//                       reference's dequant rounding), and folds them into the
//                       QK dot products and the PV accumulation of all GQA query
//                       heads of that KV head with an online softmax. Lanes are
//                       (token group tg = lane/16) x (channel slice cp = lane%16);
//                       QK partial sums reduce across the 16 channel lanes of a
//                       row with DPP butterflies. Waves merge in LDS; one
//                       (max, sum, acc[D]) partial per (query head, split).
//   attn_merge_kernel   LSE merge of the partials -> attn_output, row max/sum.
//   attn_mean_kernel    mean attention weights over query heads (:286-300),
//                       optional per-head weights, and the engine's decayed
//                       score feedback (cache_engine.cpp:511-540) in the same
//                       pass.
#include "tt_attn.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

namespace tt {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row. Butterfly pairs (xor 1, xor 2, then the
// half-row and row mirrors, which pair equal-valued quads / octets) so every
// lane of the row ends with the bit-identical total.
__device__ __forceinline__ float row_sum16(float x) {
    x = x + dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x = x + dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x = x + dpp<0x141>(x);  // row_half_mirror
    x = x + dpp<0x140>(x);  // row_mirror
    return x;
}

__device__ __forceinline__ float shfl_xor(float x, int m) { return __shfl_xor(x, m, 64); }

template <int N>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&x)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int j = 0; j < N; j += 4) {
            const float4 v = *reinterpret_cast<const float4*>(p + j);
            x[j] = v.x; x[j + 1] = v.y; x[j + 2] = v.z; x[j + 3] = v.w;
        }
    } else if constexpr (N == 2) {
        const float2 v = *reinterpret_cast<const float2*>(p);
        x[0] = v.x; x[1] = v.y;
    } else {
        x[0] = p[0];
    }
}

template <int N>
__device__ __forceinline__ void load_u32(const int32_t* __restrict__ p, uint32_t (&x)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int j = 0; j < N; j += 4) {
            const int4 v = *reinterpret_cast<const int4*>(p + j);
            x[j] = v.x; x[j + 1] = v.y; x[j + 2] = v.z; x[j + 3] = v.w;
        }
    } else if constexpr (N == 2) {
        const int2 v = *reinterpret_cast<const int2*>(p);
        x[0] = v.x; x[1] = v.y;
    } else {
        x[0] = p[0];
    }
}

template <typename MetaT, int N>
__device__ __forceinline__ void load_meta(const MetaT* __restrict__ p, float (&x)[N]) {
    if constexpr (sizeof(MetaT) == 4) {
        load_f32<N>(reinterpret_cast<const float*>(p), x);
    } else {
        if constexpr (N % 8 == 0) {
#pragma unroll
            for (int j = 0; j < N; j += 8) {
                const uint4 v = *reinterpret_cast<const uint4*>(p + j);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    x[j + 2 * k] = f16_to_f32(static_cast<uint16_t>(w[k] & 0xffffu));
                    x[j + 2 * k + 1] = f16_to_f32(static_cast<uint16_t>(w[k] >> 16));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) x[j] = f16_to_f32(reinterpret_cast<const uint16_t*>(p)[j]);
        }
    }
}

struct SplitArgs {
    AttnInputs in;
    float scale2;  // log2(e) / sqrt(head_dim): logits are kept in log2 units
    float* part_ml;
    float* part_acc;
    float* logits;
    int ld;
    int nsplit;      // partial slots per query head
    int nsplit_p;    // matrix-core workgroups over the packed store: slots [0, nsplit_p)
    int nsplit_d;    // VALU workgroups: slots [nsplit_p, nsplit)
    int dense_only;  // VALU workgroups take the FP32 tiles only
    int wd, wp;      // tile cost weights: dense, packed
};

// LDS of the VALU tile loop: per-wave (max, sum, acc[D]) for the final merge.
template <int D, int GP>
struct SplitLds {
    static constexpr int BYTES = 4 * GP * (2 + D) * 4;
};

// CPL: channels per lane (head_dim / 16). GP: query heads per workgroup
// (padded to a power of two; heads past the group are zero and never stored).
template <int CPL, int GP, typename MetaT>
__device__ __forceinline__ void split_body(const SplitArgs& a, const int split, char* lds) {
    constexpr int D = 16 * CPL;
    const AttnInputs& in = a.in;
    const int kvh = blockIdx.y;
    const int G = in.Hq / in.Hkv;
    const int g0 = blockIdx.z * GP;
    const int gc = min(GP, G - g0);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tg = lane >> 4;
    const int cp = lane & 15;

    int n0 = in.n0, n1 = in.n1, n2 = in.n2, head = in.ring_head, nb = in.num_blocks;
    if (in.state) {
        n0 = in.state[kSCount];
        n1 = in.state[kHhCount];
        n2 = in.state[kRwCount];
        head = in.state[kRwHead];
        nb = in.state[kBlocksUsed];
    }
    const int Nd = n0 + n1 + n2;
    const int W = in.kgs >> 4;
    const int Td = (Nd + 15) >> 4;
    const int Tp = a.dense_only ? 0 : nb * W;
    const int Hkv = in.Hkv;

    // Cost-balanced contiguous tile range of this split.
    const long long U = static_cast<long long>(Td) * a.wd + static_cast<long long>(Tp) * a.wp;
    const long long lo = U * split / a.nsplit_d, hi = U * (split + 1) / a.nsplit_d;
    auto cdiv = [](long long x, long long y) -> long long { return x <= 0 ? 0 : (x + y - 1) / y; };
    const int d_begin = static_cast<int>(min(cdiv(lo, a.wd), static_cast<long long>(Td)));
    const int d_end = static_cast<int>(min(cdiv(hi, a.wd), static_cast<long long>(Td)));
    const long long pb = static_cast<long long>(Td) * a.wd;
    const int p_begin = static_cast<int>(min(cdiv(lo - pb, a.wp), static_cast<long long>(Tp)));
    const int p_end = static_cast<int>(min(cdiv(hi - pb, a.wp), static_cast<long long>(Tp)));
    const int nd = d_end - d_begin;
    const int nt = nd + (p_end - p_begin);

    float q[GP][CPL];
#pragma unroll
    for (int g = 0; g < GP; ++g) {
        if (g < gc) {
            load_f32<CPL>(in.Q + static_cast<size_t>(kvh * G + g0 + g) * D + cp * CPL, q[g]);
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) q[g][j] = 0.0f;
        }
    }

    float m[GP], l[GP], acc[GP][CPL];
#pragma unroll
    for (int g = 0; g < GP; ++g) {
        m[g] = kNegInf;
        l[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[g][j] = 0.0f;
    }

    const MetaT* ks = static_cast<const MetaT*>(in.ks);
    const MetaT* kz = static_cast<const MetaT*>(in.kz);
    const MetaT* vs = static_cast<const MetaT*>(in.vs);
    const MetaT* vz = static_cast<const MetaT*>(in.vz);

    for (int it = wave; it < nt; it += 4) {
        float s[4][GP];
        float vx[4][CPL];
        bool valid[4];
        int tok0;  // logical index of token 0 of this lane's row group
        if (it < nd) {
            // ---- FP32 dense tile: logical rows 16k .. 16k+15 ----
            const int k = d_begin + it;
            tok0 = 16 * k + 4 * tg;
            float kx[4][CPL];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = tok0 + i;
                valid[i] = r < Nd;
                if (valid[i]) {
                    const float* kb;
                    const float* vb;
                    int idx;
                    if (r < n0) {
                        kb = in.k0; vb = in.v0; idx = r;
                    } else if (r < n0 + n1) {
                        kb = in.k1; vb = in.v1; idx = r - n0;
                    } else {
                        kb = in.k2; vb = in.v2;
                        idx = head + (r - n0 - n1);
                        if (idx >= in.ring_size) idx -= in.ring_size;
                    }
                    const size_t off = (static_cast<size_t>(idx) * Hkv + kvh) * D + cp * CPL;
                    load_f32<CPL>(kb + off, kx[i]);
                    load_f32<CPL>(vb + off, vx[i]);
                } else {
#pragma unroll
                    for (int j = 0; j < CPL; ++j) { kx[i][j] = 0.0f; vx[i][j] = 0.0f; }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int g = 0; g < GP; ++g) {
                    float d = 0.0f;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) d = __builtin_fmaf(q[g][j], kx[i][j], d);
                    s[i][g] = d;
                }
        } else {
            // ---- 2-bit packed tile: half (kgs 32) or whole (kgs 16) block ----
            const int kt = p_begin + (it - nd);
            const int b = kt / W, w = kt - b * W;
            const int slot0 = b * in.kgs + w * 16 + 4 * tg;
            tok0 = Nd + slot0;
            uint32_t kw[CPL];
            float ksc[CPL], kze[CPL];
            load_u32<CPL>(in.kp + ((static_cast<size_t>(b) * W + w) * Hkv + kvh) * D + cp * CPL, kw);
            const size_t moff = (static_cast<size_t>(b) * Hkv + kvh) * D + cp * CPL;
            load_meta<MetaT, CPL>(ks + moff, ksc);
            load_meta<MetaT, CPL>(kz + moff, kze);
            const longlong2 id01 = *reinterpret_cast<const longlong2*>(in.ids + slot0);
            const longlong2 id23 = *reinterpret_cast<const longlong2*>(in.ids + slot0 + 2);
            valid[0] = id01.x != -1; valid[1] = id01.y != -1;
            valid[2] = id23.x != -1; valid[3] = id23.y != -1;
            const int qhd = D / 16;
            const int cw = (cp * CPL) >> 4;
            const int sh0 = ((cp * CPL) & 15) * 2;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 4 * tg + i;  // token within the 16-token word
                const size_t vrow = static_cast<size_t>(slot0 + i) * Hkv + kvh;
                const uint32_t vwd = static_cast<uint32_t>(in.vp[vrow * qhd + cw]);
                const float vsc = Meta<MetaT>::load(vs, vrow);
                const float vze = Meta<MetaT>::load(vz, vrow);
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                    vx[i][j] = __builtin_fmaf(static_cast<float>((vwd >> (sh0 + 2 * j)) & 3u), vsc, vze);
                float kd[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                    kd[j] = __builtin_fmaf(static_cast<float>((kw[j] >> (2 * t)) & 3u), ksc[j], kze[j]);
#pragma unroll
                for (int g = 0; g < GP; ++g) {
                    float d = 0.0f;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) d = __builtin_fmaf(q[g][j], kd[j], d);
                    s[i][g] = d;
                }
            }
        }

        // QK partial sums -> full dot products (every lane of the row).
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                const float d = row_sum16(s[i][g]) * a.scale2;
                s[i][g] = valid[i] ? d : kNegInf;
            }

        if (a.logits) {
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                if (g < gc && cp == g) {
                    float* lr = a.logits + static_cast<size_t>(kvh * G + g0 + g) * a.ld;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (it >= nd || tok0 + i < Nd) lr[tok0 + i] = s[i][g];
                }
            }
        }

        // Online softmax update (max is exact, so every lane agrees on m).
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            float tm = fmaxf(fmaxf(s[0][g], s[1][g]), fmaxf(s[2][g], s[3][g]));
            tm = fmaxf(tm, shfl_xor(tm, 16));
            tm = fmaxf(tm, shfl_xor(tm, 32));
            const float mn = fmaxf(m[g], tm);
            const float alpha = (m[g] == kNegInf) ? 0.0f : exp2f(m[g] - mn);
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = (s[i][g] == kNegInf) ? 0.0f : exp2f(s[i][g] - mn);
            l[g] = __builtin_fmaf(l[g], alpha, (p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                float v = acc[g][j] * alpha;
                v = __builtin_fmaf(p[0], vx[0][j], v);
                v = __builtin_fmaf(p[1], vx[1][j], v);
                v = __builtin_fmaf(p[2], vx[2][j], v);
                v = __builtin_fmaf(p[3], vx[3][j], v);
                acc[g][j] = v;
            }
            m[g] = mn;
        }
    }

    // Reduce the four row groups (each accumulated its own tokens).
#pragma unroll
    for (int g = 0; g < GP; ++g) {
        l[g] += shfl_xor(l[g], 16);
        l[g] += shfl_xor(l[g], 32);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            acc[g][j] += shfl_xor(acc[g][j], 16);
            acc[g][j] += shfl_xor(acc[g][j], 32);
        }
    }

    // Merge the four waves in LDS and store one partial per query head.
    float* sm_m = reinterpret_cast<float*>(lds);  // [4][GP]
    float* sm_l = sm_m + 4 * GP;                   // [4][GP]
    float* sm_acc = sm_l + 4 * GP;                 // [4][GP][D]
    if (tg == 0) {
#pragma unroll
        for (int g = 0; g < GP; ++g) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) sm_acc[(wave * GP + g) * D + cp * CPL + j] = acc[g][j];
            if (cp == 0) {
                sm_m[wave * GP + g] = m[g];
                sm_l[wave * GP + g] = l[g];
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < gc * D; idx += 256) {
        const int g = idx / D, c = idx - g * D;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w * GP + g]);
        float A = 0.0f, L = 0.0f;
        if (M != kNegInf) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float mw = sm_m[w * GP + g];
                const float f = (mw == kNegInf) ? 0.0f : exp2f(mw - M);
                A = __builtin_fmaf(f, sm_acc[(w * GP + g) * D + c], A);
                L = __builtin_fmaf(f, sm_l[w * GP + g], L);
            }
        }
        const size_t pi = static_cast<size_t>(kvh * G + g0 + g) * a.nsplit + a.nsplit_p + split;
        a.part_acc[pi * D + c] = A;
        if (c == 0) {
            a.part_ml[2 * pi] = M;
            a.part_ml[2 * pi + 1] = L;
        }
    }
}

template <int CPL, int GP, typename MetaT>
__global__ void __launch_bounds__(256) attn_split_kernel(SplitArgs a) {
    __shared__ __align__(16) char lds[SplitLds<16 * CPL, GP>::BYTES];
    split_body<CPL, GP, MetaT>(a, static_cast<int>(blockIdx.x), lds);
}

#include "tt_attn_mfma.h"

// head_dim 128: workgroups [0, nsplit_p) run the matrix-core loop over the
// packed store, the rest the VALU loop over the FP32 tiles, in one launch so
// both kinds share the machine.
template <int GP, typename MetaT>
__global__ void __launch_bounds__(256) attn_tiles_kernel(SplitArgs a) {
    constexpr int kMf = 4 * MfLds<GP>::BYTES;
    constexpr int kVa = SplitLds<kMfD, GP>::BYTES;
    __shared__ __align__(16) char lds[kMf > kVa ? kMf : kVa];
    const int x = static_cast<int>(blockIdx.x);
    if (x < a.nsplit_p)
        packed_body<GP, MetaT>(a, x, lds);
    else
        split_body<8, GP, MetaT>(a, x - a.nsplit_p, lds);
}

// LSE merge of the split partials of one query head. 256 threads: the
// (max, sum) pairs are staged in LDS, the per-split weights exp(m_j - M) are
// computed once, and the weighted accumulators are summed with the splits
// divided between thread groups and the loads unrolled, so the kernel is
// bound by one pass over the partials rather than by load latency.
__global__ void __launch_bounds__(256) attn_merge_kernel(const float* __restrict__ part_ml,
                                                         const float* __restrict__ part_acc, int nsplit, int D,
                                                         float* __restrict__ out, float* __restrict__ rowstat) {
    extern __shared__ float sh[];
    float* fw = sh;                 // [nsplit] weights
    float* red = sh + nsplit;       // [256] scratch
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const float* ml = part_ml + static_cast<size_t>(h) * nsplit * 2;
    float mx = kNegInf;
    for (int j = tid; j < nsplit; j += 256) mx = fmaxf(mx, ml[2 * j]);
    red[tid] = mx;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
        __syncthreads();
    }
    const float M = red[0];
    __syncthreads();
    float lsum = 0.0f;
    for (int j = tid; j < nsplit; j += 256) {
        const float mj = ml[2 * j];
        const float f = (M == kNegInf || mj == kNegInf) ? 0.0f : exp2f(mj - M);
        fw[j] = f;
        lsum = __builtin_fmaf(f, ml[2 * j + 1], lsum);
    }
    red[tid] = lsum;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) red[tid] += red[tid + st];
        __syncthreads();
    }
    const float L = red[0];
    __syncthreads();
    // Thread groups of D threads split the splits; each thread owns channel c.
    const int groups = 256 / D;
    const int grp = tid / D, c = tid - grp * D;
    float A = 0.0f;
    if (grp < groups) {
        const float* base = part_acc + static_cast<size_t>(h) * nsplit * D + c;
        int j = grp;
        for (; j + 3 * groups < nsplit; j += 4 * groups) {
            const float a0 = base[static_cast<size_t>(j) * D];
            const float a1 = base[static_cast<size_t>(j + groups) * D];
            const float a2 = base[static_cast<size_t>(j + 2 * groups) * D];
            const float a3 = base[static_cast<size_t>(j + 3 * groups) * D];
            A = __builtin_fmaf(fw[j], a0, A);
            A = __builtin_fmaf(fw[j + groups], a1, A);
            A = __builtin_fmaf(fw[j + 2 * groups], a2, A);
            A = __builtin_fmaf(fw[j + 3 * groups], a3, A);
        }
        for (; j < nsplit; j += groups) A = __builtin_fmaf(fw[j], base[static_cast<size_t>(j) * D], A);
    }
    red[tid] = A;
    __syncthreads();
    if (tid < D) {
        float o = 0.0f;
        for (int g = 0; g < groups; ++g) o += red[g * D + tid];
        out[static_cast<size_t>(h) * D + tid] = (L > 0.0f) ? o / L : 0.0f;
    }
    if (tid == 0) {
        rowstat[2 * h] = M;
        rowstat[2 * h + 1] = L;
    }
}

struct MeanArgs {
    const float* logits;
    int ld;
    const float* rowstat;
    int Hq;
    int n_static;  // token count when no engine state
    const int* state;
    int kgs;
    float* mw;
    float* head_w;
    int head_w_ld;
    Feedback fb;
};

// One thread per attended token, one wave per workgroup so the grid covers
// every CU: w_h = exp(s_h - max_h) / sum_h summed over h = 0..Hq-1 in order
// and divided by Hq (fused_attn_avx2.cpp:286-300), then the engine's decayed
// score feedback for that token (cache_engine.cpp:511-540).
__global__ void __launch_bounds__(64) attn_mean_kernel(MeanArgs a) {
    extern __shared__ float sh[];  // [Hq] row max (log2 units), [Hq] 1/sum
    for (int h = threadIdx.x; h < a.Hq; h += blockDim.x) {
        const float M = a.rowstat[2 * h];
        const float L = a.rowstat[2 * h + 1];
        sh[h] = M;
        sh[a.Hq + h] = 1.0f / (L > 0.0f ? L : 1.0f);
    }
    __syncthreads();
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    int n = a.n_static;
    int s = 0, hh = 0, rw = 0, total = 0, Nd = 0;
    if (a.state) {
        s = a.state[kSCount];
        hh = a.state[kHhCount];
        rw = a.state[kRwCount];
        total = a.state[kTotal];
        Nd = s + hh + rw;
        n = Nd + a.state[kBlocksUsed] * a.kgs;
    }
    if (i >= n) return;
    const float* lg = a.logits + i;
    float sum = 0.0f;
    int h = 0;
    for (; h + 8 <= a.Hq; h += 8) {
        float sc[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) sc[u] = lg[static_cast<size_t>(h + u) * a.ld];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float w = (sc[u] == kNegInf) ? 0.0f : exp2f(sc[u] - sh[h + u]) * sh[a.Hq + h + u];
            sum += w;
            if (a.head_w && i < a.head_w_ld) a.head_w[static_cast<size_t>(h + u) * a.head_w_ld + i] = w;
        }
    }
    for (; h < a.Hq; ++h) {
        const float sc = lg[static_cast<size_t>(h) * a.ld];
        const float w = (sc == kNegInf) ? 0.0f : exp2f(sc - sh[h]) * sh[a.Hq + h];
        sum += w;
        if (a.head_w && i < a.head_w_ld) a.head_w[static_cast<size_t>(h) * a.head_w_ld + i] = w;
    }
    const float mean = sum / static_cast<float>(a.Hq);
    if (a.mw) a.mw[i] = mean;
    if (a.fb.g) {
        long long tid;
        int hh_slot = -1;
        if (i < s) {
            tid = i;
        } else if (i < s + hh) {
            hh_slot = i - s;
            tid = a.fb.hh_ids[hh_slot];
        } else if (i < Nd) {
            tid = static_cast<long long>(total) - rw + (i - s - hh);
        } else {
            tid = a.fb.pbs_ids[i - Nd];
        }
        if (tid >= 0 && tid < a.fb.max_seq_len) {
            const float gn = __builtin_fmaf(a.fb.decay, a.fb.g[tid], mean);
            a.fb.g[tid] = gn;
            if (hh_slot >= 0) a.fb.hh_scores[hh_slot] = gn;
        }
    }
}

template <int CPL, int GP>
int launch_split_meta(const SplitArgs& a, dim3 grid, int meta_fp16, hipStream_t st) {
    if (meta_fp16)
        hipLaunchKernelGGL((attn_split_kernel<CPL, GP, uint16_t>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((attn_split_kernel<CPL, GP, float>), grid, dim3(256), 0, st, a);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

template <int CPL>
int launch_split_g(const SplitArgs& a, dim3 grid, int gp, int meta_fp16, hipStream_t st) {
    switch (gp) {
    case 1: return launch_split_meta<CPL, 1>(a, grid, meta_fp16, st);
    case 2: return launch_split_meta<CPL, 2>(a, grid, meta_fp16, st);
    case 4: return launch_split_meta<CPL, 4>(a, grid, meta_fp16, st);
    default: return launch_split_meta<CPL, 8>(a, grid, meta_fp16, st);
    }
}

template <int GP>
int launch_tiles_meta(const SplitArgs& a, dim3 grid, int meta_fp16, hipStream_t st) {
    if (meta_fp16)
        hipLaunchKernelGGL((attn_tiles_kernel<GP, uint16_t>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((attn_tiles_kernel<GP, float>), grid, dim3(256), 0, st, a);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

int launch_tiles(const SplitArgs& a, dim3 grid, int gp, int meta_fp16, hipStream_t st) {
    switch (gp) {
    case 1: return launch_tiles_meta<1>(a, grid, meta_fp16, st);
    case 2: return launch_tiles_meta<2>(a, grid, meta_fp16, st);
    case 4: return launch_tiles_meta<4>(a, grid, meta_fp16, st);
    default: return launch_tiles_meta<8>(a, grid, meta_fp16, st);
    }
}

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int gp_for(int G) { return G >= 8 ? 8 : (G > 4 ? 8 : (G > 2 ? 4 : G)); }

// The matrix-core path serves head_dim 128 with either block size.
bool use_tiles_kernel(int D) { return D == kMfD; }

template <typename MetaT>
const void* tiles_kernel_ptr(int gp) {
    switch (gp) {
    case 1: return reinterpret_cast<const void*>(&attn_tiles_kernel<1, MetaT>);
    case 2: return reinterpret_cast<const void*>(&attn_tiles_kernel<2, MetaT>);
    case 4: return reinterpret_cast<const void*>(&attn_tiles_kernel<4, MetaT>);
    default: return reinterpret_cast<const void*>(&attn_tiles_kernel<8, MetaT>);
    }
}

template <int CPL>
const void* split_kernel_ptr(int gp, int fp16) {
    switch (gp) {
    case 1: return fp16 ? reinterpret_cast<const void*>(&attn_split_kernel<CPL, 1, uint16_t>)
                        : reinterpret_cast<const void*>(&attn_split_kernel<CPL, 1, float>);
    case 2: return fp16 ? reinterpret_cast<const void*>(&attn_split_kernel<CPL, 2, uint16_t>)
                        : reinterpret_cast<const void*>(&attn_split_kernel<CPL, 2, float>);
    case 4: return fp16 ? reinterpret_cast<const void*>(&attn_split_kernel<CPL, 4, uint16_t>)
                        : reinterpret_cast<const void*>(&attn_split_kernel<CPL, 4, float>);
    default: return fp16 ? reinterpret_cast<const void*>(&attn_split_kernel<CPL, 8, uint16_t>)
                         : reinterpret_cast<const void*>(&attn_split_kernel<CPL, 8, float>);
    }
}

// Workgroups of the split launch the device holds at once: CUs x occupancy
// (queried once per device and shape, then cached).
int resident_split_wgs(int D, int G, int fp16) {
    static std::mutex mu;
    static std::map<std::tuple<int, int, int, int>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1024;
    const int gp = gp_for(G);
    const auto key = std::make_tuple(dev, D, gp, fp16);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    const void* fn = nullptr;
    if (use_tiles_kernel(D)) {
        fn = fp16 ? tiles_kernel_ptr<uint16_t>(gp) : tiles_kernel_ptr<float>(gp);
    } else {
        switch (D) {
        case 16: fn = split_kernel_ptr<1>(gp, fp16); break;
        case 32: fn = split_kernel_ptr<2>(gp, fp16); break;
        case 64: fn = split_kernel_ptr<4>(gp, fp16); break;
        default: fn = split_kernel_ptr<16>(gp, fp16); break;
        }
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0) != hipSuccess || per_cu <= 0) {
        (void)hipGetLastError();
        per_cu = 2;
    }
    const int r = cus * per_cu;
    cache[key] = r;
    return r;
}

}  // namespace

int attn_check_shapes(int Hq, int Hkv, int D, int kgs) {
    if (Hq <= 0 || Hkv <= 0 || D <= 0)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_q_heads, num_kv_heads, and head_dim must be positive integers.");
    if (Hq % Hkv != 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_q_heads must be a multiple of num_kv_heads.");
    if (D % 16 != 0 || D > 256 || (D & (D - 1)) != 0)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "head_dim must be one of 16, 32, 64, 128, 256.");
    if (kgs != 16 && kgs != 32) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "k_group_size must be 16 or 32.");
    return TT_OK;
}

AttnPlan attn_plan(int dense_ub, int blocks_ub, int Hq, int Hkv, int D, int kgs, bool need_logits, int meta_fp16) {
    AttnPlan p;
    const int W = kgs / 16;
    const int G = Hq / Hkv;
    const int chunks = (G + gp_for(G) - 1) / gp_for(G);
    const long long heads = static_cast<long long>(Hkv) * chunks;
    const long long resident = resident_split_wgs(D, G, meta_fp16);
    const long long per_head = std::max<long long>(1, (resident + heads - 1) / heads);
    const long long dense_tiles = (dense_ub + 15) / 16;
    if (use_tiles_kernel(D)) {
        // Dense workgroups take ~8 FP32 tiles (two per wave); the packed
        // workgroups fill the rest of one resident round, with at least ~8
        // pairs of tiles each so the partials stay small.
        const long long pairs = (static_cast<long long>(blocks_ub) * W + 1) / 2;
        p.nsplit_d = static_cast<int>(std::max<long long>(1, (dense_tiles + 7) / 8));
        const long long want = std::max<long long>(1, per_head - p.nsplit_d);
        p.nsplit_p = static_cast<int>(std::max<long long>(1, std::min(want, pairs / 8)));
    } else {
        // One round of resident workgroups, but at least ~32 packed-tile
        // units of work per workgroup so the merge traffic stays small.
        const long long units = dense_tiles * 8 + static_cast<long long>(blocks_ub) * W;
        const long long cap = std::max<long long>(1, units / 32);
        p.nsplit_p = 0;
        p.nsplit_d = static_cast<int>(std::max<long long>(1, std::min(per_head, cap)));
    }
    p.nsplit = p.nsplit_p + p.nsplit_d;
    p.token_ub = dense_ub + blocks_ub * kgs;
    p.ld = (p.token_ub + 3) & ~3;
    p.logits = need_logits;
    size_t off = 0;
    p.off_ml = off;
    off = align256(off + sizeof(float) * 2 * static_cast<size_t>(Hq) * p.nsplit);
    p.off_acc = off;
    off = align256(off + sizeof(float) * static_cast<size_t>(Hq) * p.nsplit * D);
    p.off_rowstat = off;
    off = align256(off + sizeof(float) * 2 * static_cast<size_t>(Hq));
    p.off_logits = off;
    if (need_logits) off = align256(off + sizeof(float) * static_cast<size_t>(Hq) * std::max(p.ld, 4));
    p.bytes = off;
    return p;
}

int attn_launch_split(const AttnInputs& in, const AttnPlan& plan, void* ws, hipStream_t stream) {
    char* base = static_cast<char*>(ws);
    SplitArgs a;
    a.in = in;
    a.scale2 = kLog2e / sqrtf(static_cast<float>(in.D));
    a.part_ml = reinterpret_cast<float*>(base + plan.off_ml);
    a.part_acc = reinterpret_cast<float*>(base + plan.off_acc);
    a.logits = plan.logits ? reinterpret_cast<float*>(base + plan.off_logits) : nullptr;
    a.ld = plan.ld;
    a.nsplit = plan.nsplit;
    a.nsplit_p = plan.nsplit_p;
    a.nsplit_d = plan.nsplit_d;
    a.dense_only = plan.nsplit_p > 0 ? 1 : 0;
    a.wd = 8;
    a.wp = 1;
    const int G = in.Hq / in.Hkv;
    const int gp = gp_for(G);
    const dim3 grid(plan.nsplit, in.Hkv, (G + gp - 1) / gp);
    if (use_tiles_kernel(in.D)) {
        if (plan.nsplit_p <= 0) TT_FAIL(TT_ERR_RUNTIME, "attention plan does not match head_dim");
        return launch_tiles(a, grid, gp, in.meta_fp16, stream);
    }
    if (plan.nsplit_p != 0) TT_FAIL(TT_ERR_RUNTIME, "attention plan does not match head_dim");
    switch (in.D) {
    case 16: return launch_split_g<1>(a, grid, gp, in.meta_fp16, stream);
    case 32: return launch_split_g<2>(a, grid, gp, in.meta_fp16, stream);
    case 64: return launch_split_g<4>(a, grid, gp, in.meta_fp16, stream);
    case 128: return launch_split_g<8>(a, grid, gp, in.meta_fp16, stream);
    default: return launch_split_g<16>(a, grid, gp, in.meta_fp16, stream);
    }
}

int attn_launch_finalize(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out, float* mean_w,
                         const Feedback* fb, float* head_w, int head_w_ld, hipStream_t stream) {
    char* base = static_cast<char*>(ws);
    const float* part_ml = reinterpret_cast<const float*>(base + plan.off_ml);
    const float* part_acc = reinterpret_cast<const float*>(base + plan.off_acc);
    float* rowstat = reinterpret_cast<float*>(base + plan.off_rowstat);
    const size_t merge_lds = sizeof(float) * (static_cast<size_t>(plan.nsplit) + 256);
    hipLaunchKernelGGL(attn_merge_kernel, dim3(in.Hq), dim3(256), merge_lds, stream, part_ml, part_acc, plan.nsplit,
                       in.D, out, rowstat);
    TT_LAUNCH_CHECK();
    if (plan.logits && (mean_w || head_w || (fb && fb->g))) {
        MeanArgs m;
        m.logits = reinterpret_cast<const float*>(base + plan.off_logits);
        m.ld = plan.ld;
        m.rowstat = rowstat;
        m.Hq = in.Hq;
        m.n_static = in.n0 + in.n1 + in.n2 + in.num_blocks * in.kgs;
        m.state = in.state;
        m.kgs = in.kgs;
        m.mw = mean_w;
        m.head_w = head_w;
        m.head_w_ld = head_w_ld;
        m.fb = fb ? *fb : Feedback{};
        const int n = std::max(plan.token_ub, 1);
        hipLaunchKernelGGL(attn_mean_kernel, dim3((n + 63) / 64), dim3(64), sizeof(float) * 2 * in.Hq, stream, m);
        TT_LAUNCH_CHECK();
    }
    return TT_OK;
}

int attn_launch(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out, float* mean_w, const Feedback* fb,
                float* head_w, int head_w_ld, hipStream_t stream) {
    int rc = attn_launch_split(in, plan, ws, stream);
    if (rc != TT_OK) return rc;
    return attn_launch_finalize(in, plan, ws, out, mean_w, fb, head_w, head_w_ld, stream);
}

}  // namespace tt
