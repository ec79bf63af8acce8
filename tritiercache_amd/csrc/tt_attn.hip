// tt_attn.hip -- single-pass split-K decode attention over the tiered cache (gfx950).
//
// Replaces the reference's fused_attention_decode_impl
// (csrc/cpu/fused_attn_avx2.cpp:145-301), which dequantises every packed block
// into a scratch buffer, stores a [Hq, N] score matrix and makes three passes.
// Here each token's K/V bytes are read from HBM once. Logits are kept in
// log2 units (dot * log2(e) / sqrt(D)) so every exponential is one v_exp_f32.
//
//   attn_packed_kernel  head_dim 128: the 2-bit packed blocks on the matrix
//                       cores (tt_attn_mfma.h), grid (splits, Hkv, head
//                       chunks), 4 waves; one (max, sum, acc[D]) partial per
//                       (query head, split).
//   attn_split_kernel   VALU loop, grid (splits, Hkv, head chunks), 4 waves.
//                       A workgroup owns one KV head and a contiguous, cost-
//                       balanced range of 16-token tiles: the FP32 tiers (with
//                       head_dim 128 only these) and, for other head sizes,
//                       the 2-bit tiles too, unpacked in registers with the
//                       reference's dequant rounding fmaf(q, scale, zero).
//                       Lanes are (token group tg = lane/16) x (channel slice
//                       cp = lane%16); QK partial sums reduce across the 16
//                       channel lanes of a row with DPP butterflies; online
//                       softmax over all GQA query heads of the KV head.
//   attn_finalize_kernel  LSE merge of the partials -> attn_output, and in the
//                       same launch the mean attention weights over query
//                       heads (:286-300), optional per-head weights and the
//                       engine's decayed score feedback (cache_engine.cpp:
//                       511-540).
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
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int j = 0; j < N; j += 2) {
            const float2 v = *reinterpret_cast<const float2*>(p + j);
            x[j] = v.x; x[j + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) x[j] = p[j];
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
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int j = 0; j < N; j += 2) {
            const int2 v = *reinterpret_cast<const int2*>(p + j);
            x[j] = v.x; x[j + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) x[j] = static_cast<uint32_t>(p[j]);
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
    int wd, wp;      // tile cost weights: dense, packed
    int dense_delay; // FP32-tier workgroups wait this many 10 ns ticks before their first tile load
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
    const int Tp = nb * W;
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
            // The lane's channels c0 .. c0 + CPL - 1 lie in V word c0 / 16, and
            // in the next word too when CPL does not divide 16 (head_dim 48,
            // 80, 96, ...; CPL <= 16, so never a third).
            constexpr bool kOneWord = (16 % CPL) == 0;
            const int c0 = cp * CPL;
            const int cw = c0 >> 4;
            const int cw1 = kOneWord ? cw : ((c0 + CPL - 1) >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 4 * tg + i;  // token within the 16-token word
                const size_t vrow = static_cast<size_t>(slot0 + i) * Hkv + kvh;
                const uint32_t vwd = static_cast<uint32_t>(in.vp[vrow * qhd + cw]);
                const uint32_t vwd1 = kOneWord ? vwd : static_cast<uint32_t>(in.vp[vrow * qhd + cw1]);
                const float vsc = Meta<MetaT>::load(vs, vrow);
                const float vze = Meta<MetaT>::load(vz, vrow);
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const int c = c0 + j;
                    const uint32_t w = (kOneWord || (c >> 4) == cw) ? vwd : vwd1;
                    vx[i][j] = __builtin_fmaf(static_cast<float>((w >> (2 * (c & 15))) & 3u), vsc, vze);
                }
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
            const float alpha = (m[g] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(m[g] - mn);
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = (s[i][g] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(s[i][g] - mn);
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
                const float f = (mw == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
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

// head_dim 128: a 1-D grid of ceil(nsplit / 8) * 8 slots per (KV head, head
// chunk). Slots s < nsplit_p run the matrix-core loop over pair range s of
// the packed store, slots nsplit_p <= s < nsplit a VALU pass over a share of
// the FP32 tiers; every workgroup writes its own partial slot.
//
// Workgroup ids go round-robin over the 8 XCDs (id % 8), each with its own
// L2. The id -> (slot, head) map puts slot s on XCD s % 8 for every head and
// dispatches the heads of one slot back to back: a token's V words, V scale /
// zero and id sit in the same 128-byte lines for all KV heads, so they come
// from memory once per token instead of once per head.
//
// Eight-head groups are held to three waves per SIMD (168 VGPRs, no spills:
// the loop's rare tail paths and the epilogue recompute their lane indices).
//
// PAIR: head_dim-64 KV heads 2j and 2j + 1 as one head of 128 channels (the
// arguments describe num_kv_heads / 2 heads of head_dim 128; see packed_body).
template <int GP, typename MetaT, bool PAIR = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((GP == 8 || PAIR) ? 3 : 1)))
attn_packed_kernel(SplitArgs a, const int hc, const int chunks) {
    constexpr int kLds = MfLds<GP>::TOTAL > DnLds<GP>::TOTAL ? MfLds<GP>::TOTAL : DnLds<GP>::TOTAL;
    __shared__ __align__(16) char lds[kLds];
    const unsigned id = blockIdx.x;
    const unsigned q = id >> 3;
    const int hz = static_cast<int>(q % static_cast<unsigned>(hc));  // (KV head, chunk)
    const int s = static_cast<int>((q / static_cast<unsigned>(hc)) * 8 + (id & 7));
    if (s >= a.nsplit) return;  // padding slot of the last group of 8
    const int kvh = hz / chunks, chunk = hz - kvh * chunks;
    if (s >= a.nsplit_p) {
        dense_body<GP, PAIR>(a, s - a.nsplit_p, kvh, chunk, lds);
        return;
    }
    packed_body<GP, MetaT, PAIR>(a, s, kvh, chunk, lds);
}

// ---------------------------------------------------------------------------
// Finalize: one launch with two kinds of workgroups.
//   [0, Hq S)      merge the split partials of query head h (log2 units),
//                  S workgroups per head, one per 32 output channels:
//                  M = max_j m_j, L = sum_j l_j 2^(m_j - M),
//                  out = sum_j acc_j 2^(m_j - M) / L.
//   [Hq S, ...)    mean attention weights of blocks of kMeanTokens (long contexts: kMeanTokensLong) tokens
//                  (fused_attn_avx2.cpp:286-300): every such workgroup first
//                  rebuilds (M, 1/L) of all heads from the (m, l) partials,
//                  then w_h = 2^(s_h - M_h) / L_h summed over the heads and
//                  divided by Hq, optional per-head weights, and the engine's
//                  decayed score feedback (cache_engine.cpp:511-540).
// Neither kind waits for the other, so the two run side by side.
// ---------------------------------------------------------------------------
struct FinArgs {
    const float* part_ml;
    const float* part_acc;
    int nsplit;
    int D;
    int Hq;
    int pair_g;  // paired head_dim-64 heads: query heads per real KV head (0: not paired)
    float* out;
    float* rowstat;
    const float* logits;  // null: no mean-weight workgroups
    int ld;
    int n_static;         // token count when no engine state
    const int* state;
    int kgs;
    float* mw;
    float* head_w;
    int head_w_ld;
    Feedback fb;
};

// Wave-wide reductions with DPP inside rows and two cross-row swaps.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float wave_sum(float x) {
    x = row_sum16(x);
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

// Merge of query head h. Every load is issued before the first reduction:
// thread t holds (m_t, l_t) of split t, and thread (group g, channel quad c4)
// the accumulators of splits g, g + groups, ... (up to kMergeU per group and
// block of 256 splits, all in flight together).
constexpr int kMergeU = 16;

// The (m, l) statistics of two consecutive splits. A head's row starts at
// 2 * h * nsplit floats and a pair at an even split only when nsplit is even,
// so the pair is read as two 8-byte loads rather than one 16-byte load.
__device__ __forceinline__ float4 load_ml_pair(const float* p) {
    const float2 a = *reinterpret_cast<const float2*>(p);
    const float2 b = *reinterpret_cast<const float2*>(p + 2);
    return make_float4(a.x, a.y, b.x, b.y);
}

// Workgroups per query head in the merge. One workgroup holds the loads of
// kMergeU splits per thread-group in flight (16384 / width splits for `width`
// channels); a head with more than 4096 / width splits (32 at head_dim 128)
// is cut into slices of 32 channels (head_dim a multiple of 32), each merged
// by its own workgroup that rebuilds the head's (M, L) from the split
// statistics: the merge stays one round trip of loads, and each workgroup
// issues a quarter of them (32k Llama-3-8B layers, 96 splits: 640.8 against
// 650.7 us per step with f16 metadata, 656.2 against 662.7 with f32). A
// paired head_dim-64 head covers only its own 64 channels of the pair's 128.
__host__ __device__ inline int fin_merge_slices(const int D, const int pair_g, const int nsplit) {
    const int need = pair_g ? 64 : D;
    if (nsplit * need <= 4096 || need % 32 != 0) return 1;
    return need / 32;
}

__device__ __forceinline__ void fin_merge_head(const FinArgs& a, const int h, const int slice, const int msl,
                                               float* sh) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const float* ml = a.part_ml + static_cast<size_t>(h) * a.nsplit * 2;
    const int width = (a.pair_g ? 64 : a.D) / msl;
    const int c0 = (a.pair_g ? ((h % (2 * a.pair_g)) / a.pair_g) * 64 : 0) + width * slice;
    const int q = width >> 2;
    const int groups = 256 / q;
    const int g = t / q, c4 = t - g * q;
    const float* base = a.part_acc + static_cast<size_t>(h) * a.nsplit * a.D + c0 + 4 * c4;
    float* red = sh + 8;  // [256][4]
    float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float L = 0.0f, M = kNegInf;
    for (int j0 = 0; j0 < a.nsplit; j0 += 256) {
        // (max, sum) over splits j0 .. j0 + 255 folded into the running (M, L)
        const int jt = j0 + t;
        const float mt = jt < a.nsplit ? ml[2 * jt] : kNegInf;
        const float lt = jt < a.nsplit ? ml[2 * jt + 1] : 0.0f;
        float4 v[kMergeU];
        float mv[kMergeU];
#pragma unroll
        for (int u = 0; u < kMergeU; ++u) {
            const int j = j0 + g + u * groups;
            const bool in = g < groups && j < a.nsplit && j < j0 + 256;
            v[u] = in ? *reinterpret_cast<const float4*>(base + static_cast<size_t>(j) * a.D)
                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            mv[u] = in ? ml[2 * j] : kNegInf;
        }
        const float wm = wave_max(mt);
        if (lane == 0) sh[wave] = wm;
        __syncthreads();
        const float Mb = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
        const float Mn = fmaxf(M, Mb);
        const float ws = wave_sum(mt == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(mt - Mn) * lt);
        __syncthreads();
        if (lane == 0) sh[4 + wave] = ws;
        const float al = (M == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
        A.x *= al; A.y *= al; A.z *= al; A.w *= al;
#pragma unroll
        for (int u = 0; u < kMergeU; ++u) {
            const float f = (mv[u] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(mv[u] - Mn);
            A.x = __builtin_fmaf(f, v[u].x, A.x);
            A.y = __builtin_fmaf(f, v[u].y, A.y);
            A.z = __builtin_fmaf(f, v[u].z, A.z);
            A.w = __builtin_fmaf(f, v[u].w, A.w);
        }
        // splits beyond kMergeU per group in this block of 256 (groups < 16 only)
        for (int j = j0 + g + kMergeU * groups; g < groups && j < a.nsplit && j < j0 + 256; j += groups) {
            const float mj = ml[2 * j];
            const float f = (mj == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(mj - Mn);
            const float4 w = *reinterpret_cast<const float4*>(base + static_cast<size_t>(j) * a.D);
            A.x = __builtin_fmaf(f, w.x, A.x);
            A.y = __builtin_fmaf(f, w.y, A.y);
            A.z = __builtin_fmaf(f, w.z, A.z);
            A.w = __builtin_fmaf(f, w.w, A.w);
        }
        __syncthreads();
        L = L * al + ((sh[4] + sh[5]) + (sh[6] + sh[7]));
        M = Mn;
        __syncthreads();
    }
    *reinterpret_cast<float4*>(red + 4 * t) = A;
    __syncthreads();
    if (t < width) {
        const int cq = t >> 2, ci = t & 3;
        float o = 0.0f;
        for (int gg = 0; gg < groups; ++gg) o += red[4 * (gg * q + cq) + ci];
        o = (L > 0.0f) ? o / L : 0.0f;
        if (a.pair_g == 0)
            a.out[static_cast<size_t>(h) * a.D + c0 + t] = o;
        else  // a paired head_dim-64 head: its own 64 channels of the pair's 128
            a.out[static_cast<size_t>(h) * 64 + (c0 & 63) + t] = o;
    }
    if (t == 0 && slice == 0) {
        a.rowstat[2 * h] = M;
        a.rowstat[2 * h + 1] = L;
    }
}

// Max over the 8 lanes of an aligned group (xor 1, 2, 4 via DPP).
__device__ __forceinline__ float max8(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    return fmaxf(x, dpp<0x141>(x) /* row_half_mirror pairs lanes 0-7 */);
}
__device__ __forceinline__ float sum8(float x) {
    x = x + dpp<0xB1>(x);
    x = x + dpp<0x4E>(x);
    return x + dpp<0x141>(x);
}

#ifndef TT_MEAN_TOKENS
#define TT_MEAN_TOKENS 64
#endif
constexpr int kMeanTokens = TT_MEAN_TOKENS;  // tokens per mean-weight block
// Long contexts use blocks twice as long: half the workgroups rebuild the
// split statistics, and each still has 4 tokens per thread.
constexpr int kMeanTokensLong = 2 * kMeanTokens;
constexpr int kMeanLongFrom = 65536;  // attended tokens (upper bound) from which the long blocks pay
// Mean-weight workgroups at most; past that each takes an equal number of
// token blocks, so fewer of them rebuild the per-head row statistics.
#ifndef TT_MEAN_WGS
#define TT_MEAN_WGS 1024
#endif
constexpr int kMeanMaxWgs = TT_MEAN_WGS;

// Logits of token quad i0 for the heads hb + hg + groups u, u < 8 (-inf past
// the end and for missing heads); groups = head groups of a MT-token block.
template <int MT>
__device__ __forceinline__ void fin_load_logits(const FinArgs& a, const int hb, const int hg, const int i0,
                                                const int n, float4 (&lgv)[8]) {
    constexpr int kGroups = 256 / (MT / 4);
    const int Hq = a.Hq;
    const bool whole = i0 + 4 <= n;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int h = hb + hg + kGroups * u;
        lgv[u] = make_float4(kNegInf, kNegInf, kNegInf, kNegInf);
        if (h < Hq && i0 < n) {
            const float* lg = a.logits + static_cast<size_t>(h) * a.ld + i0;
            if (whole) {
                lgv[u] = *reinterpret_cast<const float4*>(lg);
            } else {
                lgv[u].x = lg[0];
                if (i0 + 1 < n) lgv[u].y = lg[1];
                if (i0 + 2 < n) lgv[u].z = lg[2];
            }
        }
    }
}

// The same logits for hb = 0 and u < NU without a branch: the row index is
// clamped to Hq - 1 and the token quad to the padded row's last one, so every
// load stays inside the logits array and is issued whatever the thread's
// position; rows h >= Hq are never read back, and tokens i0 + e >= n are
// masked where the values are used. Statistics loads issued before these can
// then be waited for alone (loads return in order).
// Eight rows (more than 4 groups of heads) keep the branches, as their
// registers would not fit beside the statistics.
template <int MT, int NU>
__device__ __forceinline__ void fin_load_logits_nb(const FinArgs& a, const int hg, const int i0, const int n,
                                                   float4 (&lgv)[8]) {
    if constexpr (NU == 8) {
        fin_load_logits<MT>(a, 0, hg, i0, n, lgv);
    } else {
        constexpr int kGroups = 256 / (MT / 4);
        const int ic = i0 < a.ld - 4 ? i0 : a.ld - 4;  // ld: a multiple of 4, at least 4
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int h = hg + kGroups * u;
            const int hc = h < a.Hq ? h : a.Hq - 1;
            lgv[u] = *reinterpret_cast<const float4*>(a.logits + static_cast<size_t>(hc) * a.ld + ic);
        }
    }
}

// Token i's position in the score vector (-1 for none) and, for a heavy
// hitter, its slot.
struct FbToken {
    long long tid;
    int hh_slot;
};

// Mean-weight workgroup `wg` of `nwg`: token blocks wg, wg + nwg, ... of
// MT tokens each. The loads of a block's feedback ids and scores are
// issued when the block starts, those of the next block's logits as soon as
// the current ones are consumed. NU: logits rows per thread of the first head
// round, a power of two with NU * (256 / (MT / 4)) >= min(Hq, 8 * (256 / (MT / 4))).
template <int MT, bool kRowstat, int NU>
__device__ __forceinline__ void fin_mean_tokens(const FinArgs& a, const int wg, const int nwg, float* sh) {
    constexpr int kQuads = MT / 4;         // token quads per block
    constexpr int kGroups = 256 / kQuads;  // head groups per workgroup
    const int t = threadIdx.x;
    const int Hq = a.Hq;
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
    if (wg * MT >= n) return;
    // Feedback target of token i (threads t < MT, one token each).
    auto fb_token = [&](const int i) {
        FbToken f{-1, -1};
        if (i >= n) return f;
        if (i < s) {
            f.tid = i;
        } else if (i < s + hh) {
            f.hh_slot = i - s;
            f.tid = a.fb.hh_ids[f.hh_slot];
        } else if (i < Nd) {
            f.tid = static_cast<long long>(total) - rw + (i - s - hh);
        } else {
            f.tid = a.fb.pbs_ids[i - Nd];
        }
        if (f.tid < 0 || f.tid >= a.fb.max_seq_len) f.tid = -1;
        return f;
    };
    const bool fb_lane = a.fb.g && t < MT;
    FbToken ft{-1, -1};
    float g_old = 0.0f;
    if (fb_lane) {
        ft = fb_token(wg * MT + t);
        if (ft.tid >= 0) g_old = a.fb.g[ft.tid];
    }
    // Thread (head group hg, token quad q): heads hg, hg + kGroups, ...;
    // tokens tok0 + 4 q .. + 3. Rows are padded to a multiple of 4 floats.
    const int q = t % kQuads, hg = t / kQuads;
    // (M_h, 1/L_h) of every head: 8 threads per head, splits 2 j0 + 16 u and
    // the one after (every workgroup rebuilds them: a second launch that waits
    // for the merge costs more than these loads). Their loads are issued
    // first and the first block's logits loads right behind them, before the
    // statistics are folded: both round trips overlap, and the fold waits for
    // the statistics alone.
    float* Mh = sh;        // [Hq]
    float* iL = sh + Hq;   // [Hq]
    float4 lgv[8];
    constexpr int kU4 = 8;
    bool logits_issued = false;
    if (kRowstat) {
        // Published by the merge (attn_finalize_kernel's merge role). The
        // first 256 heads' statistics and the first block's logits are in
        // flight together; storing the statistics waits for them alone.
        const float2 r0 = *reinterpret_cast<const float2*>(a.rowstat + 2 * (t < Hq ? t : Hq - 1));
        fin_load_logits_nb<MT, NU>(a, hg, wg * MT + 4 * q, n, lgv);
        logits_issued = true;
        if (t < Hq) {
            Mh[t] = r0.x;
            iL[t] = 1.0f / (r0.y > 0.0f ? r0.y : 1.0f);
        }
        for (int h = t + 256; h < Hq; h += 256) {
            const float2 r = *reinterpret_cast<const float2*>(a.rowstat + 2 * h);
            Mh[h] = r.x;
            iL[h] = 1.0f / (r.y > 0.0f ? r.y : 1.0f);
        }
    } else if (NU < 8 && Hq <= 32 && a.nsplit >= 2 && a.nsplit <= 16 * kU4) {
        // one pass, no branches around the loads: pair index j clamped to
        // nsplit - 2 (the float4 then holds split j - 1 and j, or neither)
        const int h = t >> 3, j0 = t & 7;
        const int hc = h < Hq ? h : Hq - 1;
        const float* ml = a.part_ml + static_cast<size_t>(hc) * a.nsplit * 2;
        float4 w[kU4];
#pragma unroll
        for (int u = 0; u < kU4; ++u) {
            const int j = 2 * j0 + 16 * u;
            const int jj = j < a.nsplit - 2 ? j : a.nsplit - 2;
            w[u] = load_ml_pair(ml + 2 * jj);
        }
        fin_load_logits_nb<MT, NU>(a, hg, wg * MT + 4 * q, n, lgv);
        __builtin_amdgcn_sched_barrier(0);  // keep both sets of loads ahead of the fold
        logits_issued = true;
        float2 v[2 * kU4];
#pragma unroll
        for (int u = 0; u < kU4; ++u) {
            const int j = 2 * j0 + 16 * u;
            const int jj = j < a.nsplit - 2 ? j : a.nsplit - 2;
            const float2 lo = make_float2(w[u].x, w[u].y), hi = make_float2(w[u].z, w[u].w);
            const float2 none = make_float2(kNegInf, 0.0f);
            v[2 * u] = (j == jj) ? lo : (j == jj + 1 ? hi : none);
            v[2 * u + 1] = (j == jj && j + 1 < a.nsplit) ? hi : none;
        }
        float mx = kNegInf;
#pragma unroll
        for (int u = 0; u < 2 * kU4; ++u) mx = fmaxf(mx, v[u].x);
        float ls = 0.0f;
#pragma unroll
        for (int u = 0; u < 2 * kU4; ++u)
            ls += (v[u].x == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(v[u].x - mx) * v[u].y;
        const float gm = max8(mx);
        const float gl = sum8((mx == kNegInf) ? 0.0f : ls * __builtin_amdgcn_exp2f(mx - gm));
        if (j0 == 0 && h < Hq) {
            Mh[h] = gm;
            iL[h] = 1.0f / (gl > 0.0f ? gl : 1.0f);
        }
    }
    for (int h0 = 0; !kRowstat && !logits_issued && h0 < Hq; h0 += 32) {
        const int h = h0 + (t >> 3), j0 = t & 7;
        const float* ml = a.part_ml + static_cast<size_t>(h < Hq ? h : 0) * a.nsplit * 2;
        float mx = kNegInf, ls = 0.0f;
        for (int jb = 2 * j0; jb < a.nsplit; jb += 16 * kU4) {
            float2 v[2 * kU4];  // (m, l) of splits jb + 16 u and jb + 16 u + 1
#pragma unroll
            for (int u = 0; u < kU4; ++u) {
                const int j = jb + 16 * u;
                if (j + 1 < a.nsplit) {
                    const float4 w = load_ml_pair(ml + 2 * j);
                    v[2 * u] = make_float2(w.x, w.y);
                    v[2 * u + 1] = make_float2(w.z, w.w);
                } else {
                    v[2 * u] = j < a.nsplit ? *reinterpret_cast<const float2*>(ml + 2 * j) : make_float2(kNegInf, 0.0f);
                    v[2 * u + 1] = make_float2(kNegInf, 0.0f);
                }
            }
            float bm = kNegInf;
#pragma unroll
            for (int u = 0; u < 2 * kU4; ++u) bm = fmaxf(bm, v[u].x);
            const float mn = fmaxf(mx, bm);
            float bs = 0.0f;
            // hardware exp2: arguments <= 0, results below 2^-126 flush to 0
#pragma unroll
            for (int u = 0; u < 2 * kU4; ++u)
                bs += (v[u].x == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(v[u].x - mn) * v[u].y;
            ls = ((mx == kNegInf) ? 0.0f : ls * __builtin_amdgcn_exp2f(mx - mn)) + bs;
            mx = mn;
        }
        const float gm = max8(mx);
        const float gl = sum8((mx == kNegInf) ? 0.0f : ls * __builtin_amdgcn_exp2f(mx - gm));
        if (j0 == 0 && h < Hq) {
            Mh[h] = gm;
            iL[h] = 1.0f / (gl > 0.0f ? gl : 1.0f);
        }
    }
    if (!logits_issued) fin_load_logits_nb<MT, NU>(a, hg, wg * MT + 4 * q, n, lgv);
    __syncthreads();
    float* red = sh + 2 * Hq;  // [kGroups][MT]
    for (int blk = wg; blk * MT < n; blk += nwg) {
        const int tok0 = blk * MT;
        const int i0 = tok0 + 4 * q;
        if (blk != wg && fb_lane) {
            ft = fb_token(tok0 + t);
            g_old = ft.tid >= 0 ? a.fb.g[ft.tid] : 0.0f;
        }
        float w4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (i0 < n) {
            for (int hb = 0; hb < Hq; hb += 8 * kGroups) {
                if (hb > 0) fin_load_logits<MT>(a, hb, hg, i0, n, lgv);  // heads past 8 groups of the first round
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int h = hb + hg + kGroups * u;
                    if (h >= Hq) break;
                    const float sc[4] = {lgv[u].x, lgv[u].y, lgv[u].z, lgv[u].w};
                    const float mh = Mh[h], il = iL[h];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        // s <= M_h, so 2^(s - M_h) <= 1 (flushed to 0 below 2^-126)
                        const float w = (sc[e] == kNegInf || i0 + e >= n)
                                            ? 0.0f
                                            : __builtin_amdgcn_exp2f(sc[e] - mh) * il;
                        w4[e] += w;
                        if (a.head_w && i0 + e < n && i0 + e < a.head_w_ld)
                            a.head_w[static_cast<size_t>(h) * a.head_w_ld + i0 + e] = w;
                    }
                }
            }
        }
        const int nxt = blk + nwg;
        if (nxt * MT < n) fin_load_logits_nb<MT, NU>(a, hg, nxt * MT + 4 * q, n, lgv);
#pragma unroll
        for (int e = 0; e < 4; ++e) red[hg * MT + 4 * q + e] = w4[e];
        __syncthreads();
        const int i = tok0 + t;
        if (t < MT && i < n) {
            float sum = 0.0f;
#pragma unroll
            for (int g = 0; g < kGroups; ++g) sum += red[g * MT + t];
            const float mean = sum / static_cast<float>(Hq);
            if (a.mw) a.mw[i] = mean;
            if (fb_lane && ft.tid >= 0) {
                const float gn = __builtin_fmaf(a.fb.decay, g_old, mean);
                a.fb.g[ft.tid] = gn;
                if (ft.hh_slot >= 0) a.fb.hh_scores[ft.hh_slot] = gn;
            }
        }
        __syncthreads();  // `red` is rewritten by the next block
    }
}

// Logits rows per thread in the first head round of a MT-token block (see
// fin_mean_tokens).
template <int MT>
__host__ __device__ constexpr int fin_rows(const int Hq) {
    constexpr int kGroups = 256 / (MT / 4);
    return Hq <= kGroups ? 1 : Hq <= 2 * kGroups ? 2 : Hq <= 4 * kGroups ? 4 : 8;
}

template <int MT, bool kRowstat>
__device__ __forceinline__ void fin_mean_dispatch(const FinArgs& a, const int wg, const int nwg, float* sh) {
    switch (fin_rows<MT>(a.Hq)) {
    case 1: fin_mean_tokens<MT, kRowstat, 1>(a, wg, nwg, sh); break;
    case 2: fin_mean_tokens<MT, kRowstat, 2>(a, wg, nwg, sh); break;
    case 4: fin_mean_tokens<MT, kRowstat, 4>(a, wg, nwg, sh); break;
    default: fin_mean_tokens<MT, kRowstat, 8>(a, wg, nwg, sh); break;
    }
}

template <int MT>
__global__ void __launch_bounds__(256) attn_finalize_kernel(FinArgs a) {
    extern __shared__ float sh[];
    const int b = static_cast<int>(blockIdx.x);
    const int msl = fin_merge_slices(a.D, a.pair_g, a.nsplit);
    const int merges = a.Hq * msl;
    if (b < merges)
        fin_merge_head(a, b / msl, b % msl, msl, sh);
    else
        fin_mean_dispatch<MT, false>(a, b - merges, static_cast<int>(gridDim.x) - merges, sh);
}

// The merge of one call's partials (workgroups [0, Hq S)) beside the mean
// weights of an earlier merge-only call whose partials, logits and row
// statistics sit in another workspace: a caller that runs layers back to back
// folds each layer's mean weights into the next layer's finalize launch.
template <int MT>
__global__ void __launch_bounds__(256) attn_finalize_deferred_kernel(FinArgs am, FinArgs aw) {
    extern __shared__ float sh[];
    const int b = static_cast<int>(blockIdx.x);
    const int msl = fin_merge_slices(am.D, am.pair_g, am.nsplit);
    const int merges = am.Hq * msl;
    if (b < merges)
        fin_merge_head(am, b / msl, b % msl, msl, sh);
    else
        fin_mean_dispatch<MT, true>(aw, b - merges, static_cast<int>(gridDim.x) - merges, sh);
}

// The mean-weight role alone, after a merge-only finalize of the same
// partials: the per-head (M, L) come from the merge's row statistics.
template <int MT>
__global__ void __launch_bounds__(256) attn_mean_kernel(FinArgs a) {
    extern __shared__ float sh[];
    fin_mean_dispatch<MT, true>(a, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), sh);
}

// ---------------------------------------------------------------------------
// Batched ragged decode (head_dim 128). One launch of the split kernel covers
// many sequences: the partial slots of all of them form one global slot
// range (sequence i owns slots [slot_base[i], slot_base[i + 1])), laid over
// the grid exactly as attn_packed_kernel lays out one sequence's slots, so
// the KV heads of one slot still share an XCD. A workgroup finds its sequence
// by a binary search of the prefix table in the kernel arguments and reads
// that sequence's tier pointers from the caller's device array.

struct BatchArgs {
    const tt_decode_seq* __restrict__ seqs;
    float* ml;
    float* acc;
    float* logits;
    float scale2;
    int nseq, total_slots, Hq, Hkv, kgs, meta_fp16, hc, chunks;
    int slot_base[kMaxBatchSeqs + 1];
    int tok_base[kMaxBatchSeqs + 1];
    int pk_base[kMaxBatchSeqs + 1];  // launch order: packed slots of all sequences, then
    int dn_base[kMaxBatchSeqs + 1];  // their FP32-tier slots
};

// Largest i < n with base[i] <= x (base non-decreasing, base[0] = 0 <= x).
__device__ __forceinline__ int batch_find(const int* base, const int n, const int x) {
    int lo = 0, hi = n;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (base[mid] <= x)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

template <int GP, typename MetaT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GP == 8 ? 3 : 1)))
attn_batched_kernel(const BatchArgs b) {
    constexpr int kLds = MfLds<GP>::TOTAL > DnLds<GP>::TOTAL ? MfLds<GP>::TOTAL : DnLds<GP>::TOTAL;
    __shared__ __align__(16) char lds[kLds];
    const unsigned id = blockIdx.x;
    const unsigned q = id >> 3;
    const int hz = static_cast<int>(q % static_cast<unsigned>(b.hc));
    const int g = static_cast<int>((q / static_cast<unsigned>(b.hc)) * 8 + (id & 7));
    if (g >= b.total_slots) return;  // padding slot of the last group of 8
    // launch slot g -> (sequence i, its split s): the packed slots of all
    // sequences first, then all FP32-tier slots
    const int npk = b.pk_base[b.nseq];
    int i, s;
    if (g < npk) {
        i = batch_find(b.pk_base, b.nseq, g);
        s = g - b.pk_base[i];
    } else {
        i = batch_find(b.dn_base, b.nseq, g - npk);
        s = (b.pk_base[i + 1] - b.pk_base[i]) + (g - npk - b.dn_base[i]);
    }
    const tt_decode_seq& d = b.seqs[i];
    SplitArgs a;
    a.in.Q = d.Q;
    a.in.k0 = d.dense_K;
    a.in.v0 = d.dense_V;
    a.in.n0 = d.dense_count;
    a.in.kp = d.PBS_K_Packed;
    a.in.ks = d.PBS_K_Scales;
    a.in.kz = d.PBS_K_Zeroes;
    a.in.vp = d.PBS_V_Packed;
    a.in.vs = d.PBS_V_Scales;
    a.in.vz = d.PBS_V_Zeroes;
    a.in.ids = d.PBS_token_ids;
    a.in.num_blocks = d.num_blocks;
    a.in.Hq = b.Hq;
    a.in.Hkv = b.Hkv;
    a.in.D = kMfD;
    a.in.kgs = b.kgs;
    a.in.meta_fp16 = b.meta_fp16;
    a.scale2 = b.scale2;
    a.part_ml = b.ml + static_cast<size_t>(b.slot_base[i]) * b.Hq * 2;
    a.part_acc = b.acc + static_cast<size_t>(b.slot_base[i]) * b.Hq * kMfD;
    a.logits = d.mean_attn_weights ? b.logits + static_cast<size_t>(b.tok_base[i]) * b.Hq : nullptr;
    a.ld = b.tok_base[i + 1] - b.tok_base[i];
    a.nsplit = b.slot_base[i + 1] - b.slot_base[i];
    a.nsplit_p = b.pk_base[i + 1] - b.pk_base[i];
    a.nsplit_d = a.nsplit - a.nsplit_p;
    a.wd = 8;
    a.wp = 1;
    a.dense_delay = 0;
    const int kvh = hz / b.chunks, chunk = hz - kvh * b.chunks;
    if (s >= a.nsplit_p) {
        dense_body<GP>(a, s - a.nsplit_p, kvh, chunk, lds);
        return;
    }
    packed_body<GP, MetaT>(a, s, kvh, chunk, lds);
}

struct FinBatchArgs {
    const tt_decode_seq* __restrict__ seqs;
    const float* ml;
    const float* acc;
    const float* logits;
    float* rowstat;
    int nseq, Hq, kgs;
    int msl;  // merge workgroups per (sequence, query head)
    int slot_base[kMaxBatchSeqs + 1];
    int tok_base[kMaxBatchSeqs + 1];
    int mean_base[kMaxBatchSeqs + 1];
};

__device__ __forceinline__ FinArgs fin_batch_args(const FinBatchArgs& b, const int i) {
    const tt_decode_seq& d = b.seqs[i];
    FinArgs a;
    a.part_ml = b.ml + static_cast<size_t>(b.slot_base[i]) * b.Hq * 2;
    a.part_acc = b.acc + static_cast<size_t>(b.slot_base[i]) * b.Hq * kMfD;
    a.nsplit = b.slot_base[i + 1] - b.slot_base[i];
    a.D = kMfD;
    a.Hq = b.Hq;
    a.pair_g = 0;
    a.out = d.attn_output;
    a.rowstat = b.rowstat + static_cast<size_t>(i) * 2 * b.Hq;
    a.logits = d.mean_attn_weights ? b.logits + static_cast<size_t>(b.tok_base[i]) * b.Hq : nullptr;
    a.ld = b.tok_base[i + 1] - b.tok_base[i];
    a.n_static = d.dense_count + d.num_blocks * b.kgs;
    a.state = nullptr;
    a.kgs = b.kgs;
    a.mw = d.mean_attn_weights;
    a.head_w = nullptr;
    a.head_w_ld = 0;
    a.fb = Feedback{};
    return a;
}

// Workgroups [0, nseq Hq S): the merge of (sequence, query head, channel
// slice); the rest:
// mean weights, sequence i owning [mean_base[i], mean_base[i + 1]).
__global__ void __launch_bounds__(256) attn_finalize_batched_kernel(const FinBatchArgs b) {
    extern __shared__ float sh[];
    const int blk = static_cast<int>(blockIdx.x);
    const int msl = b.msl;
    const int merges = b.nseq * b.Hq * msl;
    if (blk < merges) {
        const int i = blk / (b.Hq * msl);
        const FinArgs a = fin_batch_args(b, i);
        const int r = blk - i * b.Hq * msl;
        fin_merge_head(a, r / msl, r % msl, msl, sh);
        return;
    }
    const int m = blk - merges;
    const int i = batch_find(b.mean_base, b.nseq, m);
    const FinArgs a = fin_batch_args(b, i);
    fin_mean_dispatch<kMeanTokens, false>(a, m - b.mean_base[i], b.mean_base[i + 1] - b.mean_base[i], sh);
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

// Grid of attn_packed_kernel: ceil(nsplit / 8) groups of 8 slots for each
// (KV head, head chunk).
template <int GP, bool PAIR = false>
int launch_packed_meta(const SplitArgs& a, int Hkv, int chunks, int meta_fp16, hipStream_t st) {
    const int hc = Hkv * chunks;
    const long long wgs = static_cast<long long>((a.nsplit + 7) / 8) * 8 * hc;
    if (wgs > 0x7fffffffLL) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "attention grid too large");
    const dim3 grid(static_cast<unsigned>(wgs));
    if (meta_fp16)
        hipLaunchKernelGGL((attn_packed_kernel<GP, uint16_t, PAIR>), grid, dim3(256), 0, st, a, hc, chunks);
    else
        hipLaunchKernelGGL((attn_packed_kernel<GP, float, PAIR>), grid, dim3(256), 0, st, a, hc, chunks);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

// Paired head_dim-64 heads form groups of 2 G query heads: 2, 4 or 8 per
// workgroup (G = 1, 2, 4, or 8 and more in chunks of 8).
int launch_packed(const SplitArgs& a, int Hkv, int chunks, int gp, int meta_fp16, bool pair, hipStream_t st) {
    if (pair) {
        switch (gp) {
        case 2: return launch_packed_meta<2, true>(a, Hkv, chunks, meta_fp16, st);
        case 4: return launch_packed_meta<4, true>(a, Hkv, chunks, meta_fp16, st);
        default: return launch_packed_meta<8, true>(a, Hkv, chunks, meta_fp16, st);
        }
    }
    switch (gp) {
    case 1: return launch_packed_meta<1>(a, Hkv, chunks, meta_fp16, st);
    case 2: return launch_packed_meta<2>(a, Hkv, chunks, meta_fp16, st);
    case 4: return launch_packed_meta<4>(a, Hkv, chunks, meta_fp16, st);
    default: return launch_packed_meta<8>(a, Hkv, chunks, meta_fp16, st);
    }
}

template <int GP>
int launch_batched_meta(const BatchArgs& b, unsigned wgs, int meta_fp16, hipStream_t st) {
    if (meta_fp16)
        hipLaunchKernelGGL((attn_batched_kernel<GP, uint16_t>), dim3(wgs), dim3(256), 0, st, b);
    else
        hipLaunchKernelGGL((attn_batched_kernel<GP, float>), dim3(wgs), dim3(256), 0, st, b);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int gp_for(int G) { return G >= 8 ? 8 : (G > 4 ? 8 : (G > 2 ? 4 : G)); }


template <typename MetaT>
const void* packed_kernel_ptr(int gp, bool pair) {
    if (pair) {
        switch (gp) {
        case 2: return reinterpret_cast<const void*>(&attn_packed_kernel<2, MetaT, true>);
        case 4: return reinterpret_cast<const void*>(&attn_packed_kernel<4, MetaT, true>);
        default: return reinterpret_cast<const void*>(&attn_packed_kernel<8, MetaT, true>);
        }
    }
    switch (gp) {
    case 1: return reinterpret_cast<const void*>(&attn_packed_kernel<1, MetaT>);
    case 2: return reinterpret_cast<const void*>(&attn_packed_kernel<2, MetaT>);
    case 4: return reinterpret_cast<const void*>(&attn_packed_kernel<4, MetaT>);
    default: return reinterpret_cast<const void*>(&attn_packed_kernel<8, MetaT>);
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

// CUs of the device and workgroups of the split launch one CU holds at once
// (queried once per device and shape, then cached).
struct Residency {
    int cus = 256;
    int per_cu = 2;
};

Residency split_residency(int D, int G, int fp16, bool pair = false) {
    static std::mutex mu;
    static std::map<std::tuple<int, int, int, int, int>, Residency> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return Residency{};
    const int gp = gp_for(G);
    const auto key = std::make_tuple(dev, D, gp, fp16, pair ? 1 : 0);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    const void* fn = nullptr;
    if (use_packed_kernel(D)) {
        fn = fp16 ? packed_kernel_ptr<uint16_t>(gp, pair) : packed_kernel_ptr<float>(gp, pair);
    } else {
        // the instantiation the launch runs (channels per lane = head_dim / 16)
        switch (D / 16) {
        case 1: fn = split_kernel_ptr<1>(gp, fp16); break;
        case 2: fn = split_kernel_ptr<2>(gp, fp16); break;
        case 3: fn = split_kernel_ptr<3>(gp, fp16); break;
        case 4: fn = split_kernel_ptr<4>(gp, fp16); break;
        case 5: fn = split_kernel_ptr<5>(gp, fp16); break;
        case 6: fn = split_kernel_ptr<6>(gp, fp16); break;
        case 7: fn = split_kernel_ptr<7>(gp, fp16); break;
        case 8: fn = split_kernel_ptr<8>(gp, fp16); break;
        case 9: fn = split_kernel_ptr<9>(gp, fp16); break;
        case 10: fn = split_kernel_ptr<10>(gp, fp16); break;
        case 11: fn = split_kernel_ptr<11>(gp, fp16); break;
        case 12: fn = split_kernel_ptr<12>(gp, fp16); break;
        case 13: fn = split_kernel_ptr<13>(gp, fp16); break;
        case 14: fn = split_kernel_ptr<14>(gp, fp16); break;
        case 15: fn = split_kernel_ptr<15>(gp, fp16); break;
        default: fn = split_kernel_ptr<16>(gp, fp16); break;
        }
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0) != hipSuccess || per_cu <= 0) {
        (void)hipGetLastError();
        per_cu = 2;
    }
    const Residency r{cus, per_cu};
    cache[key] = r;
    return r;
}

}  // namespace

// The matrix-core path serves head_dim 128 with either block size.
bool use_packed_kernel(int D) { return D == kMfD; }

int attn_check_shapes(int Hq, int Hkv, int D, int kgs) {
    if (Hq <= 0 || Hkv <= 0 || D <= 0)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_q_heads, num_kv_heads, and head_dim must be positive integers.");
    if (Hq % Hkv != 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_q_heads must be a multiple of num_kv_heads.");
    if (D % 16 != 0 || D > 256)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "head_dim must be a multiple of 16, at most 256.");
    if (kgs != 16 && kgs != 32) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "k_group_size must be 16 or 32.");
    return TT_OK;
}

namespace {
AttnPlan attn_plan_impl(int dense_ub, int blocks_ub, int Hq, int Hkv, int D, int kgs, bool need_logits,
                        int meta_fp16, bool pair);
}  // namespace

// Head_dim 64 with an even number of KV heads runs as half as many heads of
// head_dim 128 on the matrix-core kernel: KV heads 2j and 2j + 1 sit next to
// each other in every tier (K words and scale / zero per block, V words per
// token, FP32 rows), so they read like one head of 128 channels, and the
// query heads of both form one group whose queries fill the half of their own
// head (zeros in the other half), which leaves their logits exact.
AttnPlan attn_plan(int dense_ub, int blocks_ub, int Hq, int Hkv, int D, int kgs, bool need_logits, int meta_fp16) {
    if (D == 64 && Hkv % 2 == 0) {
        AttnPlan p = attn_plan_impl(dense_ub, blocks_ub, Hq, Hkv / 2, kMfD, kgs, need_logits, meta_fp16, true);
        p.pair64 = true;
        return p;
    }
    return attn_plan_impl(dense_ub, blocks_ub, Hq, Hkv, D, kgs, need_logits, meta_fp16, false);
}

namespace {
AttnPlan attn_plan_impl(int dense_ub, int blocks_ub, int Hq, int Hkv, int D, int kgs, bool need_logits,
                        int meta_fp16, bool pair) {
    AttnPlan p;
    const int W = kgs / 16;
    const int G = Hq / Hkv;
    const int chunks = (G + gp_for(G) - 1) / gp_for(G);
    const long long heads = static_cast<long long>(Hkv) * chunks;
    const Residency res = split_residency(D, G, meta_fp16, pair);
    const long long resident = static_cast<long long>(res.cus) * res.per_cu;
    const long long per_head = std::max<long long>(1, (resident + heads - 1) / heads);
    const long long dense_tiles = (dense_ub + 15) / 16;
    if (use_packed_kernel(D)) {
        // One resident round of workgroups per head, at least ~4 units of work
        // each so the partials stay small (a 32-token pair of packed tiles is
        // one unit, a 16-token FP32 tile kDenseTileCost), shared between
        // packed and FP32 workgroups in proportion to their work. (With ~8
        // units as the bar for the whole-round layout, 32/8 heads at 8k and
        // 12k took 8.9 and 10.3 us per launch against 8.5 and 9.9.)
        //
        // When the launch fills the device, each kind gets whole dispatch
        // rounds (one workgroup per CU each): the kernel's workgroup order
        // sends slot groups of every head to the XCDs round-robin, so a round
        // of `cus / heads` slots lands one workgroup on every CU, and every CU
        // then runs the same mix of packed and FP32 work.
        constexpr long long kDenseTileCost = 4;  // ~3.7x the bytes of a pair
        const long long pairs = (static_cast<long long>(blocks_ub) * W + 1) / 2;
        const long long dense_units = dense_tiles * kDenseTileCost;
        const long long units = pairs + dense_units;
        const long long round = (res.cus % heads == 0) ? res.cus / heads : 0;  // slots per dispatch round
        if (round > 0 && round % 8 == 0 && res.per_cu >= 2 && units / 4 >= round * res.per_cu) {
            long long rd = 0;
            if (dense_tiles > 0) {
                rd = (res.per_cu * dense_units + units / 2) / units;
                rd = std::max<long long>(1, std::min<long long>(rd, res.per_cu - 1));
            }
            p.nsplit_d = static_cast<int>(std::min(rd * round, dense_tiles));
            p.nsplit_p = static_cast<int>((res.per_cu - rd) * round);
        } else {
            // Without whole dispatch rounds (the heads do not divide the CUs
            // into groups of 8 slots), whole groups of 8 slots per head (slot
            // s runs on XCD s % 8, so a padded group leaves its XCDs
            // unevenly loaded): the per-head share rounded up to a multiple
            // of 8, which may leave a second round of (short, FP32-tier)
            // workgroups to start as the first ones finish, unless those
            // would wait before their first load (see below): then as many
            // groups as every XCD holds at once. Per launch: 40/40 heads at
            // 8k context 23.1 us with 24 slots per head against 25.2 with 20;
            // 40/10 heads at 16k 13.8 with 72 against 20.7 with 77 and 21.3
            // with 80 (the share rounded up, whose late FP32-tier workgroups
            // would then wait).
            auto split = [&](const long long w, long long& np, long long& nd) {
                nd = 0;
                if (dense_tiles > 0) {
                    nd = (w * dense_units + units / 2) / units;
                    nd = std::max<long long>(1, std::min(nd, dense_tiles));
                }
                np = std::max<long long>(1, w - nd);
            };
            auto waits = [&](const long long np, const long long nd) {
                const long long tp = (pairs + 4LL * np - 1) / (4LL * np);
                const long long td = nd > 0 ? (dense_tiles + 4LL * nd - 1) / (4LL * nd) : 0;
                return td > 0 && tp >= 3 * td;
            };
            // (short contexts: at least ~4 work units per slot; with 8, 32/8
            // heads at 4k took 8.0 us per launch against 7.3, at 2k 7.9
            // against 7.1, 28/4 heads at 8k 8.6 against 7.7)
            const long long share = std::max<long long>(1, std::min(per_head, units / 4));
            long long np, nd;
            split(share >= 8 ? (share + 7) / 8 * 8 : share, np, nd);
            const long long fit = 8 * (resident / (8 * heads));
            if (waits(np, nd) && fit > 0 && np + nd > fit) split(std::min(fit, share), np, nd);
            p.nsplit_d = static_cast<int>(nd);
            p.nsplit_p = static_cast<int>(np);
        }
        // The FP32 workgroups' first tiles, requested at the start, compete
        // with the packed waves' first pairs. When a packed wave has at least
        // three times the work items of an FP32 wave, the FP32 workgroups wait
        // about the time the first pairs take to arrive at 1.9 TB/s (at most
        // 5.5 us) before their first tile load; they still finish within the
        // packed waves' time. (At the 32k Llama-3-8B shape: 4.97 us; 3.8, 6.5
        // and 8 us measured 2.5%, 2.5% and 10% slower per launch.)
        const long long tp = (pairs + 4LL * p.nsplit_p - 1) / (4LL * p.nsplit_p);
        const long long td = p.nsplit_d > 0 ? (dense_tiles + 4LL * p.nsplit_d - 1) / (4LL * p.nsplit_d) : 0;
        if (td > 0 && tp >= 3 * td) {
            const long long m = meta_fp16 ? 2 : 4;
            const long long pair_bytes = 2 * (512 + 256 * m / W + 512 + 32 * m + 128);
            const long long burst = std::min(pairs, 4LL * p.nsplit_p) * heads * pair_bytes;
            p.dense_delay = static_cast<int>(std::min<long long>(550, burst / 19000));
        }
    } else {
        // One round of resident workgroups, two when four or more fit on a
        // CU (head_dim up to ~128 at one or two heads per group), with at
        // least ~8 packed-tile units of work per workgroup and round: the
        // loop is arithmetic-bound, and fewer, longer workgroups left CUs
        // idle. Per launch: head_dim 256 with 16/8 heads at 8k context (two
        // workgroups per CU) 20.9 us against 35.9 with ~32 units per
        // workgroup and 24.6 with two rounds; head_dim 80 with 32/32 heads at
        // 2k (five per CU) 11.2 against 18.2 and 12.8 (one round); head_dim 96
        // with 32/32 heads at 4k (four per CU) 17.0 against 23.1 (one round);
        // head_dim 64 with 12/3 heads at 8k 9.5 against 10.6 (one round).
        const long long units = dense_tiles * 8 + static_cast<long long>(blocks_ub) * W;
        const long long rounds = res.per_cu >= 4 ? 2 : 1;
        const long long cap = std::max<long long>(1, units * rounds / 8);
        p.nsplit_p = 0;
        p.nsplit_d = static_cast<int>(std::max<long long>(1, std::min(rounds * per_head, cap)));
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
}  // namespace

int attn_launch_split(const AttnInputs& real_in, const AttnPlan& plan, void* ws, hipStream_t stream) {
    if (plan.logits && !logits_fit(real_in.Hq, plan.ld))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_q_heads x tokens exceeds the 4 GiB logits buffer of the mean weights.");
    // paired head_dim-64 heads: the kernel sees half as many heads of 128 channels
    AttnInputs in = real_in;
    if (plan.pair64) {
        in.D = kMfD;
        in.Hkv = real_in.Hkv / 2;
    }
    char* base = static_cast<char*>(ws);
    SplitArgs a;
    a.in = in;
    a.scale2 = kLog2e / sqrtf(static_cast<float>(real_in.D));
    a.part_ml = reinterpret_cast<float*>(base + plan.off_ml);
    a.part_acc = reinterpret_cast<float*>(base + plan.off_acc);
    a.logits = plan.logits ? reinterpret_cast<float*>(base + plan.off_logits) : nullptr;
    a.ld = plan.ld;
    a.nsplit = plan.nsplit;
    a.nsplit_p = plan.nsplit_p;
    a.nsplit_d = plan.nsplit_d;
    a.wd = 8;
    a.wp = 1;
    a.dense_delay = plan.dense_delay;
    const int G = in.Hq / in.Hkv;
    const int gp = gp_for(G);
    const int chunks = (G + gp - 1) / gp;
    if (use_packed_kernel(in.D)) {
        if (plan.nsplit_p <= 0) TT_FAIL(TT_ERR_RUNTIME, "attention plan does not match head_dim");
        return launch_packed(a, in.Hkv, chunks, gp, in.meta_fp16, plan.pair64, stream);
    }
    const dim3 grid(plan.nsplit, in.Hkv, chunks);
    if (plan.nsplit_p != 0) TT_FAIL(TT_ERR_RUNTIME, "attention plan does not match head_dim");
    switch (in.D / 16) {
    case 1: return launch_split_g<1>(a, grid, gp, in.meta_fp16, stream);
    case 2: return launch_split_g<2>(a, grid, gp, in.meta_fp16, stream);
    case 3: return launch_split_g<3>(a, grid, gp, in.meta_fp16, stream);
    case 4: return launch_split_g<4>(a, grid, gp, in.meta_fp16, stream);
    case 5: return launch_split_g<5>(a, grid, gp, in.meta_fp16, stream);
    case 6: return launch_split_g<6>(a, grid, gp, in.meta_fp16, stream);
    case 7: return launch_split_g<7>(a, grid, gp, in.meta_fp16, stream);
    case 8: return launch_split_g<8>(a, grid, gp, in.meta_fp16, stream);
    case 9: return launch_split_g<9>(a, grid, gp, in.meta_fp16, stream);
    case 10: return launch_split_g<10>(a, grid, gp, in.meta_fp16, stream);
    case 11: return launch_split_g<11>(a, grid, gp, in.meta_fp16, stream);
    case 12: return launch_split_g<12>(a, grid, gp, in.meta_fp16, stream);
    case 13: return launch_split_g<13>(a, grid, gp, in.meta_fp16, stream);
    case 14: return launch_split_g<14>(a, grid, gp, in.meta_fp16, stream);
    case 15: return launch_split_g<15>(a, grid, gp, in.meta_fp16, stream);
    default: return launch_split_g<16>(a, grid, gp, in.meta_fp16, stream);
    }
}

namespace {
FinArgs fin_args(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out, float* mean_w, const Feedback* fb,
                 float* head_w, int head_w_ld) {
    char* base = static_cast<char*>(ws);
    FinArgs f;
    f.part_ml = reinterpret_cast<const float*>(base + plan.off_ml);
    f.part_acc = reinterpret_cast<const float*>(base + plan.off_acc);
    f.nsplit = plan.nsplit;
    f.D = plan.pair64 ? kMfD : in.D;
    f.pair_g = plan.pair64 ? in.Hq / in.Hkv : 0;
    f.Hq = in.Hq;
    f.out = out;
    f.rowstat = reinterpret_cast<float*>(base + plan.off_rowstat);
    const bool weights = plan.logits && (mean_w || head_w || (fb && fb->g));
    f.logits = weights ? reinterpret_cast<const float*>(base + plan.off_logits) : nullptr;
    f.ld = plan.ld;
    f.n_static = in.n0 + in.n1 + in.n2 + in.num_blocks * in.kgs;
    f.state = in.state;
    f.kgs = in.kgs;
    f.mw = mean_w;
    f.head_w = head_w;
    f.head_w_ld = head_w_ld;
    f.fb = fb ? *fb : Feedback{};
    return f;
}

int fin_mean_tokens_per_block(const AttnPlan& plan) {
    return plan.token_ub >= kMeanLongFrom ? kMeanTokensLong : kMeanTokens;
}

// Mean-weight workgroups of a plan (0 without weights).
int fin_mean_wgs(const AttnPlan& plan, const bool weights) {
    if (!weights) return 0;
    const int mt = fin_mean_tokens_per_block(plan);
    const int blocks = (std::max(plan.token_ub, 1) + mt - 1) / mt;
    const int per_wg = (blocks + kMeanMaxWgs - 1) / kMeanMaxWgs;
    return (blocks + per_wg - 1) / per_wg;
}

size_t fin_lds_bytes(const int Hq) {
    return sizeof(float) * std::max<size_t>(8 + 4 * 256, 2 * static_cast<size_t>(Hq) + 256 * 4);
}
}  // namespace

int attn_launch_finalize(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out, float* mean_w,
                         const Feedback* fb, float* head_w, int head_w_ld, hipStream_t stream, FinRoles roles) {
    const FinArgs f = fin_args(in, plan, ws, out, mean_w, fb, head_w, head_w_ld);
    const bool weights = f.logits != nullptr;
    const int mt = fin_mean_tokens_per_block(plan);
    const int mean_wgs = fin_mean_wgs(plan, weights && roles != FinRoles::kMerge);
    const size_t lds = fin_lds_bytes(in.Hq);
    const int merges = in.Hq * fin_merge_slices(f.D, f.pair_g, f.nsplit);
    if (roles == FinRoles::kMean) {
        if (mean_wgs == 0) return TT_OK;
        if (mt == kMeanTokensLong)
            hipLaunchKernelGGL(attn_mean_kernel<kMeanTokensLong>, dim3(mean_wgs), dim3(256), lds, stream, f);
        else
            hipLaunchKernelGGL(attn_mean_kernel<kMeanTokens>, dim3(mean_wgs), dim3(256), lds, stream, f);
    } else if (mt == kMeanTokensLong) {
        hipLaunchKernelGGL(attn_finalize_kernel<kMeanTokensLong>, dim3(merges + mean_wgs), dim3(256), lds, stream, f);
    } else {
        hipLaunchKernelGGL(attn_finalize_kernel<kMeanTokens>, dim3(merges + mean_wgs), dim3(256), lds, stream, f);
    }
    TT_LAUNCH_CHECK();
    return TT_OK;
}

int attn_launch_finalize_deferred(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out,
                                  const AttnInputs& prev_in, const AttnPlan& prev_plan, void* prev_ws,
                                  float* prev_mean_w, const Feedback* prev_fb, hipStream_t stream) {
    const FinArgs am = fin_args(in, plan, ws, out, nullptr, nullptr, nullptr, 0);
    const FinArgs aw = fin_args(prev_in, prev_plan, prev_ws, nullptr, prev_mean_w, prev_fb, nullptr, 0);
    if (!aw.logits) TT_FAIL(TT_ERR_RUNTIME, "deferred mean weights without logits in the earlier workspace");
    const int mean_wgs = fin_mean_wgs(prev_plan, true);
    const size_t lds = std::max(fin_lds_bytes(in.Hq), fin_lds_bytes(prev_in.Hq));
    const int merges = in.Hq * fin_merge_slices(am.D, am.pair_g, am.nsplit);
    if (fin_mean_tokens_per_block(prev_plan) == kMeanTokensLong)
        hipLaunchKernelGGL(attn_finalize_deferred_kernel<kMeanTokensLong>, dim3(merges + mean_wgs), dim3(256), lds,
                           stream, am, aw);
    else
        hipLaunchKernelGGL(attn_finalize_deferred_kernel<kMeanTokens>, dim3(merges + mean_wgs), dim3(256), lds,
                           stream, am, aw);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

int attn_launch(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out, float* mean_w, const Feedback* fb,
                float* head_w, int head_w_ld, hipStream_t stream) {
    int rc = attn_launch_split(in, plan, ws, stream);
    if (rc != TT_OK) return rc;
    return attn_launch_finalize(in, plan, ws, out, mean_w, fb, head_w, head_w_ld, stream);
}

BatchPlan batch_plan(const tt_decode_seq* seqs, int nseq, int Hq, int Hkv, int D, int kgs, int meta_fp16) {
    BatchPlan p;
    p.nseq = nseq;
    const int W = kgs / 16;
    const int G = Hq / Hkv;
    const int gp = gp_for(G);
    const long long heads = static_cast<long long>(Hkv) * ((G + gp - 1) / gp);
    const Residency res = split_residency(D, G, meta_fp16);
    // Slots per head that fill the device once; fewer when the batch is small
    // (at least ~8 units of work per slot, as for one sequence).
    const long long round = std::max<long long>(1, static_cast<long long>(res.cus) * res.per_cu / heads);
    constexpr long long kDenseTileCost = 4;
    constexpr long long kBatchSlotUnits = 40;  // work units per slot below which another round does not pay
    long long units[kMaxBatchSeqs], dunits[kMaxBatchSeqs], total = 0, mean_blocks = 0;
    for (int i = 0; i < nseq; ++i) {
        const long long pairs = (static_cast<long long>(seqs[i].num_blocks) * W + 1) / 2;
        dunits[i] = (static_cast<long long>(seqs[i].dense_count) + 15) / 16 * kDenseTileCost;
        units[i] = pairs + dunits[i];
        total += units[i];
        if (seqs[i].mean_attn_weights)
            mean_blocks += (static_cast<long long>(seqs[i].dense_count) + static_cast<long long>(seqs[i].num_blocks) * kgs +
                            kMeanTokens - 1) / kMeanTokens;
    }
    const long long target = std::max<long long>(1, std::min<long long>(round, total / 8));
    const long long per_wg = std::max<long long>(1, (mean_blocks + kMeanMaxWgs - 1) / kMeanMaxWgs);
    // Per sequence: packed slots np[i] (at least one) and FP32-tier slots
    // nd[i] (at most one per tile), sized to the work rather than rounded
    // from each sequence's fraction of it (with a few slots per sequence,
    // rounding left slots up to 40% above the mean). `cap` is the work units a
    // slot may carry; the smallest cap whose slots fit in `budget` is found
    // by bisection.
    long long np[kMaxBatchSeqs], nd[kMaxBatchSeqs];
    auto packed_slots = [&](const int i, const long long cap) {
        return std::max<long long>(1, (units[i] - dunits[i] + cap - 1) / cap);
    };
    auto dense_slots = [&](const int i, const long long cap) {
        const long long dtiles = dunits[i] / kDenseTileCost;
        return dtiles > 0 ? std::min(dtiles, std::max<long long>(1, (dunits[i] + cap - 1) / cap)) : 0LL;
    };
    auto min_cap = [&](const long long budget, auto&& slots_at) {
        long long lo = 1, hi = 1;
        for (int i = 0; i < nseq; ++i) hi = std::max(hi, units[i]);
        if (slots_at(hi) > budget) return hi;  // one slot per sequence and kind is already over
        while (lo < hi) {
            const long long mid = lo + (hi - lo) / 2;
            if (slots_at(mid) <= budget)
                hi = mid;
            else
                lo = mid + 1;
        }
        return hi;
    };
    long long total_d = 0;
    for (int i = 0; i < nseq; ++i) total_d += dunits[i];
    const long long per_round = (res.cus % heads == 0) ? res.cus / heads : 0;  // slots of one dispatch round
    // Resident rounds of workgroups the batch's work fills at about kBatchSlotUnits units per slot (at most 3)
    const long long rounds = std::min<long long>(3, total / (kBatchSlotUnits * round));
    auto one_cap = [&](const long long budget) {
        const long long c = min_cap(budget, [&](const long long cc) {
            long long n = 0;
            for (int i = 0; i < nseq; ++i) n += packed_slots(i, cc) + dense_slots(i, cc);
            return n;
        });
        for (int i = 0; i < nseq; ++i) {
            np[i] = packed_slots(i, c);
            nd[i] = dense_slots(i, c);
        }
    };
    if (rounds >= 2) {
        // Several resident rounds under one cap: a slot is a fraction of a
        // sequence, and workgroups that finish early hand their CU to the
        // next ones, which evens out what the per-sequence slot counts cannot
        // (16 sequences of 5k-32k tokens, 32/8 heads: 3.71-3.73 ms per step
        // with three rounds, 3.87 with two, 4.05-4.09 with the one-round plan
        // below, 3.91 with four).
        one_cap(rounds * round);
    } else if (per_round > 0 && res.per_cu >= 2 && total_d > 0 && total / 8 >= per_round * res.per_cu) {
        // The device filled once, each kind in whole dispatch rounds (one
        // workgroup per CU each), as for one sequence: every CU runs the same
        // mix of packed and FP32-tier work. (16 sequences of 5k-32k tokens,
        // 32/8 heads: 4.06-4.12 against 4.62-4.67 ms per 32-layer step; the
        // per-sequence caps alone 4.47-4.55.)
        long long rd = (res.per_cu * total_d + total / 2) / total;
        rd = std::max<long long>(1, std::min<long long>(rd, res.per_cu - 1));
        const long long cp = min_cap((res.per_cu - rd) * per_round, [&](const long long c) {
            long long n = 0;
            for (int i = 0; i < nseq; ++i) n += packed_slots(i, c);
            return n;
        });
        const long long cd = min_cap(rd * per_round, [&](const long long c) {
            long long n = 0;
            for (int i = 0; i < nseq; ++i) n += dense_slots(i, c);
            return n;
        });
        for (int i = 0; i < nseq; ++i) {
            np[i] = packed_slots(i, cp);
            nd[i] = dense_slots(i, cd);
        }
    } else {
        one_cap(target);
    }
    long long slot = 0, tok = 0, mean = 0, pk = 0, dn = 0;
    for (int i = 0; i < nseq; ++i) {
        p.slot_base[i] = static_cast<int>(slot);
        p.pk_base[i] = static_cast<int>(pk);
        p.dn_base[i] = static_cast<int>(dn);
        slot += np[i] + nd[i];
        pk += np[i];
        dn += nd[i];
        p.tok_base[i] = static_cast<int>(tok);
        p.mean_base[i] = static_cast<int>(mean);
        if (seqs[i].mean_attn_weights) {
            const long long tub = static_cast<long long>(seqs[i].dense_count) + static_cast<long long>(seqs[i].num_blocks) * kgs;
            tok += (tub + 3) & ~3LL;
            mean += ((tub + kMeanTokens - 1) / kMeanTokens + per_wg - 1) / per_wg;
        }
    }
    p.pk_base[nseq] = static_cast<int>(pk);
    p.dn_base[nseq] = static_cast<int>(dn);
    p.slot_base[nseq] = static_cast<int>(slot);
    p.tok_base[nseq] = static_cast<int>(tok);
    p.mean_base[nseq] = static_cast<int>(mean);
    p.total_slots = static_cast<int>(slot);
    size_t off = 0;
    p.off_ml = off;
    off = align256(off + sizeof(float) * 2 * static_cast<size_t>(Hq) * slot);
    p.off_acc = off;
    off = align256(off + sizeof(float) * static_cast<size_t>(Hq) * slot * D);
    p.off_rowstat = off;
    off = align256(off + sizeof(float) * 2 * static_cast<size_t>(Hq) * std::max(nseq, 1));
    p.off_logits = off;
    off = align256(off + sizeof(float) * static_cast<size_t>(Hq) * std::max<long long>(tok, 4));
    p.bytes = off;
    return p;
}

int batch_launch(const BatchPlan& plan, const tt_decode_seq* seqs_dev, int Hq, int Hkv, int kgs, int meta_fp16,
                 void* ws, hipStream_t stream) {
    if (plan.nseq <= 0) return TT_OK;
    char* base = static_cast<char*>(ws);
    const int G = Hq / Hkv;
    const int gp = gp_for(G);
    const int chunks = (G + gp - 1) / gp;
    BatchArgs b;
    b.seqs = seqs_dev;
    b.ml = reinterpret_cast<float*>(base + plan.off_ml);
    b.acc = reinterpret_cast<float*>(base + plan.off_acc);
    b.logits = reinterpret_cast<float*>(base + plan.off_logits);
    b.scale2 = kLog2e / sqrtf(static_cast<float>(kMfD));
    b.nseq = plan.nseq;
    b.total_slots = plan.total_slots;
    b.Hq = Hq;
    b.Hkv = Hkv;
    b.kgs = kgs;
    b.meta_fp16 = meta_fp16 ? 1 : 0;
    b.hc = Hkv * chunks;
    b.chunks = chunks;
    std::memcpy(b.slot_base, plan.slot_base, sizeof(b.slot_base));
    std::memcpy(b.tok_base, plan.tok_base, sizeof(b.tok_base));
    std::memcpy(b.pk_base, plan.pk_base, sizeof(b.pk_base));
    std::memcpy(b.dn_base, plan.dn_base, sizeof(b.dn_base));
    const long long wgs = static_cast<long long>((plan.total_slots + 7) / 8) * 8 * b.hc;
    if (wgs > 0x7fffffffLL) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "attention grid too large");
    int rc = TT_OK;
    switch (gp) {
    case 1: rc = launch_batched_meta<1>(b, static_cast<unsigned>(wgs), meta_fp16, stream); break;
    case 2: rc = launch_batched_meta<2>(b, static_cast<unsigned>(wgs), meta_fp16, stream); break;
    case 4: rc = launch_batched_meta<4>(b, static_cast<unsigned>(wgs), meta_fp16, stream); break;
    default: rc = launch_batched_meta<8>(b, static_cast<unsigned>(wgs), meta_fp16, stream); break;
    }
    if (rc) return rc;
    FinBatchArgs f;
    f.seqs = seqs_dev;
    f.ml = b.ml;
    f.acc = b.acc;
    f.logits = b.logits;
    f.rowstat = reinterpret_cast<float*>(base + plan.off_rowstat);
    f.nseq = plan.nseq;
    f.Hq = Hq;
    f.kgs = kgs;
    int max_split = 1;
    for (int i = 0; i < plan.nseq; ++i) max_split = std::max(max_split, plan.slot_base[i + 1] - plan.slot_base[i]);
    f.msl = fin_merge_slices(kMfD, 0, max_split);
    std::memcpy(f.slot_base, plan.slot_base, sizeof(f.slot_base));
    std::memcpy(f.tok_base, plan.tok_base, sizeof(f.tok_base));
    std::memcpy(f.mean_base, plan.mean_base, sizeof(f.mean_base));
    const size_t lds = sizeof(float) * std::max<size_t>(8 + 4 * 256, 2 * static_cast<size_t>(Hq) + 256 * 4);
    const long long fwgs = static_cast<long long>(plan.nseq) * Hq * f.msl + plan.mean_base[plan.nseq];
    hipLaunchKernelGGL(attn_finalize_batched_kernel, dim3(static_cast<unsigned>(fwgs)), dim3(256), lds, stream, f);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

}  // namespace tt
