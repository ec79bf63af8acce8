// tt_attn_mfma.h -- matrix-core tile loop over the 2-bit packed store
// (head_dim 128, gfx950). Included by tt_attn.hip inside its anonymous
// namespace; uses SplitArgs, AttnInputs, Meta<> and the DPP helpers there.
//
// Replaces the packed-block half of fused_attention_decode_impl
// (csrc/cpu/fused_attn_avx2.cpp:145-301) for one KV head. The reference
// dequantises every block (x = fmaf(q, scale, zero), dequantize_avx2.cpp) and
// dots it with Q; here the dequantisation is folded into the operands of
// v_mfma_f32_16x16x32_f16:
//
//   QK:  s[t][h] = sum_c Q[h][c] (q[t][c] ks[c] + kz[c])
//              = sum_c q[t][c] (Q[h][c] ks[c]) + sum_c Q[h][c] kz[c]
//        A = the 2-bit codes q, B = a[c][h] = Q[h][c] ks[c] split into an
//        f16 high part and an f16 low part (two MFMAs, ~22 significant bits),
//        plus a per-head bias in f32.
//   PV:  o[h][c] = sum_t p[h][t] (q[t][c] vs[t] + vz[t])
//              = sum_t (p[h][t] vs[t]) q[t][c] + sum_t p[h][t] vz[t]
//        A = p vs split hi/lo, B = the 2-bit codes, plus a per-head f32 term.
//
// The 2-bit codes become f16 operands with two instructions per pair of
// values: the code at bit offset 2k of a byte is masked in place and OR-ed
// into the f16 pattern of 1024.0 (v_and_or_b32), giving 1024 + q 4^k, and a
// packed f16 subtract of 1024 leaves q 4^k exactly (v_pk_add_f16); one
// power of four per output row (QK) or column (PV) undoes the 4^k. The values
// are normal f16 numbers on purpose: the matrix cores keep fewer bits of a
// product whose f16 input is subnormal (about two bits per factor of four
// below the normal range), so masking the codes as f16 subnormals, which
// would save the subtract, costs up to ten bits of the dot product.
// The reference's K words hold 16 tokens of one channel and its V words 16
// channels of one token, while an MFMA lane needs one row with 8 reduction
// elements; each wave therefore re-lays a 32-token pair of tiles out in LDS
// at byte granularity (v_perm within a lane for K, a 4x4 byte transpose
// across a DPP quad for V) before reading the operands with wide LDS loads.
//
// Softmax runs online in log2 units. The running reference m of each head is
// kept at least max(s) - sigma, where 2^sigma * max|vs| < 2^13 for every tile
// seen, so p * vs = 2^(s - m) vs stays below 2^15 and never overflows the f16
// operand; the sum l and the accumulators use the same reference, which
// leaves acc / l unchanged. The reference only moves when a tile would
// break that bound by more than 2^2, so the rescale of the accumulators is
// rare.

typedef _Float16 mf_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mf_h2 __attribute__((ext_vector_type(2)));
typedef float mf_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t mf_u4 __attribute__((ext_vector_type(4)));

constexpr int kMfD = 128;       // head_dim of this path
constexpr float kMfTau = 2.0f;  // slack of the lazy rescale, log2 units

// Per-wave LDS staging of one 32-token pair (byte offsets).
template <int GP>
struct MfLds {
    static constexpr int KT = 0;       // [2 tiles][4 token quads][128 channel bytes]
    static constexpr int VT = 1024;    // [32 byte columns][32 token bytes in MFMA order]
    static constexpr int KSZ = 2048;   // [2 tiles][scale | zero][128] f32
    static constexpr int VS = 4096;    // [32] f32, MFMA token order
    static constexpr int VZ = 4224;    // [32] f32
    static constexpr int BIAS = 4352;  // [16] f32 per-head QK bias
    static constexpr int BHI = 4416;   // [GP][128] f16 QK coefficients, MFMA channel order
    static constexpr int BLO = BHI + GP * 2 * kMfD;
    static constexpr int BYTES = BLO + GP * 2 * kMfD;
    // final merge of the four waves, reusing the staging area
    static constexpr int MERGE = 4 * GP * (3 + kMfD) * 4;
    static_assert(MERGE <= 4 * BYTES, "merge area must fit in the staging area");
};

__device__ __forceinline__ float row_max16(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return x;
}

__device__ __forceinline__ uint32_t dpp_u32_quad1(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t dpp_u32_quad2(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x4E, 0xF, 0xF, false));
}

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// data (LDS instructions of one wave execute in issue order).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ mf_f4 mfma16x16x32(mf_u4 a, mf_u4 b, mf_f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mf_h8, a), __builtin_bit_cast(mf_h8, b), c, 0,
                                                  0, 0);
}

// Two 2-bit codes of x at bit offsets 2k and 16 + 2k (mk selects them) ->
// the f16 pair (q0 4^k, q1 4^k), exact.
__device__ __forceinline__ uint32_t code_f16(uint32_t x, uint32_t mk) {
    const mf_h2 v = __builtin_bit_cast(mf_h2, (x & mk) | 0x64006400u);
    const mf_h2 off = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    return __builtin_bit_cast(uint32_t, v - off);
}

// x0, x1 -> (hi, lo) f16 pairs with x ~= hi + lo: hi truncated, lo the
// rounded-to-nearest remainder (exact in f32).
__device__ __forceinline__ uint2 split_hl(float x0, float x1) {
    const mf_h2 h = __builtin_bit_cast(mf_h2, __builtin_amdgcn_cvt_pkrtz(x0, x1));
    const float r0 = x0 - static_cast<float>(h.x);
    const float r1 = x1 - static_cast<float>(h.y);
    mf_h2 l;
    l.x = static_cast<_Float16>(r0);
    l.y = static_cast<_Float16>(r1);
    return make_uint2(__builtin_bit_cast(uint32_t, h), __builtin_bit_cast(uint32_t, l));
}

// Four split pairs -> (hi operand, lo operand).
__device__ __forceinline__ void split_hl4(float a0, float a1, float b0, float b1, float c0, float c1, float d0,
                                          float d1, mf_u4& hi, mf_u4& lo) {
    const uint2 x = split_hl(a0, a1), y = split_hl(b0, b1), z = split_hl(c0, c1), w = split_hl(d0, d1);
    hi = mf_u4{x.x, y.x, z.x, w.x};
    lo = mf_u4{x.y, y.y, z.y, w.y};
}

template <typename MetaT>
__device__ __forceinline__ float4 load_meta4(const MetaT* __restrict__ p) {
    if constexpr (sizeof(MetaT) == 4) {
        return *reinterpret_cast<const float4*>(p);
    } else {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        return make_float4(f16_to_f32(static_cast<uint16_t>(v.x & 0xffffu)), f16_to_f32(static_cast<uint16_t>(v.x >> 16)),
                           f16_to_f32(static_cast<uint16_t>(v.y & 0xffffu)), f16_to_f32(static_cast<uint16_t>(v.y >> 16)));
    }
}

// One workgroup: KV head blockIdx.y, query heads [GP * blockIdx.z, +GP), a
// contiguous range of 32-token pairs of packed tiles; wave w takes pairs
// w, w + 4, ... of the range. Writes partial slot `split` of each head.
template <int GP, typename MetaT>
__device__ __forceinline__ void packed_body(const SplitArgs& a, const int split, char* lds) {
    constexpr int NP = GP >= 4 ? GP / 4 : 1;  // coefficient passes (4 heads x 16 chunks each)
    using L = MfLds<GP>;
    const AttnInputs& in = a.in;
    const int kvh = blockIdx.y;
    const int G = in.Hq / in.Hkv;
    const int g0 = blockIdx.z * GP;
    const int gc = min(GP, G - g0);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 15;   // MFMA column: query head (QK) / channel group (PV); chunk of 8 channels (coefficients)
    const int gk = lane >> 4;  // MFMA reduction group
    const int Hkv = in.Hkv;

    int n0 = in.n0, n1 = in.n1, n2 = in.n2, nb = in.num_blocks;
    if (in.state) {
        n0 = in.state[kSCount];
        n1 = in.state[kHhCount];
        n2 = in.state[kRwCount];
        nb = in.state[kBlocksUsed];
    }
    const int Nd = n0 + n1 + n2;
    const int W = in.kgs >> 4;
    const int Tp = nb * W;           // 16-token tiles
    const int nslots = nb * in.kgs;  // packed token slots
    const int P = (Tp + 1) >> 1;     // 32-token pairs
    const int pb = static_cast<int>(static_cast<long long>(P) * split / a.nsplit_p);
    const int pe = static_cast<int>(static_cast<long long>(P) * (split + 1) / a.nsplit_p);

    char* wl = lds + wave * L::BYTES;
    uint32_t* kt_l = reinterpret_cast<uint32_t*>(wl + L::KT);
    uint32_t* vt_l = reinterpret_cast<uint32_t*>(wl + L::VT);
    float* ksz_l = reinterpret_cast<float*>(wl + L::KSZ);
    float* vs_l = reinterpret_cast<float*>(wl + L::VS);
    float* vz_l = reinterpret_cast<float*>(wl + L::VZ);
    float* bias_l = reinterpret_cast<float*>(wl + L::BIAS);
    char* bhi_l = wl + L::BHI;
    char* blo_l = wl + L::BLO;

    // Q' = Q 2^-e per head (e = exponent of max |Q_h|) in the coefficient
    // layout: pass pp, head 4 pp + gk, channels 8 n .. 8 n + 7.
    float qv[NP][8];
    float cpass[NP];
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
        const int h = 4 * pp + gk;
        if (h < gc) {
            const float* qp = in.Q + static_cast<size_t>(kvh * G + g0 + h) * kMfD + 8 * n;
            const float4 x0 = *reinterpret_cast<const float4*>(qp);
            const float4 x1 = *reinterpret_cast<const float4*>(qp + 4);
            qv[pp][0] = x0.x; qv[pp][1] = x0.y; qv[pp][2] = x0.z; qv[pp][3] = x0.w;
            qv[pp][4] = x1.x; qv[pp][5] = x1.y; qv[pp][6] = x1.z; qv[pp][7] = x1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) qv[pp][j] = 0.0f;
        }
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(qv[pp][j]));
        mx = row_max16(mx);
        const int e = (mx > 0.0f) ? __builtin_amdgcn_frexp_expf(mx) : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) qv[pp][j] = __builtin_amdgcn_ldexpf(qv[pp][j], -e);
        cpass[pp] = (h < gc) ? __builtin_amdgcn_ldexpf(a.scale2, e) : 0.0f;
    }
    // Column scale of query head n: lane 16 (n & 3) of pass n >> 2 holds it.
    float ccol = 0.0f;
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
        const float t = __shfl(cpass[pp], 16 * (n & 3), 64);
        if ((n >> 2) == pp) ccol = t;
    }
    float crow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) crow[r] = __builtin_amdgcn_ldexpf(ccol, -2 * r);

    const uint32_t kmask = (3u << (2 * (lane & 3))) | (3u << (16 + 2 * (lane & 3)));
    const uint32_t qsel1 = (lane & 1) ? 0x03070105u : 0x06020400u;
    const uint32_t qsel2 = (lane & 2) ? 0x03020706u : 0x05040100u;

    const MetaT* ks = static_cast<const MetaT*>(in.ks);
    const MetaT* kz = static_cast<const MetaT*>(in.kz);
    const MetaT* vs = static_cast<const MetaT*>(in.vs);
    const MetaT* vz = static_cast<const MetaT*>(in.vz);

    mf_f4 acc[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[s] = mf_f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = kNegInf, l_run = 0.0f, pz = 0.0f;

    // Registers of the pair being fetched.
    mf_u4 kw, vw;
    float4 ksr, kzr;
    float vm = 0.0f;
    long long idv = -1;

    auto fetch = [&](const int p) {
        const int kt = min(2 * p + (lane >> 5), Tp - 1);
        const int bk = (W == 2) ? (kt >> 1) : kt;
        kw = *reinterpret_cast<const mf_u4*>(in.kp + (static_cast<size_t>(kt) * Hkv + kvh) * kMfD + 4 * (lane & 31));
        const size_t mo = (static_cast<size_t>(bk) * Hkv + kvh) * kMfD + 4 * (lane & 31);
        ksr = load_meta4<MetaT>(ks + mo);
        kzr = load_meta4<MetaT>(kz + mo);
        const int sv = min(32 * p + 4 * (lane >> 3) + (lane & 3), nslots - 1);
        vw = *reinterpret_cast<const mf_u4*>(in.vp + (static_cast<size_t>(sv) * Hkv + kvh) * (kMfD / 16) +
                                             4 * ((lane >> 2) & 1));
        const int sm = min(32 * p + (lane & 31), nslots - 1);
        vm = Meta<MetaT>::load(lane < 32 ? vs : vz, static_cast<size_t>(sm) * Hkv + kvh);
        const int si = 32 * p + lane;
        idv = -1;
        if (lane < 32 && si < nslots) idv = in.ids[si];
    };

    // Lays the fetched pair out in LDS; returns the token-validity mask.
    auto stage = [&]() -> uint32_t {
        // K: bytes tq of channels c..c+3 -> one dword per token quad.
        const uint32_t u0 = __builtin_amdgcn_perm(kw.y, kw.x, 0x05010400u);
        const uint32_t u1 = __builtin_amdgcn_perm(kw.y, kw.x, 0x07030602u);
        const uint32_t v0 = __builtin_amdgcn_perm(kw.w, kw.z, 0x05010400u);
        const uint32_t v1 = __builtin_amdgcn_perm(kw.w, kw.z, 0x07030602u);
        uint32_t* kd = kt_l + (lane >> 5) * 128 + (lane & 31);
        kd[0] = __builtin_amdgcn_perm(v0, u0, 0x05040100u);
        kd[32] = __builtin_amdgcn_perm(v0, u0, 0x07060302u);
        kd[64] = __builtin_amdgcn_perm(v1, u1, 0x05040100u);
        kd[96] = __builtin_amdgcn_perm(v1, u1, 0x07060302u);
        // V: 4x4 byte transpose across the quad (tokens 4m..4m+3).
        const int m = lane >> 3;
        const int hf = (lane >> 2) & 1;
        uint32_t* vd = vt_l + (16 * hf + (lane & 3)) * 8 + 2 * (m & 3) + (m >> 2);
        const uint32_t vwv[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t x = vwv[g];
            const uint32_t t = __builtin_amdgcn_perm(dpp_u32_quad1(x), x, qsel1);
            const uint32_t y = __builtin_amdgcn_perm(dpp_u32_quad2(t), t, qsel2);
            vd[g * 32] = y;  // byte column 4 (4 hf + g) + (lane & 3)
        }
        float* kzd = ksz_l + (lane >> 5) * 256 + 4 * (lane & 31);
        *reinterpret_cast<float4*>(kzd) = ksr;
        *reinterpret_cast<float4*>(kzd + 128) = kzr;
        const int t2 = lane & 31;
        const int pos = 8 * ((t2 & 15) >> 2) + 4 * (t2 >> 4) + (t2 & 3);
        (lane < 32 ? vs_l : vz_l)[pos] = vm;
        return static_cast<uint32_t>(__ballot(idv != -1));
    };

    int p = pb + wave;
    if (p < pe) fetch(p);
    for (; p < pe; p += 4) {
        const uint32_t vmask = stage();
        if (p + 4 < pe) fetch(p + 4);
        wave_lds_sync();
        const bool full = (vmask == 0xffffffffu);

        float s2[2][4];
#pragma unroll
        for (int tile = 0; tile < 2; ++tile) {
            if (tile == 0 || W == 1) {
                // QK coefficients of this tile's block, MFMA channel order.
#pragma unroll
                for (int pp = 0; pp < NP; ++pp) {
                    const int h = 4 * pp + gk;
                    const float* kss = ksz_l + tile * 256 + 8 * n;
                    const float4 sa = *reinterpret_cast<const float4*>(kss);
                    const float4 sb = *reinterpret_cast<const float4*>(kss + 4);
                    const float4 za = *reinterpret_cast<const float4*>(kss + 128);
                    const float4 zb = *reinterpret_cast<const float4*>(kss + 132);
                    const float sc[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
                    const float zc[8] = {za.x, za.y, za.z, za.w, zb.x, zb.y, zb.z, zb.w};
                    float av[8];
                    float bp = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        av[j] = qv[pp][j] * sc[j];
                        bp = __builtin_fmaf(qv[pp][j], zc[j], bp);
                    }
                    mf_u4 hi, lo;
                    split_hl4(av[0], av[2], av[1], av[3], av[4], av[6], av[5], av[7], hi, lo);
                    bp = row_sum16(bp);
                    if (h < GP) {
                        *reinterpret_cast<mf_u4*>(bhi_l + (h * kMfD + 8 * n) * 2) = hi;
                        *reinterpret_cast<mf_u4*>(blo_l + (h * kMfD + 8 * n) * 2) = lo;
                        if (n == 0) bias_l[h] = bp;
                    }
                }
                wave_lds_sync();
            }
            // A: codes of token t = lane & 15 (k = t & 3), channels 32 gk .. 32 gk + 31.
            const mf_u4* ka = reinterpret_cast<const mf_u4*>(kt_l + (tile * 4 + ((lane & 15) >> 2)) * 32 + 8 * gk);
            const mf_u4 ra = ka[0], rb = ka[1];
            mf_u4 bh[4], bl[4];
            float bias = 0.0f;
            if (n < GP) {
                const mf_u4* ph = reinterpret_cast<const mf_u4*>(bhi_l + (n * kMfD + 32 * gk) * 2);
                const mf_u4* pl = reinterpret_cast<const mf_u4*>(blo_l + (n * kMfD + 32 * gk) * 2);
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    bh[s] = ph[s];
                    bl[s] = pl[s];
                }
                bias = bias_l[n];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    bh[s] = mf_u4{0u, 0u, 0u, 0u};
                    bl[s] = mf_u4{0u, 0u, 0u, 0u};
                }
            }
            mf_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const uint32_t x = (s < 2) ? ra[2 * s] : rb[2 * s - 4];
                const uint32_t y = (s < 2) ? ra[2 * s + 1] : rb[2 * s - 3];
                const mf_u4 av = {code_f16(x, kmask), code_f16(x >> 8, kmask), code_f16(y, kmask),
                                  code_f16(y >> 8, kmask)};
                d = mfma16x16x32(av, bh[s], d);
                d = mfma16x16x32(av, bl[s], d);
            }
            const float bc = bias * ccol;
#pragma unroll
            for (int r = 0; r < 4; ++r) s2[tile][r] = __builtin_fmaf(d[r], crow[r], bc);
        }

        if (!full) {
#pragma unroll
            for (int tile = 0; tile < 2; ++tile)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (!((vmask >> (16 * tile + 4 * gk + r)) & 1u)) s2[tile][r] = kNegInf;
        }
        if (a.logits && n < gc) {
            float* row = a.logits + static_cast<size_t>(kvh * G + g0 + n) * a.ld + Nd + 32 * p;
#pragma unroll
            for (int tile = 0; tile < 2; ++tile)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * tile + 4 * gk + r;
                    if (32 * p + t < nslots) row[t] = s2[tile][r];
                }
        }

        // V scale / zero of this lane's tokens: [tile 0 r 0..3, tile 1 r 0..3].
        const float4 va = *reinterpret_cast<const float4*>(vs_l + 8 * gk);
        const float4 vb = *reinterpret_cast<const float4*>(vs_l + 8 * gk + 4);
        const float4 za = *reinterpret_cast<const float4*>(vz_l + 8 * gk);
        const float4 zb = *reinterpret_cast<const float4*>(vz_l + 8 * gk + 4);
        const float vsv[2][4] = {{va.x, va.y, va.z, va.w}, {vb.x, vb.y, vb.z, vb.w}};
        const float vzv[2][4] = {{za.x, za.y, za.z, za.w}, {zb.x, zb.y, zb.z, zb.w}};

        float mx = kNegInf, vmx = 0.0f;
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                mx = fmaxf(mx, s2[tile][r]);
                const float av = fabsf(vsv[tile][r]);
                vmx = fmaxf(vmx, (full || s2[tile][r] != kNegInf) ? av : 0.0f);
            }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        vmx = fmaxf(vmx, shfl_xor(vmx, 16));
        vmx = fmaxf(vmx, shfl_xor(vmx, 32));
        const int ev = (vmx > 0.0f) ? __builtin_amdgcn_frexp_expf(vmx) : 0;
        const float cand = mx - static_cast<float>(13 - ev);
        const bool up = cand > m_run + kMfTau;
        if (__ballot(up)) {
            const float mn = up ? cand : m_run;
            const float al = up ? exp2f(m_run - mn) : 1.0f;
            l_run *= al;
            pz *= al;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float ar = __shfl(al, 4 * gk + r, 64);
#pragma unroll
                for (int s = 0; s < 8; ++s) acc[s][r] *= ar;
            }
            m_run = mn;
        }

        float pv[2][4];
        float lsum = 0.0f;
#pragma unroll
        for (int tile = 0; tile < 2; ++tile)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float e = exp2f(s2[tile][r] - m_run);
                if (!full) e = (s2[tile][r] == kNegInf) ? 0.0f : e;
                lsum += e;
                // invalid slots may hold any scale / zero: keep them out of the sums
                const bool use = full || e != 0.0f;
                pz = use ? __builtin_fmaf(e, vzv[tile][r], pz) : pz;
                pv[tile][r] = use ? e * vsv[tile][r] : 0.0f;
            }
        l_run += lsum;
        mf_u4 ahi, alo;
        split_hl4(pv[0][0], pv[0][2], pv[0][1], pv[0][3], pv[1][0], pv[1][2], pv[1][1], pv[1][3], ahi, alo);

        // B: codes of channel 4 beta + k for the lane's 8 tokens,
        // beta = n (nsteps 0..3) and n + 16 (nsteps 4..7), k = nstep & 3.
        const uint2* vtr = reinterpret_cast<const uint2*>(vt_l);
        const uint2 q0 = vtr[n * 4 + gk];
        const uint2 q1 = vtr[(n + 16) * 4 + gk];
        const uint32_t q0a = q0.x >> 8, q0b = q0.y >> 8, q1a = q1.x >> 8, q1b = q1.y >> 8;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t mk = (3u << (2 * k)) | (3u << (16 + 2 * k));
            const mf_u4 b0 = {code_f16(q0.x, mk), code_f16(q0a, mk), code_f16(q0.y, mk), code_f16(q0b, mk)};
            acc[k] = mfma16x16x32(ahi, b0, acc[k]);
            acc[k] = mfma16x16x32(alo, b0, acc[k]);
            const mf_u4 b1 = {code_f16(q1.x, mk), code_f16(q1a, mk), code_f16(q1.y, mk), code_f16(q1b, mk)};
            acc[4 + k] = mfma16x16x32(ahi, b1, acc[4 + k]);
            acc[4 + k] = mfma16x16x32(alo, b1, acc[4 + k]);
        }
        wave_lds_sync();
    }

    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
    pz += shfl_xor(pz, 16);
    pz += shfl_xor(pz, 32);

    __syncthreads();  // every wave is done with its staging area
    float* sm_m = reinterpret_cast<float*>(lds);  // [4][GP]
    float* sm_l = sm_m + 4 * GP;                   // [4][GP]
    float* sm_z = sm_l + 4 * GP;                   // [4][GP]
    float* sm_acc = sm_z + 4 * GP;                 // [4][GP][128]
    if (lane < GP) {
        sm_m[wave * GP + lane] = m_run;
        sm_l[wave * GP + lane] = l_run;
        sm_z[wave * GP + lane] = pz;
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * gk + r;
            if (h < GP) {
                const int c = 4 * n + 64 * (s >> 2) + (s & 3);
                sm_acc[(wave * GP + h) * kMfD + c] = __builtin_amdgcn_ldexpf(acc[s][r], -2 * (s & 3));
            }
        }
    __syncthreads();
    for (int idx = threadIdx.x; idx < gc * kMfD; idx += 256) {
        const int g = idx / kMfD, c = idx - g * kMfD;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w * GP + g]);
        float A = 0.0f, Ls = 0.0f;
        if (M != kNegInf) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float mw = sm_m[w * GP + g];
                const float f = (mw == kNegInf) ? 0.0f : exp2f(mw - M);
                A = __builtin_fmaf(f, sm_acc[(w * GP + g) * kMfD + c] + sm_z[w * GP + g], A);
                Ls = __builtin_fmaf(f, sm_l[w * GP + g], Ls);
            }
        }
        const size_t pi = static_cast<size_t>(kvh * G + g0 + g) * a.nsplit + split;
        a.part_acc[pi * kMfD + c] = A;
        if (c == 0) {
            a.part_ml[2 * pi] = M;
            a.part_ml[2 * pi + 1] = Ls;
        }
    }
}
