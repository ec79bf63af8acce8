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
//              = sum_t (p[h][t] vs[t] / 2) (2 q[t][c] - 3) + sum_t p[h][t] (vz[t] + 1.5 vs[t])
//        A = p vs split hi/lo, B = the centred codes 2q - 3, plus a per-head
//        f32 term. Centring keeps both sums near the size of the output: with
//        the raw codes they would both grow like the row minimum vz (about
//        -2.5 for N(0,1) rows, the same sign for every token) and cancel, and
//        their float32 rounding would dominate the output's error.
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

// Per-wave LDS staging of one 32-token pair (byte offsets). Row strides are
// padded so that the wide LDS accesses of one instruction (8 lanes x 16
// bytes, 16 lanes x 8 bytes) fall into distinct banks.
constexpr int kKTS = 36;   // dwords per K row (token quad): 128 channel bytes + 4 dwords pad
// V byte column r (32 token bytes = 8 dwords, in MFMA order) starts at dword
// 8 r + (r >> 4) with its dwords permuted by XOR 2 ((r >> 2) & 3): the lay-out
// writes (16 lanes of 4 bytes per cycle) and the operand reads (16 lanes of
// 8 bytes) then each fall into 32 distinct banks; columns 16..31 start at an
// odd dword, so their 8-byte reads are two 4-byte reads.
__device__ __forceinline__ int vt_dword(const int r, const int d) { return 8 * r + (r >> 4) + (d ^ (2 * ((r >> 2) & 3))); }
constexpr int kKSZ = 144;  // floats per K scale (zero) row: channel c at c + 4 (c / 32)
constexpr int kBRS = 136;  // halves per coefficient row: 128 + 8 pad
template <int GP>
struct MfLds {
    static constexpr int KT = 0;       // [2 tiles][4 token quads][kKTS dwords]
    static constexpr int VT = 1152;    // [32 byte columns][8 dwords] + 1 (vt_dword), token bytes in MFMA order
    static constexpr int KSZ = 2432;   // [2 tiles][scale | zero][kKSZ] f32
    static constexpr int VS = 4736;    // [2 halves][32] f32, MFMA token order (0 for masked slots); half 1: paired heads
    static constexpr int VZ = 4992;    // [2][32] f32
    static constexpr int BIAS = 5248;  // [2 tiles][8] f32 per-head QK bias
    static constexpr int BHL = 5312;   // [NBT tiles][hi rows 0..GP-1, lo rows GP..2GP-1][kBRS] f16
    static constexpr int BHL_TILE = 2 * GP * kBRS * 2;
    // Coefficient tiles held at once. Eight heads keep one (the second tile
    // of a pair reuses it), which brings the workgroup under a third of the
    // CU's 160 KB and lets three workgroups share a CU.
    static constexpr int NBT = GP > 4 ? 1 : 2;
    static constexpr int BYTES = BHL + NBT * BHL_TILE;
    // final merge of the four waves, reusing the staging area
    static constexpr int MERGE = 4 * GP * (3 + kMfD) * 4;
    static_assert(MERGE <= 4 * BYTES, "merge area must fit in the staging area");
    static_assert(VT + 4 * (8 * 31 + 1 + 7 + 1) <= KSZ, "V byte columns must fit before the K scales");
    // the workgroup's query heads [GP][128] f32, after the four staging areas
    static constexpr int QL = 4 * BYTES;
    // 128 zero f16 coefficients (a B row that contributes nothing)
    static constexpr int ZERO = QL + GP * kMfD * 4;
    // Per-wave logits of the last LB_PAIRS pairs, [GP][LB_PAIRS * 32 + 4] f32 (the
    // 4 floats of padding put the heads' 16-byte writes in distinct banks): they
    // reach memory in runs of LB_PAIRS * 128 bytes per head, stored early in
    // the next pair (one wait counter covers loads and stores, so a store issued
    // late in a pair would hold up the next lay-out). Eight heads store their
    // logits directly (a buffer of one pair measured 3% slower there: it
    // spills a register at 168 VGPRs).
    static constexpr int LB_PAIRS = GP > 4 ? 0 : 4;
    static constexpr int LB = ZERO + 256;
    static constexpr int LB_HEAD = LB_PAIRS > 0 ? LB_PAIRS * 32 + 4 : 0;  // floats per head
    static constexpr int LB_WAVE = GP * LB_HEAD * 4;
    static constexpr int TOTAL = LB + 4 * LB_WAVE;
};

// LDS of an FP32-tier workgroup (byte offsets): the query heads, then the
// per-wave partials [4][GP][max, sum, acc[128]].
template <int GP>
struct DnLds {
    static constexpr int QL = 0;                 // [16][128] f32: one row per MFMA column, zeros past the group
    static constexpr int PART = 16 * kMfD * 4;
    static constexpr int TOTAL = PART + 4 * GP * (2 + kMfD) * 4;
};

// max(a, b) for operands that are never NaN: one v_max_f32, without the
// quieting of the operands that fmaxf adds for values it cannot see the origin of.
__device__ __forceinline__ float fmax_nn(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// max(|a|, |b|), likewise
__device__ __forceinline__ float fmax_abs_nn(float a, float b) {
    float r;
    asm("v_max_f32_e64 %0, |%1|, |%2|" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Reductions over the four 16-lane rows of a wave (lanes n, n+16, n+32, n+48).
__device__ __forceinline__ float xrow_max(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmax_nn(__uint_as_float(s[0]), __uint_as_float(s[1]));
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmax_nn(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float xrow_sum(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

__device__ __forceinline__ float row_max16(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return x;
}

// Quad permutations (every lane reads a valid source, so no old value).
__device__ __forceinline__ uint32_t dpp_u32_quad1(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t dpp_u32_quad2(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xF, 0xF, true));
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
// `one024` holds 0x64006400 in a VGPR: v_and_or_b32 may read only one SGPR
// (the mask) on this target, so a second scalar constant would split it in two.
__device__ __forceinline__ uint32_t code_f16(uint32_t x, uint32_t mk, uint32_t one024) {
    const mf_h2 v = __builtin_bit_cast(mf_h2, (x & mk) | one024);
    const mf_h2 off = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    return __builtin_bit_cast(uint32_t, v - off);
}

// Two centred codes: x holds the codes at bit offsets 2k + 1 and 17 + 2k (a
// word shifted left by one; mk2 selects them) -> the f16 pair
// ((2 q0 - 3) 4^k, (2 q1 - 3) 4^k), exact: 1024 + 2 q 4^k minus 1024 + 3 4^k
// (an integer, so the constant and the difference are exact f16 values).
__device__ __forceinline__ uint32_t code_f16_centred(uint32_t x, uint32_t mk2, uint32_t one024, int k) {
    const mf_h2 v = __builtin_bit_cast(mf_h2, (x & mk2) | one024);
    const _Float16 c = static_cast<_Float16>(1024.0f + 3.0f * static_cast<float>(1 << (2 * k)));
    const mf_h2 off = {c, c};
    return __builtin_bit_cast(uint32_t, v - off);
}

// x - m * f16 (low / high half of h), one v_fma_mix_f32 (exact for m = 1
// and h a rounding of x: the difference fits in f32).
__device__ __forceinline__ float fma_mix_lo(uint32_t h, float negm, float x) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(negm), "v"(x));
    return r;
}
__device__ __forceinline__ float fma_mix_hi(uint32_t h, float negm, float x) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(negm), "v"(x));
    return r;
}

__device__ __forceinline__ uint32_t cvt_pk_f16(float x0, float x1) {
    mf_h2 v;
    v.x = static_cast<_Float16>(x0);
    v.y = static_cast<_Float16>(x1);
    return __builtin_bit_cast(uint32_t, v);
}

// x0, x1 -> (hi, lo) f16 pairs with x ~= hi + lo: hi and the remainder lo
// both rounded to nearest (the remainder is exact in f32).
__device__ __forceinline__ uint2 split_hl(float x0, float x1) {
    const uint32_t hi = cvt_pk_f16(x0, x1);
    return make_uint2(hi, cvt_pk_f16(fma_mix_lo(hi, -1.0f, x0), fma_mix_hi(hi, -1.0f, x1)));
}

// One half of the split per lane: hi where negm = 0, lo where negm = -1
// (the rounding of x, then of its remainder, exactly as split_hl).
__device__ __forceinline__ uint32_t split_half(float x0, float x1, float negm) {
    const uint32_t hi = cvt_pk_f16(x0, x1);
    return cvt_pk_f16(fma_mix_lo(hi, negm, x0), fma_mix_hi(hi, negm, x1));
}

// Four split pairs -> (hi operand, lo operand).
__device__ __forceinline__ void split_hl4(float a0, float a1, float b0, float b1, float c0, float c1, float d0,
                                          float d1, mf_u4& hi, mf_u4& lo) {
    const uint2 x = split_hl(a0, a1), y = split_hl(b0, b1), z = split_hl(c0, c1), w = split_hl(d0, d1);
    hi = mf_u4{x.x, y.x, z.x, w.x};
    lo = mf_u4{x.y, y.y, z.y, w.y};
}

// Prefetched metadata stays in its stored width until the pair is laid out:
// a conversion next to the load would make the prefetch wait for its own data.
// Four values (K scale or zero of four channels) and one (V scale or zero).
// The K-side loads (K words, K scale and zero; each line is read once) are
// non-temporal, which measured ~2% faster per launch at 32k and 128k
// contexts; the same for the V words or the FP32 tiers measured slower.
template <typename MetaT>
struct MetaRaw;
template <>
struct MetaRaw<float> {
    using Four = float4;
    using One = float;
    __device__ __forceinline__ static Four load4(const float* p) {
        const mf_f4 v = __builtin_nontemporal_load(reinterpret_cast<const mf_f4*>(p));
        return make_float4(v[0], v[1], v[2], v[3]);
    }
    __device__ __forceinline__ static One load1(const float* p) { return *p; }
    __device__ __forceinline__ static float4 f4(const Four v) { return v; }
    __device__ __forceinline__ static float f1(const One v) { return v; }
    // two adjacent values (the V scale or zero of a pair of head_dim-64 heads)
    using Two = float2;
    __device__ __forceinline__ static Two load2(const float* p) { return *reinterpret_cast<const float2*>(p); }
    __device__ __forceinline__ static float2 f2(const Two v) { return v; }
};
template <>
struct MetaRaw<uint16_t> {
    using Four = uint2;
    using One = uint32_t;
    __device__ __forceinline__ static Four load4(const uint16_t* p) {
        typedef uint32_t u2v __attribute__((ext_vector_type(2)));
        const u2v v = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(p));
        return make_uint2(v[0], v[1]);
    }
    __device__ __forceinline__ static One load1(const uint16_t* p) { return *p; }
    __device__ __forceinline__ static float4 f4(const Four v) {
        return make_float4(f16_to_f32(static_cast<uint16_t>(v.x & 0xffffu)), f16_to_f32(static_cast<uint16_t>(v.x >> 16)),
                           f16_to_f32(static_cast<uint16_t>(v.y & 0xffffu)), f16_to_f32(static_cast<uint16_t>(v.y >> 16)));
    }
    __device__ __forceinline__ static float f1(const One v) { return f16_to_f32(static_cast<uint16_t>(v)); }
    using Two = uint32_t;
    __device__ __forceinline__ static Two load2(const uint16_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
    __device__ __forceinline__ static float2 f2(const Two v) {
        return make_float2(f16_to_f32(static_cast<uint16_t>(v & 0xffffu)), f16_to_f32(static_cast<uint16_t>(v >> 16)));
    }
};

// Stores that write through the L2 (device scope): the partials and logits
// are read by the next launch from other XCDs, and lines left dirty in the L2
// would be written back at the end of this launch instead.
typedef unsigned int tt_u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st_dev4(float* base, const uint32_t bytes, const uint32_t off, const float4 v) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
    const tt_u4v w = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
    __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, 16 /* sc1 */);
}
__device__ __forceinline__ void st_dev1(float* p, const float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Even split of `count` items over `parts`: the first item of part `i`,
// floor(count * i / parts), in 32-bit arithmetic for any count < 2^31 and
// i <= parts < 2^16 (a 64-bit divide is a long software loop):
// count * i = (q * parts + r) * i, so the floor is q * i + floor(r * i / parts)
// with r * i < parts^2.
__device__ __forceinline__ int part_begin(const int count, const int i, const int parts) {
    // The divides are expanded into vector instructions; readfirstlane hands
    // the (wave-uniform) result back to the scalar unit so loop bounds and the
    // branches that depend on them stay uniform.
    const unsigned c = static_cast<unsigned>(count), n = static_cast<unsigned>(parts), k = static_cast<unsigned>(i);
    const unsigned q = c / n, r = c - q * n;
    return __builtin_amdgcn_readfirstlane(static_cast<int>(q * k + r * k / n));
}

// FP32 16-token tiles [d0, d1) of FP32 workgroup `dsplit` of nsplit_d.
__device__ __forceinline__ void dense_range(const SplitArgs& a, const int Nd, const int dsplit, int& d0, int& d1) {
    const int Td = (Nd + 15) >> 4;
    d0 = part_begin(Td, dsplit, a.nsplit_d);
    d1 = part_begin(Td, dsplit + 1, a.nsplit_d);
}

// The group's query heads into LDS ([GP][128] f32, heads past gc as zeros).
// Issued before any other global load of the workgroup: loads return in
// order, so the barrier that follows then waits for this load only.
// PAIR (head_dim-64 heads 2j, 2j + 1 as one head of 128 channels): the query
// of the group's head g has 64 channels and fills the half of its own KV head,
// (g0 + g) / (G / 2), with zeros in the other half, so its logits are those of
// its own head.
template <int GP, bool PAIR = false>
__device__ __forceinline__ void load_q_lds(const AttnInputs& in, const int kvh, const int g0, const int gc,
                                           float* q_l) {
    const int G = in.Hq / in.Hkv;
    for (int idx = threadIdx.x; idx < GP * (kMfD / 4); idx += 256) {
        const int g = idx / (kMfD / 4), c4 = idx - g * (kMfD / 4);
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (g < gc) {
            const size_t row = static_cast<size_t>(kvh * G + g0 + g);
            if constexpr (PAIR) {
                if ((c4 >> 4) == (g0 + g) / (G >> 1))
                    v = *reinterpret_cast<const float4*>(in.Q + row * (kMfD / 2) + 4 * (c4 & 15));
            } else {
                v = *reinterpret_cast<const float4*>(in.Q + row * kMfD + 4 * c4);
            }
        }
        *reinterpret_cast<float4*>(q_l + g * kMfD + 4 * c4) = v;
    }
}

// Tier pointers and counts of the FP32 tokens (device counters for the engine).
struct DenseView {
    int n0, n1, n2, head, Nd;
};

__device__ __forceinline__ DenseView dense_view(const AttnInputs& in) {
    DenseView v{in.n0, in.n1, in.n2, in.ring_head, 0};
    if (in.state) {
        v.n0 = in.state[kSCount];
        v.n1 = in.state[kHhCount];
        v.n2 = in.state[kRwCount];
        v.head = in.state[kRwHead];
    }
    v.Nd = v.n0 + v.n1 + v.n2;
    return v;
}

// One 16-token FP32 tile for one lane (g = lane / 16, n = lane % 16) in the
// operand layouts of v_mfma_f32_16x16x4_f32:
//   k: keys of token n, channels 32 g .. 32 g + 31 (QK A operand, row n);
//   v: values of tokens 4 g + j (j = 0..3), channels 8 n .. 8 n + 7 (PV B
//      operand, column n of output block b holding channel 8 n + b).
struct DenseTile {
    float4 k[8];
    float4 v[4][2];
};

// K and V rows of token `r0` (clamped to the last tier row; rows past the
// tiers are masked later) in the logical FP32 order sinks -> heavy hitters ->
// recent ring.
struct DenseRow {
    const float* k;
    const float* v;
};
__device__ __forceinline__ DenseRow dense_row(const AttnInputs& in, const DenseView& dv, const int kvh, const int r0) {
    const int r = r0 < dv.Nd ? r0 : dv.Nd - 1;
    const bool in0 = r < dv.n0, in1 = r < dv.n0 + dv.n1;
    int ring = dv.head + (r - dv.n0 - dv.n1);
    ring = ring >= in.ring_size ? ring - in.ring_size : ring;
    const int idx = in0 ? r : (in1 ? r - dv.n0 : ring);
    const float* kb = in0 ? in.k0 : (in1 ? in.k1 : in.k2);
    const float* vb = in0 ? in.v0 : (in1 ? in.v1 : in.v2);
    const size_t off = (static_cast<size_t>(idx) * in.Hkv + kvh) * kMfD;
    return DenseRow{kb + off, vb + off};
}

// Issues the loads of tile k.
__device__ __forceinline__ void dense_load(const AttnInputs& in, const DenseView& dv, const int kvh, const int k,
                                           DenseTile& t) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const int tok0 = 16 * k;
    {
        const float* kb = dense_row(in, dv, kvh, tok0 + n).k + 32 * g;
#pragma unroll
        for (int i = 0; i < 8; ++i) t.k[i] = *reinterpret_cast<const float4*>(kb + 4 * i);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float* vb = dense_row(in, dv, kvh, tok0 + 4 * g + j).v + 8 * n;
        t.v[j][0] = *reinterpret_cast<const float4*>(vb);
        t.v[j][1] = *reinterpret_cast<const float4*>(vb + 4);
    }
}

// One 16-token FP32 tile for the VALU path of query groups of one or two
// heads: lane (tg = lane / 16, cp = lane % 16) holds keys and values of
// tokens 4 tg .. 4 tg + 3, channels 8 cp .. 8 cp + 7.
struct DenseTileV {
    float kx[4][8], vx[4][8];
};

__device__ __forceinline__ void dense_load(const AttnInputs& in, const DenseView& dv, const int kvh, const int k,
                                           DenseTileV& t) {
    const int lane = threadIdx.x & 63;
    const int tg = lane >> 4, cp = lane & 15;
    const int tok0 = 16 * k + 4 * tg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const DenseRow r = dense_row(in, dv, kvh, tok0 + i);
        load_f32<8>(r.k + 8 * cp, t.kx[i]);
        load_f32<8>(r.v + 8 * cp, t.vx[i]);
    }
}

// The FP32 tiers of the workgroup's share on the VALU, for GP <= 2. An f32
// matrix-core tile (v_mfma_f32_16x16x4_f32, 32 cycles for 16 x 16 x 4) puts
// one query head in each of its 16 columns, so with one or two heads it does
// 8 or 4 times the work the VALU does for the same tile (per launch: an
// 8k-context 32/32-head layer 18.1 against 16.7 us, a 32k 16/8-head layer
// 15.8 against 15.1 us, head_dim-64 heads in pairs at 8k 32/32 heads 12.0
// against 11.6 us). Same tile order, logits
// and LDS partial layout as dense_share. Lane (tg, cp) sums its 8-channel
// products, a DPP row sum completes the logit of token 4 tg + i; the online
// softmax is exact (the reference moves with every tile's maximum).
template <int GP>
__device__ __forceinline__ void dense_share_valu(const SplitArgs& a, const DenseView& dv, const int d0,
                                                 const int d1, const int kvh, const int g0, const int gc,
                                                 const int wave, const float* q_l, const DenseTileV& t0,
                                                 float* dl) {
    static_assert(GP <= 2, "the VALU path holds every head's accumulators");
    const AttnInputs& in = a.in;
    const int lane = threadIdx.x & 63;
    const int tg = lane >> 4, cp = lane & 15;
    const int G = in.Hq / in.Hkv;
    const int Nd = dv.Nd;
    float m[GP], l[GP], acc[GP][8];
#pragma unroll
    for (int g = 0; g < GP; ++g) {
        m[g] = kNegInf;
        l[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;
    }
    auto consume = [&](const DenseTileV& t, const int k) {
        const int tok0 = 16 * k + 4 * tg;
        float s[4][GP];
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            const float4 qa = *reinterpret_cast<const float4*>(q_l + g * kMfD + cp * 8);
            const float4 qb = *reinterpret_cast<const float4*>(q_l + g * kMfD + cp * 8 + 4);
            const float qg[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) d = __builtin_fmaf(qg[j], t.kx[i][j], d);
                const float v = row_sum16(d) * a.scale2;
                s[i][g] = (tok0 + i < Nd) ? v : kNegInf;
            }
        }
        if (a.logits) {
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                if (g < gc && cp == g) {
                    float* lr = a.logits + static_cast<size_t>(kvh * G + g0 + g) * a.ld + tok0;
                    if (tok0 + 4 <= Nd) {
                        st_dev4(a.logits, static_cast<uint32_t>(in.Hq) * a.ld * 4u,
                                static_cast<uint32_t>((lr - a.logits) * 4),
                                make_float4(s[0][g], s[1][g], s[2][g], s[3][g]));
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (tok0 + i < Nd) lr[i] = s[i][g];
                    }
                }
            }
        }
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            const float tm = xrow_max(fmaxf(fmaxf(s[0][g], s[1][g]), fmaxf(s[2][g], s[3][g])));
            const float mn = fmaxf(m[g], tm);
            const float alpha = (m[g] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(m[g] - mn);
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = (s[i][g] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(s[i][g] - mn);
            l[g] = __builtin_fmaf(l[g], alpha, (p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float v = acc[g][j] * alpha;
                v = __builtin_fmaf(p[0], t.vx[0][j], v);
                v = __builtin_fmaf(p[1], t.vx[1][j], v);
                v = __builtin_fmaf(p[2], t.vx[2][j], v);
                v = __builtin_fmaf(p[3], t.vx[3][j], v);
                acc[g][j] = v;
            }
            m[g] = mn;
        }
    };
    int kb = d0 + wave;
    if (kb < d1) {
        consume(t0, kb);  // in flight since the start of the kernel
        kb += 4;
    }
#pragma unroll 1
    for (int k = kb; k < d1; k += 4) {
        DenseTileV t;
        dense_load(in, dv, kvh, k, t);
        consume(t, k);
    }
    // The four token groups share m: sum them, then the partial into LDS.
    float* my = dl + wave * GP * (2 + kMfD);
#pragma unroll
    for (int g = 0; g < GP; ++g) {
        const float lt = xrow_sum(l[g]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = xrow_sum(acc[g][j]);
        if (tg == 0) {
            float* pg = my + g * (2 + kMfD);
#pragma unroll
            for (int j = 0; j < 8; ++j) pg[2 + cp * 8 + j] = acc[g][j];
            if (cp == 0) {
                pg[0] = m[g];
                pg[1] = lt;
            }
        }
    }
}

// Component r (a constant after unrolling) of a float4, and that component
// scaled (values, not references, so the accumulators stay in registers).
__device__ __forceinline__ float f4_get(const float4 v, const int r) {
    return r == 0 ? v.x : (r == 1 ? v.y : (r == 2 ? v.z : v.w));
}
__device__ __forceinline__ float4 f4_scale(const float4 v, const int r, const float f) {
    return make_float4(r == 0 ? v.x * f : v.x, r == 1 ? v.y * f : v.y, r == 2 ? v.z * f : v.z, r == 3 ? v.w * f : v.w);
}

__device__ __forceinline__ float4 mfma4x4f32(const float a, const float b, const float4 c) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v r = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, f4v{c.x, c.y, c.z, c.w}, 0, 0, 0);
    return make_float4(r[0], r[1], r[2], r[3]);
}

// FP32 tiers of the workgroup's share (16-token tiles [d0, d1)) on the
// matrix cores in f32 (v_mfma_f32_16x16x4_f32: the tier values are the
// operands as they are stored). Wave w takes tiles d0 + w, d0 + w + 4, ...;
// the caller has already issued the loads of the first one into `t0`.
//   QK: D[token][head] = sum_c K[token][c] Q[head][c], channels 32 g + i of
//       MFMA i in lane group g; lane (g, n) receives the logits of tokens
//       4 g .. 4 g + 3 for head n (columns past the group's heads are unused).
//   PV: O[head][c] = sum_t P[head][t] V[t][c], MFMA (j, b) over the tokens
//       4 g + j (k = g), whose A operand is the QK result's register j as it
//       lies, and channel 8 n + b in column n; lane (g, n) accumulates heads
//       4 g .. 4 g + 3, channels 8 n + b.
// Softmax online in log2 units with a lazy reference: a head's reference
// moves only when a tile's maximum passes it by more than 16 (f32 holds the
// 2^16 factor), so most tiles skip the rescale. Leaves one (max, sum,
// acc[128]) partial per head in `dl` ([GP][2 + 128] per wave) and writes
// the logits.
template <int GP>
__device__ __forceinline__ void dense_share(const SplitArgs& a, const DenseView& dv, const int d0, const int d1,
                                            const int kvh, const int g0, const int gc, const int wave,
                                            const float* q_l, const DenseTile& t0, float* dl) {
    static_assert(GP <= 16, "one MFMA column per query head");
    constexpr float kTau = 16.0f;
    const AttnInputs& in = a.in;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const int G = in.Hq / in.Hkv;
    const int Nd = dv.Nd;
    float4 acc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[b] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float m_run = kNegInf, l_run = 0.0f;
    auto consume = [&](const DenseTile& t, const int k) {
        const int tok0 = 16 * k + 4 * g;
        // read per tile (an opaque offset keeps the compiler from holding
        // the 32 query values over the loop)
        int qo = n * kMfD + 32 * g;
        asm volatile("" : "+v"(qo));
        const float* qrow = q_l + qo;
        float4 d = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 qb = *reinterpret_cast<const float4*>(qrow + 4 * i);
            d = mfma4x4f32(t.k[i].x, qb.x, d);
            d = mfma4x4f32(t.k[i].y, qb.y, d);
            d = mfma4x4f32(t.k[i].z, qb.z, d);
            d = mfma4x4f32(t.k[i].w, qb.w, d);
        }
        float sv[4] = {d.x * a.scale2, d.y * a.scale2, d.z * a.scale2, d.w * a.scale2};
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[r] = (tok0 + r < Nd) ? sv[r] : kNegInf;
        if (a.logits && n < gc) {
            float* lr = a.logits + static_cast<size_t>(kvh * G + g0 + n) * a.ld + tok0;
            if (tok0 + 4 <= Nd) {
                st_dev4(a.logits, static_cast<uint32_t>(in.Hq) * a.ld * 4u, static_cast<uint32_t>((lr - a.logits) * 4),
                        make_float4(sv[0], sv[1], sv[2], sv[3]));
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (tok0 + r < Nd) lr[r] = sv[r];
            }
        }
        // the head's maximum over the tile (the four lane groups of column n)
        const float hm = xrow_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
        if (__ballot(hm > m_run + kTau)) {
            const bool up = hm > m_run + kTau;
            const float mn = up ? hm : m_run;
            const float al = (m_run == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(m_run - mn);
            l_run *= al;
            // accumulator row r of lane group g is head 4 g + r, whose factor
            // sits in column 4 g + r
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float ar = __shfl(al, 4 * g + r, 64);
#pragma unroll
                for (int b = 0; b < 8; ++b) acc[b] = f4_scale(acc[b], r, ar);
            }
            m_run = mn;
        }
        float pv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pv[r] = (sv[r] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(sv[r] - m_run);
        l_run += (pv[0] + pv[1]) + (pv[2] + pv[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float vv[8] = {t.v[j][0].x, t.v[j][0].y, t.v[j][0].z, t.v[j][0].w,
                                 t.v[j][1].x, t.v[j][1].y, t.v[j][1].z, t.v[j][1].w};
#pragma unroll
            for (int b = 0; b < 8; ++b) acc[b] = mfma4x4f32(pv[j], vv[b], acc[b]);
        }
    };
    int kb = d0 + wave;
    if (kb < d1) {
        consume(t0, kb);  // in flight since the start of the kernel
        kb += 4;
    }
#pragma unroll 1
    for (int k = kb; k < d1; k += 4) {
        DenseTile t;
        dense_load(in, dv, kvh, k, t);
        consume(t, k);
    }
    // The head's sum over its four lane groups, then the partial in LDS:
    // lane (0, h) holds (m, l) of head h, lane (g, n) the accumulators of
    // heads 4 g + r, channels 8 n .. 8 n + 7.
    l_run = xrow_sum(l_run);
    float* my = dl + wave * GP * (2 + kMfD);
    if (g == 0 && n < GP) {
        my[n * (2 + kMfD)] = m_run;
        my[n * (2 + kMfD) + 1] = l_run;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int h = 4 * g + r;
        if (h < GP) {
            float* pg = my + h * (2 + kMfD) + 2 + 8 * n;
#pragma unroll
            for (int b = 0; b < 8; ++b) pg[b] = f4_get(acc[b], r);
        }
    }
}

// One FP32-tier workgroup: KV head kvh, query heads [GP * chunk, +GP), FP32
// tiles [d0, d1) of share `dsplit`. The four waves' partials merge in LDS
// into partial slot nsplit_p + dsplit of each head.
template <int GP, bool PAIR = false>
__device__ __forceinline__ void dense_body(const SplitArgs& a, const int dsplit, const int kvh, const int chunk,
                                           char* lds) {
    using L = DnLds<GP>;
    const AttnInputs& in = a.in;
    const int G = in.Hq / in.Hkv;
    const int g0 = chunk * GP;
    const int gc = min(GP, G - g0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const DenseView dv = dense_view(in);
    int d0, d1;
    dense_range(a, dv.Nd, dsplit, d0, d1);
    float* q_l = reinterpret_cast<float*>(lds + L::QL);
    float* dl = reinterpret_cast<float*>(lds + L::PART);
    load_q_lds<16, PAIR>(in, kvh, g0, gc, q_l);  // rows past the group's heads are zeros
    if (a.dense_delay > 0) {
        // bounded by the constant-rate real-time counter
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        while (__builtin_amdgcn_s_memrealtime() - t0 < static_cast<unsigned long long>(a.dense_delay))
            __builtin_amdgcn_s_sleep(8);
    }
    if constexpr (GP <= 2) {
        DenseTileV dt;
        if (d0 + wave < d1) dense_load(in, dv, kvh, d0 + wave, dt);
        __syncthreads();
        dense_share_valu<GP>(a, dv, d0, d1, kvh, g0, gc, wave, q_l, dt, dl);
    } else {
        DenseTile dt;
        if (d0 + wave < d1) dense_load(in, dv, kvh, d0 + wave, dt);
        __syncthreads();
        dense_share<GP>(a, dv, d0, d1, kvh, g0, gc, wave, q_l, dt, dl);
    }
    __syncthreads();
    const int split = a.nsplit_p + dsplit;
    for (int idx = threadIdx.x; idx < gc * kMfD; idx += 256) {
        const int g = idx / kMfD, c = idx - g * kMfD;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, dl[(w * GP + g) * (2 + kMfD)]);
        float A = 0.0f, Ls = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float* dg = dl + (w * GP + g) * (2 + kMfD);
            const float f = (dg[0] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(dg[0] - M);  // waves without tiles add nothing
            A = __builtin_fmaf(f, dg[2 + c], A);
            Ls = __builtin_fmaf(f, dg[1], Ls);
        }
        const size_t pi = static_cast<size_t>(kvh * G + g0 + g) * a.nsplit + split;
        st_dev1(a.part_acc + pi * kMfD + c, A);
        if (c == 0) {
            st_dev1(a.part_ml + 2 * pi, (Ls > 0.0f) ? M : kNegInf);
            st_dev1(a.part_ml + 2 * pi + 1, Ls);
        }
    }
}

// One packed workgroup: KV head kvh, query heads [GP * chunk, +GP), a
// contiguous range of 32-token pairs of packed tiles; each wave takes a
// contiguous quarter of it. Writes partial slot `split` of each head.
//
// The high and low f16 halves of the QK coefficients sit in MFMA columns
// h and h + 8, so one MFMA per 32 channels yields both products; a DPP
// row rotation by 8 adds them, after which columns h and h + 8 carry the same
// logits and run the same softmax. The PV operand likewise puts p vs high in
// row h and low in row h + 8; the two accumulator rows are added once at the
// end. Columns / rows of padding heads repeat head 0 and are never stored.
//
// Four heads fill only half of those columns, so there the two tiles of a
// pair share one score block instead (TP): tile T sits in columns 4T + h
// (high) and 8 + 4T + h (low). Its four QK MFMAs read a zero coefficient row
// in the other tile's columns, so one accumulator chain over both tiles
// leaves every column the logits of its own tile, and each lane runs the
// softmax over 4 tokens rather than 8. In the PV operand the K elements
// of the other tile are zero, which keeps the token order of the V codes.
template <int GP, typename MetaT, bool PAIR = false>
__device__ __forceinline__ void packed_body(const SplitArgs& a, const int split, const int kvh, const int chunk,
                                            char* lds) {
    static_assert(GP >= 1 && GP <= 8, "at most 8 query heads per workgroup");
    constexpr int NP = GP >= 4 ? GP / 4 : 1;  // coefficient passes (4 heads x 16 chunks each)
    using L = MfLds<GP>;
    const AttnInputs& in = a.in;
    const int G = in.Hq / in.Hkv;
    const int g0 = chunk * GP;
    const int gc = min(GP, G - g0);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loop control
    const int n = lane & 15;   // MFMA column (QK) / channel group (PV); chunk of 8 channels (coefficients)
    const int gk = lane >> 4;  // MFMA reduction group
    const int hn = n & 7;      // query head of column n
    const bool lo_col = n >= 8;
    const float negm_col = lo_col ? -1.0f : 0.0f;  // PV operand: lo rows take the remainder
    constexpr bool TP = GP == 4;
    constexpr int NT = TP ? 1 : 2;                 // tiles held by one lane's scores
    const int ctile = TP ? (n >> 2) & 1 : 0;       // TP: the tile of column n
    const int chead = TP ? n & 3 : hn;             // query head of column n
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
    const int pb = part_begin(P, split, a.nsplit_p);
    const int pe = part_begin(P, split + 1, a.nsplit_p);
    const int tstride = Hkv * kMfD;         // words (or meta entries) between tiles / blocks of one head
    const int vstride = Hkv * (kMfD / 16);  // V words between tokens

    char* wl = lds + wave * L::BYTES;
    uint32_t* kt_l = reinterpret_cast<uint32_t*>(wl + L::KT);
    uint32_t* vt_l = reinterpret_cast<uint32_t*>(wl + L::VT);
    float* ksz_l = reinterpret_cast<float*>(wl + L::KSZ);
    float* vs_l = reinterpret_cast<float*>(wl + L::VS);
    float* vz_l = reinterpret_cast<float*>(wl + L::VZ);
    float* bias_l = reinterpret_cast<float*>(wl + L::BIAS);
    char* bhl_l = wl + L::BHL;

    // The query heads first (the barrier below waits for them only), then the
    // wave's first pair of packed tiles, whose latency overlaps theirs.
    float* q_l = reinterpret_cast<float*>(lds + L::QL);
    load_q_lds<GP, PAIR>(in, kvh, g0, gc, q_l);
    const int32_t* kp_h = in.kp + kvh * kMfD;
    const MetaT* ks_h = static_cast<const MetaT*>(in.ks) + kvh * kMfD;
    const MetaT* kz_h = static_cast<const MetaT*>(in.kz) + kvh * kMfD;
    const int32_t* vp_h = in.vp + kvh * (kMfD / 16);
    // V scale / zero per (token, KV head); paired heads: the two of the pair, adjacent
    const int hkv_m = PAIR ? 2 * Hkv : Hkv;
    const MetaT* vs_h = static_cast<const MetaT*>(in.vs) + (PAIR ? 2 * kvh : kvh);
    const MetaT* vz_h = static_cast<const MetaT*>(in.vz) + (PAIR ? 2 * kvh : kvh);
    const int lk = 4 * (lane & 31);
    const int tv = 4 * (lane >> 3) + (lane & 3);
    const int hfo = 4 * ((lane >> 2) & 1);
    const int t2 = lane & 31;

    // Per-lane byte offsets of a pair's loads from the pair's (wave-uniform)
    // base addresses, so the loads take a scalar base and a 32-bit lane
    // offset: those of a whole pair, and those of the store's last pair, which
    // may hold one tile (kto = 0 for both halves) and fewer slots (lanes past
    // the end re-read the last slot and are masked).
    struct PairOffs {
        uint32_t k, km, v, vm, id;
    };
    auto pair_offs = [&](const int kto, const int lim) {
        const int ts = min(t2, lim);
        return PairOffs{static_cast<uint32_t>(kto * tstride + lk) * 4u,
                        static_cast<uint32_t>(((W == 2) ? 0 : kto) * tstride + lk) * static_cast<uint32_t>(sizeof(MetaT)),
                        static_cast<uint32_t>(min(tv, lim) * vstride + hfo) * 4u,
                        static_cast<uint32_t>(ts * hkv_m) * static_cast<uint32_t>(sizeof(MetaT)),
                        static_cast<uint32_t>(ts) * 8u};
    };
    const PairOffs off_full = pair_offs(lane >> 5, 31);
    const int lim_last = nslots - 1 - 32 * (P - 1);
    const PairOffs off_last = pair_offs(min(lane >> 5, Tp - 1 - 2 * (P - 1)), lim_last);

    // Registers of the pair being fetched.
    using MR = MetaRaw<MetaT>;
    mf_u4 kw, vw;
    typename MR::Four ksr, kzr;
    typename MR::One vm = 0;
    typename MR::Two vm2{};
    long long idv = -1;
    bool okv = false;

    // Wave-uniform bases (scalar) plus the per-lane offsets.
    auto at = [](const void* base, const uint32_t off) { return static_cast<const char*>(base) + off; };
    auto fetch_at = [&](const int p, const PairOffs& o) {
        const size_t kb = static_cast<size_t>(2 * p) * tstride;
        const size_t mb = static_cast<size_t>((W == 2) ? p : 2 * p) * tstride;
        const size_t s0 = static_cast<size_t>(32 * p);
        kw = __builtin_nontemporal_load(reinterpret_cast<const mf_u4*>(at(kp_h + kb, o.k)));
        ksr = MR::load4(reinterpret_cast<const MetaT*>(at(ks_h + mb, o.km)));
        kzr = MR::load4(reinterpret_cast<const MetaT*>(at(kz_h + mb, o.km)));
        vw = *reinterpret_cast<const mf_u4*>(at(vp_h + s0 * vstride, o.v));
        // V scale in lanes 0-31, V zero in lanes 32-63 (two half-wave loads)
        if constexpr (PAIR) {
            if (lane < 32)
                vm2 = MR::load2(reinterpret_cast<const MetaT*>(at(vs_h + s0 * hkv_m, o.vm)));
            else
                vm2 = MR::load2(reinterpret_cast<const MetaT*>(at(vz_h + s0 * hkv_m, o.vm)));
        } else {
            if (lane < 32)
                vm = MR::load1(reinterpret_cast<const MetaT*>(at(vs_h + s0 * Hkv, o.vm)));
            else
                vm = MR::load1(reinterpret_cast<const MetaT*>(at(vz_h + s0 * Hkv, o.vm)));
        }
        idv = *reinterpret_cast<const long long*>(at(in.ids + s0, o.id));
    };
    auto fetch = [&](const int p) {
        if (p == P - 1) {
            fetch_at(p, off_last);
            okv = t2 <= lim_last;
        } else {
            fetch_at(p, off_full);
            okv = true;
        }
    };

    // this wave's quarter of the workgroup's pairs
    const int wp0 = pb + part_begin(pe - pb, wave, 4);
    const int wp1 = pb + part_begin(pe - pb, wave + 1, 4);
    if (wp0 < wp1) fetch(wp0);
    if (TP && threadIdx.x < 64) reinterpret_cast<uint32_t*>(lds + L::ZERO)[threadIdx.x] = 0u;
    __syncthreads();

    // Q' = Q 2^-e per head (e = exponent of max |Q_h|) in the coefficient
    // layout: pass pp, head 4 pp + gk, channels 8 n .. 8 n + 7.
    float qv[NP][8];
    float cpass[NP];
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
        const int h = 4 * pp + gk;
        {
            // heads past gc are zero in q_l
            const float* qp = q_l + (h < GP ? h : 0) * kMfD + 8 * n;
            const float4 x0 = *reinterpret_cast<const float4*>(qp);
            const float4 x1 = *reinterpret_cast<const float4*>(qp + 4);
            const bool hv = h < GP;
            qv[pp][0] = hv ? x0.x : 0.0f; qv[pp][1] = hv ? x0.y : 0.0f;
            qv[pp][2] = hv ? x0.z : 0.0f; qv[pp][3] = hv ? x0.w : 0.0f;
            qv[pp][4] = hv ? x1.x : 0.0f; qv[pp][5] = hv ? x1.y : 0.0f;
            qv[pp][6] = hv ? x1.z : 0.0f; qv[pp][7] = hv ? x1.w : 0.0f;
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
    // Column scale of query head chead: lane 16 (chead & 3) of pass chead >> 2 holds it.
    float ccol = 0.0f;
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
        const float t = __shfl(cpass[pp], 16 * (chead & 3), 64);
        if ((chead >> 2) == pp) ccol = t;
    }
    float crow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) crow[r] = __builtin_amdgcn_ldexpf(ccol, -2 * r);
    const int bhead = chead < GP ? chead : 0;
    const int brow = bhead + (lo_col ? GP : 0);
    const char* zero_l = lds + L::ZERO;

    const uint32_t kmask = (3u << (2 * (lane & 3))) | (3u << (16 + 2 * (lane & 3)));
    uint32_t one024;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(one024));
    // byte selectors of the V transpose (paired eight-head groups recompute
    // them in the lay-out from an opaque copy of the thread id: held over the
    // loop they would push that kernel past 168 VGPRs)
    constexpr bool kLeanSel = PAIR && GP == 8;
    const uint32_t qsel1_c = (lane & 1) ? 0x03070105u : 0x06020400u;
    const uint32_t qsel2_c = (lane & 2) ? 0x03020706u : 0x05040100u;

    mf_f4 acc[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[s] = mf_f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -1.0e30f, l_run = 0.0f, pz = 0.0f;

    // Lays the fetched pair out in LDS; returns the token-validity mask.
    auto stage = [&]() -> uint32_t {
        // K: bytes tq of channels c..c+3 -> one dword per token quad.
        const uint32_t u0 = __builtin_amdgcn_perm(kw.y, kw.x, 0x05010400u);
        const uint32_t u1 = __builtin_amdgcn_perm(kw.y, kw.x, 0x07030602u);
        const uint32_t v0 = __builtin_amdgcn_perm(kw.w, kw.z, 0x05010400u);
        const uint32_t v1 = __builtin_amdgcn_perm(kw.w, kw.z, 0x07030602u);
        uint32_t* kd = kt_l + (lane >> 5) * 4 * kKTS + (lane & 31);
        kd[0] = __builtin_amdgcn_perm(v0, u0, 0x05040100u);
        kd[kKTS] = __builtin_amdgcn_perm(v0, u0, 0x07060302u);
        kd[2 * kKTS] = __builtin_amdgcn_perm(v1, u1, 0x05040100u);
        kd[3 * kKTS] = __builtin_amdgcn_perm(v1, u1, 0x07060302u);
        // V: 4x4 byte transpose across the quad (tokens 4m..4m+3).
        const int m = lane >> 3;
        const int hf = (lane >> 2) & 1;
        const uint32_t vwv[4] = {vw.x, vw.y, vw.z, vw.w};
        uint32_t qsel1 = qsel1_c, qsel2 = qsel2_c;
        if constexpr (kLeanSel) {
            int tx = static_cast<int>(threadIdx.x);
            asm volatile("" : "+v"(tx));
            qsel1 = (tx & 1) ? 0x03070105u : 0x06020400u;
            qsel2 = (tx & 2) ? 0x03020706u : 0x05040100u;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t x = vwv[g];
            const uint32_t t = __builtin_amdgcn_perm(dpp_u32_quad1(x), x, qsel1);
            const uint32_t y = __builtin_amdgcn_perm(dpp_u32_quad2(t), t, qsel2);
            // byte column 4 (4 hf + g) + (lane & 3), token-quad dword 2 (m & 3) + (m >> 2)
            vt_l[vt_dword(16 * hf + 4 * g + (lane & 3), 2 * (m & 3) + (m >> 2))] = y;
        }
        float* kzd = ksz_l + (lane >> 5) * 2 * kKSZ + lk + 4 * ((lane & 31) >> 3);
        *reinterpret_cast<float4*>(kzd) = MR::f4(ksr);
        *reinterpret_cast<float4*>(kzd + kKSZ) = MR::f4(kzr);
        const bool ok = okv && idv != -1;
        const int pos = 8 * ((t2 & 15) >> 2) + 4 * (t2 >> 4) + (t2 & 3);
        // lanes 32-63 hold the token's zero, lanes 0-31 its scale: the zero of
        // the centred codes is vz + 1.5 vs (the middle of the row's range)
        if constexpr (PAIR) {
            // both heads of the pair: half 0 at [0, 32), half 1 at [32, 64)
            const float2 mv = MR::f2(vm2);
            const auto sx = __builtin_amdgcn_permlane32_swap(__float_as_uint(mv.x), __float_as_uint(mv.x), false, false);
            const auto sy = __builtin_amdgcn_permlane32_swap(__float_as_uint(mv.y), __float_as_uint(mv.y), false, false);
            const float mx = lane < 32 ? mv.x : __builtin_fmaf(1.5f, __uint_as_float(sx[0]), mv.x);
            const float my = lane < 32 ? mv.y : __builtin_fmaf(1.5f, __uint_as_float(sy[0]), mv.y);
            float* dst = lane < 32 ? vs_l : vz_l;
            dst[pos] = ok ? mx : 0.0f;  // masked slots contribute nothing
            dst[32 + pos] = ok ? my : 0.0f;
        } else {
            const float mv = MR::f1(vm);
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mv), __float_as_uint(mv), false, false);
            const float mc = lane < 32 ? mv : __builtin_fmaf(1.5f, __uint_as_float(sw[0]), mv);
            (lane < 32 ? vs_l : vz_l)[pos] = ok ? mc : 0.0f;  // masked slots contribute nothing
        }
        return static_cast<uint32_t>(__ballot(ok));
    };

    // QK coefficients of one tile's block: hi in rows h, lo in rows GP + h.
    auto coeffs = [&](const int tile, const int slot) {
        char* bt = bhl_l + slot * L::BHL_TILE;
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) {
            const int h = 4 * pp + gk;
            const float* kss = ksz_l + tile * 2 * kKSZ + 8 * n + 4 * (n >> 2);
            const float4 sa = *reinterpret_cast<const float4*>(kss);
            const float4 sb = *reinterpret_cast<const float4*>(kss + 4);
            const float4 za = *reinterpret_cast<const float4*>(kss + kKSZ);
            const float4 zb = *reinterpret_cast<const float4*>(kss + kKSZ + 4);
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
            if (GP >= 4 || h < GP) {
                *reinterpret_cast<mf_u4*>(bt + (h * kBRS + 8 * n) * 2) = hi;
                *reinterpret_cast<mf_u4*>(bt + ((GP + h) * kBRS + 8 * n) * 2) = lo;
                bias_l[slot * 8 + h] = bp;  // the 16 lanes of the row hold the same total
            }
        }
    };

    constexpr int kLbTok = L::LB_PAIRS * 32;  // logits per head in the buffer (rows of L::LB_HEAD floats)
    float* lb = reinterpret_cast<float*>(lds + L::LB + wave * L::LB_WAVE);
    int pbuf = wp0;  // first pair held in the logits buffer
    // Stores the buffered pairs [pbuf, q1) (the caller orders the buffer's LDS
    // writes first): lane = (head, token quad) with kLbTok / 4 quads per head,
    // quads past the held pairs idle.
    auto flush_lb = [&](const int q1) {
        constexpr int kQuads = kLbTok > 0 ? kLbTok / 4 : 64;  // a power of two
        constexpr int kHeadsPass = 64 / kQuads;
        const int qd = lane & (kQuads - 1);
        const int tok = 32 * pbuf + 4 * qd;
        if (qd < (q1 - pbuf) * 8) {
#pragma unroll
            for (int h0 = 0; h0 < GP; h0 += kHeadsPass) {
                const int hh = h0 + lane / kQuads;
                if (hh < gc) {
                    const float4 v = *reinterpret_cast<const float4*>(lb + hh * L::LB_HEAD + 4 * qd);
                    float* dst = a.logits + static_cast<size_t>(kvh * G + g0 + hh) * a.ld + Nd + tok;
                    if (tok + 4 <= nslots) {
                        st_dev4(a.logits, static_cast<uint32_t>(a.in.Hq) * a.ld * 4u,
                                static_cast<uint32_t>((dst - a.logits) * 4), v);
                    } else {
                        if (tok < nslots) dst[0] = v.x;
                        if (tok + 1 < nslots) dst[1] = v.y;
                        if (tok + 2 < nslots) dst[2] = v.z;
                    }
                }
            }
        }
    };
    for (int p = wp0; p < wp1; ++p) {
        // Issue priority by the pairs still to do: the SIMD arbiter otherwise
        // favours the oldest waves, so the workgroups of the first dispatch
        // round finish ~3 us before those of the second and the launch ends
        // at low occupancy. Waves with more work left issue first, and the
        // waves of a CU finish closer together (1-2% per launch with one to
        // four heads per group; neutral with eight, which keeps the default).
        if constexpr (GP <= 4) {
            const int rem = wp1 - p;  // this pair included
            if (rem >= 4)
                __builtin_amdgcn_s_setprio(3);
            else if (rem == 3)
                __builtin_amdgcn_s_setprio(2);
            else if (rem == 2)
                __builtin_amdgcn_s_setprio(1);
            else
                __builtin_amdgcn_s_setprio(0);
        }
        const uint32_t vmask = stage();
        if (p + 1 < wp1) fetch(p + 1);
        // the stores go out early in the pair, so they are acknowledged before
        // the next lay-out waits for the fetch just issued
        if (L::LB_PAIRS > 0 && a.logits && p - pbuf == L::LB_PAIRS) {
            wave_lds_sync();
            flush_lb(p);
            wave_lds_sync();
            pbuf = p;
        }
        wave_lds_sync();
        coeffs(0, 0);
        if (W == 1 && L::NBT == 2) coeffs(1, 1);
        wave_lds_sync();

        // s2[i][r]: logit of token 4 gk + r of tile tt(i) in column n, tt(i) = ctile
        // with the tiles packed (TP), else i.
        float s2[NT][4];
        auto tt = [&](const int i) { return TP ? ctile : i; };
        // V scale / zero of this lane's tokens ([tile 0 r 0..3, tile 1 r 0..3] at 8 gk)
        // and the pair's V codes. Four-head groups read them ahead of the QK
        // MFMAs (off the chain that follows them); eight-head groups after the
        // scores, as read ahead they would not fit in 168 VGPRs.
        float vsv[NT][4], vzv[NT][4];
        uint2 q0, q1;
        auto read_v = [&]() {
            // paired heads: the V scale / zero of the column's own head
            const int vh = PAIR ? 32 * min(1, (g0 + bhead) / (G >> 1)) : 0;
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const float4 vq = *reinterpret_cast<const float4*>(vs_l + vh + 8 * gk + 4 * tt(i));
                const float4 zq = *reinterpret_cast<const float4*>(vz_l + vh + 8 * gk + 4 * tt(i));
                vsv[i][0] = vq.x; vsv[i][1] = vq.y; vsv[i][2] = vq.z; vsv[i][3] = vq.w;
                vzv[i][0] = zq.x; vzv[i][1] = zq.y; vzv[i][2] = zq.z; vzv[i][3] = zq.w;
            }
            const int d0 = vt_dword(n, 2 * gk), d1 = vt_dword(n + 16, 2 * gk);
            q0 = *reinterpret_cast<const uint2*>(vt_l + d0);
            q1 = make_uint2(vt_l[d1], vt_l[d1 + 1]);
        };
        if constexpr (TP) read_v();
        if constexpr (TP) {
            // a chain per tile; the other tile's columns read the zero row
            mf_f4 dt[2];
#pragma unroll
            for (int tile = 0; tile < 2; ++tile) {
                mf_f4& d = dt[tile];
                d = mf_f4{0.0f, 0.0f, 0.0f, 0.0f};
                const int tb = (W == 2) ? 0 : tile;
                const mf_u4* ka = reinterpret_cast<const mf_u4*>(kt_l + (tile * 4 + ((lane & 15) >> 2)) * kKTS + 8 * gk);
                const mf_u4 ra = ka[0], rb = ka[1];
                const char* kbase =
                    (tile == ctile) ? bhl_l + tb * L::BHL_TILE + (brow * kBRS + 32 * gk) * 2 : zero_l + 64 * gk;
                const mf_u4* kb = reinterpret_cast<const mf_u4*>(kbase);
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const uint32_t x = (s < 2) ? ra[2 * s] : rb[2 * s - 4];
                    const uint32_t y = (s < 2) ? ra[2 * s + 1] : rb[2 * s - 3];
                    const mf_u4 av = {code_f16(x, kmask, one024), code_f16(x >> 8, kmask, one024),
                                      code_f16(y, kmask, one024), code_f16(y >> 8, kmask, one024)};
                    d = mfma16x16x32(av, kb[s], d);
                }
            }
            const float bc = bias_l[((W == 2) ? 0 : ctile) * 8 + bhead] * ccol;
            const mf_f4 d = dt[0] + dt[1];
#pragma unroll
            for (int r = 0; r < 4; ++r) s2[0][r] = __builtin_fmaf(d[r] + dpp<0x128>(d[r]), crow[r], bc);
        } else {
#pragma unroll
            for (int tile = 0; tile < 2; ++tile) {
                const int tb = (W == 2 || L::NBT == 1) ? 0 : tile;
                if (W == 1 && L::NBT == 1 && tile == 1) {
                    wave_lds_sync();  // tile 0's coefficients and bias are read
                    coeffs(1, 0);
                    wave_lds_sync();
                }
                // A: codes of token t = lane & 15 (k = t & 3), channels 32 gk .. 32 gk + 31.
                const mf_u4* ka = reinterpret_cast<const mf_u4*>(kt_l + (tile * 4 + ((lane & 15) >> 2)) * kKTS + 8 * gk);
                const mf_u4 ra = ka[0], rb = ka[1];
                const mf_u4* kb = reinterpret_cast<const mf_u4*>(bhl_l + tb * L::BHL_TILE + (brow * kBRS + 32 * gk) * 2);
                mf_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const uint32_t x = (s < 2) ? ra[2 * s] : rb[2 * s - 4];
                    const uint32_t y = (s < 2) ? ra[2 * s + 1] : rb[2 * s - 3];
                    const mf_u4 av = {code_f16(x, kmask, one024), code_f16(x >> 8, kmask, one024),
                                      code_f16(y, kmask, one024), code_f16(y >> 8, kmask, one024)};
                    d = mfma16x16x32(av, kb[s], d);
                }
                const float bc = bias_l[tb * 8 + bhead] * ccol;
#pragma unroll
                for (int r = 0; r < 4; ++r) s2[tile][r] = __builtin_fmaf(d[r] + dpp<0x128>(d[r]), crow[r], bc);
            }
        }

        const bool full = (vmask == 0xffffffffu);
        if (!full) {
#pragma unroll
            for (int i = 0; i < NT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (!((vmask >> (16 * tt(i) + 4 * gk + r)) & 1u)) s2[i][r] = kNegInf;
        }
        // The columns of the high parts leave the logits of their head in the
        // wave's buffer (stored when the buffer is full or the loop ends), or
        // with eight heads in memory directly.
        if (L::LB_PAIRS > 0 && a.logits && !lo_col && chead < GP) {
#pragma unroll
            for (int i = 0; i < NT; ++i)
                *reinterpret_cast<float4*>(lb + chead * L::LB_HEAD + 32 * (p - pbuf) + 16 * tt(i) + 4 * gk) =
                    make_float4(s2[i][0], s2[i][1], s2[i][2], s2[i][3]);
        }
        if (L::LB_PAIRS == 0 && a.logits && !lo_col && chead < gc) {
            float* row = a.logits + static_cast<size_t>(kvh * G + g0 + chead) * a.ld + Nd + 32 * p + 4 * gk;
            if (32 * p + 32 <= nslots) {
#pragma unroll
                for (int i = 0; i < NT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) row[16 * tt(i) + r] = s2[i][r];
            } else {
                // the store's last pair (rare): the token offset from an
                // opaque copy of the thread id, so that no register holds it
                // over the loop
                int tx = static_cast<int>(threadIdx.x);
                asm volatile("" : "+v"(tx));
                const int t0 = 32 * p + 4 * ((tx >> 4) & 3);
#pragma unroll
                for (int i = 0; i < NT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (t0 + 16 * tt(i) + r < nslots) row[16 * tt(i) + r] = s2[i][r];
            }
        }


        if constexpr (!TP) read_v();
        float mx = fmax_nn(fmax_nn(s2[0][0], s2[0][1]), fmax_nn(s2[0][2], s2[0][3]));
        float vmx = fmax_nn(fmax_abs_nn(vsv[0][0], vsv[0][1]), fmax_abs_nn(vsv[0][2], vsv[0][3]));
#pragma unroll
        for (int i = 1; i < NT; ++i) {
            mx = fmax_nn(mx, fmax_nn(fmax_nn(s2[i][0], s2[i][1]), fmax_nn(s2[i][2], s2[i][3])));
            vmx = fmax_nn(vmx, fmax_nn(fmax_abs_nn(vsv[i][0], vsv[i][1]), fmax_abs_nn(vsv[i][2], vsv[i][3])));
        }
        // Each lane tests the bound on its own tokens; the reductions over the
        // head's lanes (and the rescale) run only when some lane breaks it.
        const int evl = (vmx > 0.0f) ? __builtin_amdgcn_frexp_expf(vmx) : 0;
        if (__ballot(mx - static_cast<float>(13 - evl) > m_run + kMfTau)) {
            mx = xrow_max(mx);
            vmx = xrow_max(vmx);
            if constexpr (TP) {
                // column n +- 4 holds the same head's other tile
                mx = fmax_nn(mx, dpp<0x124>(mx));
                vmx = fmax_nn(vmx, dpp<0x124>(vmx));
            }
            const int ev = (vmx > 0.0f) ? __builtin_amdgcn_frexp_expf(vmx) : 0;
            const float cand = mx - static_cast<float>(13 - ev);
            const bool up = cand > m_run + kMfTau;  // uniform over the head's lanes
            const float mn = up ? cand : m_run;
            const float al = up ? __builtin_amdgcn_exp2f(m_run - mn) : 1.0f;
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

        float pv[NT][4];
        float lsum = 0.0f;
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(s2[i][r] - m_run);  // flushes below 2^-126
                lsum += e;
                pz = __builtin_fmaf(e, vzv[i][r], pz);
                pv[i][r] = e * vsv[i][r];
            }
        l_run += lsum;
        mf_u4 ap;
        if constexpr (TP) {
            // K elements 0..3 are tile 0's tokens, 4..7 tile 1's (the V code order)
            const uint32_t h0 = split_half(pv[0][0], pv[0][2], negm_col);
            const uint32_t h1 = split_half(pv[0][1], pv[0][3], negm_col);
            ap = ctile ? mf_u4{0u, 0u, h0, h1} : mf_u4{h0, h1, 0u, 0u};
        } else {
            ap = mf_u4{split_half(pv[0][0], pv[0][2], negm_col), split_half(pv[0][1], pv[0][3], negm_col),
                       split_half(pv[NT - 1][0], pv[NT - 1][2], negm_col),
                       split_half(pv[NT - 1][1], pv[NT - 1][3], negm_col)};
        }

        // B: centred codes of channel 4 beta + k for the lane's 8 tokens,
        // beta = n (nsteps 0..3) and n + 16 (nsteps 4..7), k = nstep & 3;
        // bytes 0 and 2 of a word shifted left by one, bytes 1 and 3 shifted
        // right by seven (the bit shifted into bit 0 is never selected).
        const uint32_t q0e = q0.x << 1, q0f = q0.y << 1, q1e = q1.x << 1, q1f = q1.y << 1;
        const uint32_t q0a = q0.x >> 7, q0b = q0.y >> 7, q1a = q1.x >> 7, q1b = q1.y >> 7;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t mk2 = (6u << (2 * k)) | (6u << (16 + 2 * k));
            const mf_u4 b0 = {code_f16_centred(q0e, mk2, one024, k), code_f16_centred(q0a, mk2, one024, k),
                              code_f16_centred(q0f, mk2, one024, k), code_f16_centred(q0b, mk2, one024, k)};
            acc[k] = mfma16x16x32(ap, b0, acc[k]);
            const mf_u4 b1 = {code_f16_centred(q1e, mk2, one024, k), code_f16_centred(q1a, mk2, one024, k),
                              code_f16_centred(q1f, mk2, one024, k), code_f16_centred(q1b, mk2, one024, k)};
            acc[4 + k] = mfma16x16x32(ap, b1, acc[4 + k]);
        }
        wave_lds_sync();
    }

    if (L::LB_PAIRS > 0 && a.logits && wp1 > pbuf) {
        wave_lds_sync();
        flush_lb(wp1);
    }
    l_run = xrow_sum(l_run);
    pz = xrow_sum(pz);
    if constexpr (TP) {
        // add the other tile's column of the head
        l_run += dpp<0x124>(l_run);
        pz += dpp<0x124>(pz);
    }

    // Merge of the four waves through LDS. Lane (g = lane / 16, n = lane % 16)
    // holds rows 4 g .. 4 g + 3 of the PV output, column n of each of the
    // eight MFMAs: row 4 g + r is head r of tile g & 1 (high parts g < 2, low
    // parts g >= 2) with packed tiles, else head (4 g + r) & 7 (high parts
    // g < 2). Every lane stores its raw accumulators (channels 4 n + 64 q ..
    // + 3 as one 16-byte write per (row, q)) and the merge threads add the
    // row groups of a head and the waves in one pass, instead of reducing
    // across lanes first.
    constexpr int RR = GP < 4 ? GP : 4;                  // rows of a group that hold heads
    constexpr int NGI = TP ? 4 : 2 * ((GP + 3) / 4);     // row groups that hold heads
    constexpr int XW = NGI * RR * kMfD;                  // floats per wave
    static_assert(4 * XW * 4 + 3 * 4 * GP * 4 <= 4 * L::BYTES, "merge area must fit in the staging area");
    __syncthreads();  // every wave is done with its staging area
    float* sm_x = reinterpret_cast<float*>(lds);  // [4 waves][NGI][RR][128]
    float* sm_m = sm_x + 4 * XW;                   // [4][GP]
    float* sm_l = sm_m + 4 * GP;                   // [4][GP]
    float* sm_z = sm_l + 4 * GP;                   // [4][GP]
    // The lane's indices again, from an opaque copy of the thread id: held
    // over the loop instead, they would cost registers the loop needs.
    int tx = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tx));
    const int lane_e = tx & 63, n_e = tx & 15, g_e = (tx >> 4) & 3;
    if (lane_e < GP) {
        sm_m[wave * GP + lane_e] = m_run;
        sm_l[wave * GP + lane_e] = l_run;
        sm_z[wave * GP + lane_e] = pz;
    }
    {
        // row group g_e -> slot gi (TP: all four; else the high group of
        // heads 4 (g & 1) .. and the low group of the same heads)
        const int gi = TP ? g_e : ((g_e & 1) + (g_e >> 1) * (NGI / 2));
        const bool keep = TP || ((g_e & 1) < NGI / 2);
        if (keep) {
            float* xw = sm_x + wave * XW + gi * RR * kMfD + 4 * n_e;
#pragma unroll
            for (int r = 0; r < RR; ++r)
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    *reinterpret_cast<float4*>(xw + r * kMfD + 64 * q) =
                        make_float4(acc[4 * q][r], acc[4 * q + 1][r], acc[4 * q + 2][r], acc[4 * q + 3][r]);
        }
    }
    __syncthreads();
    // Thread (head h, channels 4 c4 .. 4 c4 + 3). The codes were scaled by
    // 4^(c & 3) and centred as 2 q - 3, so channel c's sum carries 2^(2 (c & 3) + 1).
    for (int idx = threadIdx.x; idx < gc * (kMfD / 4); idx += 256) {
        const int h = idx / (kMfD / 4), c4 = idx - h * (kMfD / 4);
        float M = -1.0e30f;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w * GP + h]);
        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float Ls = 0.0f, Z = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            // a wave without pairs has m = -1e30, l = 0, acc = 0: it adds nothing
            const float f = __builtin_amdgcn_exp2f(sm_m[w * GP + h] - M);
            const float* xw = sm_x + w * XW + 4 * c4;
            float4 S;
            if constexpr (TP) {
                const float4 x0 = *reinterpret_cast<const float4*>(xw + (0 * RR + h) * kMfD);
                const float4 x1 = *reinterpret_cast<const float4*>(xw + (1 * RR + h) * kMfD);
                const float4 x2 = *reinterpret_cast<const float4*>(xw + (2 * RR + h) * kMfD);
                const float4 x3 = *reinterpret_cast<const float4*>(xw + (3 * RR + h) * kMfD);
                S = make_float4((x0.x + x1.x) + (x2.x + x3.x), (x0.y + x1.y) + (x2.y + x3.y),
                                (x0.z + x1.z) + (x2.z + x3.z), (x0.w + x1.w) + (x2.w + x3.w));
            } else {
                const int gh = h >> 2, r = h & 3;
                const float4 x0 = *reinterpret_cast<const float4*>(xw + (gh * RR + r) * kMfD);
                const float4 x1 = *reinterpret_cast<const float4*>(xw + ((NGI / 2 + gh) * RR + r) * kMfD);
                S = make_float4(x0.x + x1.x, x0.y + x1.y, x0.z + x1.z, x0.w + x1.w);
            }
            A.x = __builtin_fmaf(f, S.x, A.x);
            A.y = __builtin_fmaf(f, S.y, A.y);
            A.z = __builtin_fmaf(f, S.z, A.z);
            A.w = __builtin_fmaf(f, S.w, A.w);
            Z = __builtin_fmaf(f, sm_z[w * GP + h], Z);
            Ls = __builtin_fmaf(f, sm_l[w * GP + h], Ls);
        }
        A = make_float4(__builtin_fmaf(A.x, 0.5f, Z), __builtin_fmaf(A.y, 0.125f, Z),
                        __builtin_fmaf(A.z, 0.03125f, Z), __builtin_fmaf(A.w, 0.0078125f, Z));
        const size_t pi = static_cast<size_t>(kvh * G + g0 + h) * a.nsplit + split;
        st_dev4(a.part_acc, static_cast<uint32_t>(static_cast<size_t>(in.Hq) * a.nsplit * kMfD * 4u),
                static_cast<uint32_t>((pi * kMfD + 4 * c4) * 4), A);
        if (c4 == 0) {
            st_dev1(a.part_ml + 2 * pi, (Ls > 0.0f) ? M : kNegInf);
            st_dev1(a.part_ml + 2 * pi + 1, Ls);
        }
    }
}
