// tt_engine.hip -- device-resident TriTierCache engine (gfx950).
//
// Replaces TriTierCacheEngine (csrc/include/cache_engine.h:10-123,
// csrc/cache_engine.cpp). Every tier buffer and every counter lives in HBM; a
// decode step enqueues a handful of kernels and never waits for the device:
//
//   * the counters whose evolution does not depend on data (sink/ring fill,
//     ring head, total tokens, evictions, and the threshold recompute cadence
//     last_calc_pos) are mirrored on the host, so the host decides which
//     kernels to launch and with which ring slot / evicted id;
//   * the data-dependent tier decisions (heavy-hitter promotion, argmin
//     demotion, waiting-room fill and flush) run in one single-workgroup
//     kernel that reads the scores and counters from device memory;
//   * attention reads the tiers in place (no dense-assembly copy,
//     cache_engine.cpp:433-459) and the decayed score feedback is fused into
//     the mean-weight kernel.
//
// The packed store is allocated up front for max_seq_len tokens (plus a
// margin) instead of the reference's 64-block growth, so buffers never move
// in the decode loop; pbs_allocated_blocks still reports the reference's
// logical value, kept on the device by the flush/prefill code.
#include "tt_attn.h"
#include "tt_quant_dev.h"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <vector>

namespace tt {
namespace {

// ---------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------

// Sink / recent-window fill without eviction (cache_engine.cpp:406-413).
__global__ void __launch_bounds__(256) append_row_kernel(const float* __restrict__ k_new,
                                                         const float* __restrict__ v_new, float* __restrict__ k_dst,
                                                         float* __restrict__ v_dst, int kvs, int* st, int counter_slot) {
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < kvs; e += gridDim.x * blockDim.x) {
        k_dst[e] = k_new[e];
        v_dst[e] = v_new[e];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        st[counter_slot] += 1;
        st[kTotal] += 1;
    }
}

// Exact k-th smallest of g[0..n) by an MSB radix select on order-preserving
// keys, three passes of 11, 11 and 10 bits; any exact selection equals
// std::nth_element's pick (cache_engine.cpp:126-144). Writes the threshold
// and last_calc_pos. One workgroup: every thread keeps kThrBatch loads in
// flight per pass step, and the digit of each pass is found with a parallel
// prefix sum over the histogram.
constexpr int kThrBatch = 32;

__device__ __forceinline__ unsigned int wave_incl_scan(unsigned int x) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const unsigned int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    return x;
}

__global__ void __launch_bounds__(1024) threshold_kernel(const float* __restrict__ g, int n, long long k, int* st,
                                                         int total) {
    __shared__ unsigned int hist[2048];
    __shared__ unsigned int wtot[16];
    __shared__ unsigned int s_prefix, s_mask, s_k;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_k = static_cast<unsigned int>(k);  // k < n < 2^31
    }
    for (int pass = 0; pass < 3; ++pass) {
        const int bits = pass < 2 ? 11 : 10;
        const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
        const unsigned int dm = (1u << bits) - 1u;
        for (int i = tid; i < 2048; i += 1024) hist[i] = 0;
        __syncthreads();
        const unsigned int prefix = s_prefix, mask = s_mask;
        for (int base = 0; base < n; base += 1024 * kThrBatch) {
            unsigned int u[kThrBatch];
#pragma unroll
            for (int j = 0; j < kThrBatch; ++j) {
                const int i = base + j * 1024 + tid;
                u[j] = i < n ? __float_as_uint(g[i]) : 0u;
            }
#pragma unroll
            for (int j = 0; j < kThrBatch; ++j) {
                const unsigned int key = (u[j] & 0x80000000u) ? ~u[j] : (u[j] | 0x80000000u);
                if (base + j * 1024 + tid < n && (key & mask) == prefix) atomicAdd(&hist[(key >> shift) & dm], 1u);
            }
        }
        __syncthreads();
        // Thread t owns bins 2t and 2t + 1; the digit is the bin where the
        // running count passes s_k (exactly one thread finds it).
        const unsigned int h0 = hist[2 * tid], h1 = hist[2 * tid + 1];
        const unsigned int incl = wave_incl_scan(h0 + h1);
        if (lane == 63) wtot[wave] = incl;
        __syncthreads();
        unsigned int before = incl - (h0 + h1);
        for (int w = 0; w < wave; ++w) before += wtot[w];
        const unsigned int kk = s_k;
        __syncthreads();  // everyone has read s_k
        if (before <= kk && kk < before + h0 + h1) {
            const unsigned int d = (kk < before + h0) ? 2u * tid : 2u * tid + 1u;
            s_k = kk - before - (d & 1u ? h0 : 0u);
            s_prefix = prefix | (d << shift);
            s_mask = mask | (dm << shift);
        }
        __syncthreads();
    }
    if (tid == 0) {
        const unsigned int key = s_prefix;
        const unsigned int u = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
        st[kThreshold] = static_cast<int>(u);
        st[kLastCalcPos] = total;
    }
}

// The same selection spread over many workgroups: per pass, thr_hist_kernel
// adds the digit histogram of the candidates that match the prefix found so
// far into a global histogram (LDS histogram per workgroup, then one atomic
// per non-empty bin), and thr_select_kernel (one workgroup) finds the digit
// where the running count passes k, narrows prefix / mask / k, clears the
// histogram for the next pass and, after the last pass, writes the threshold.
// Selection state (`ts`): hist[2048], then prefix, mask, k; all zero between
// selections (the last pass leaves them so).
constexpr int kThrHistWgs = 64;   // at most, each 256 threads x kThrHistPer candidates per round
constexpr int kThrHistPer = 16;
constexpr int kThrStateWords = 2048 + 4;
// Candidate counts from which the six launches of the spread selection beat
// the single-workgroup kernel.
#ifndef TT_THR_MULTI_MIN
#define TT_THR_MULTI_MIN 16384
#endif
constexpr size_t kThrMultiMin = TT_THR_MULTI_MIN;

__device__ __forceinline__ int thr_bits(int pass) { return pass < 2 ? 11 : 10; }
__device__ __forceinline__ int thr_shift(int pass) { return pass == 0 ? 21 : (pass == 1 ? 10 : 0); }

__global__ void __launch_bounds__(256) thr_hist_kernel(const float* __restrict__ g, int n, int pass,
                                                       unsigned int* ts) {
    __shared__ unsigned int hist[2048];
    const int tid = threadIdx.x;
    for (int i = tid; i < 2048; i += 256) hist[i] = 0;
    __syncthreads();
    const int shift = thr_shift(pass);
    const unsigned int dm = (1u << thr_bits(pass)) - 1u;
    const unsigned int prefix = ts[2048], mask = ts[2049];
    const int stride = gridDim.x * 256 * kThrHistPer;
    for (int base = blockIdx.x * 256 * kThrHistPer; base < n; base += stride) {
        unsigned int u[kThrHistPer];
#pragma unroll
        for (int j = 0; j < kThrHistPer; ++j) {
            const int i = base + j * 256 + tid;
            u[j] = i < n ? __float_as_uint(g[i]) : 0u;
        }
#pragma unroll
        for (int j = 0; j < kThrHistPer; ++j) {
            const unsigned int key = (u[j] & 0x80000000u) ? ~u[j] : (u[j] | 0x80000000u);
            if (base + j * 256 + tid < n && (key & mask) == prefix) atomicAdd(&hist[(key >> shift) & dm], 1u);
        }
    }
    __syncthreads();
    for (int i = tid; i < 2048; i += 256)
        if (hist[i]) atomicAdd(&ts[i], hist[i]);
}

__global__ void __launch_bounds__(1024) thr_select_kernel(int pass, long long k0, unsigned int* ts, int* st,
                                                          int total) {
    __shared__ unsigned int wtot[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int shift = thr_shift(pass);
    const unsigned int dm = (1u << thr_bits(pass)) - 1u;
    const unsigned int prefix = ts[2048], mask = ts[2049];
    const unsigned int kk = pass == 0 ? static_cast<unsigned int>(k0) : ts[2050];  // k < n < 2^31
    // Thread t owns bins 2t and 2t + 1 (read, then cleared for the next pass).
    const unsigned int h0 = ts[2 * tid], h1 = ts[2 * tid + 1];
    ts[2 * tid] = 0;
    ts[2 * tid + 1] = 0;
    const unsigned int incl = wave_incl_scan(h0 + h1);
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    unsigned int before = incl - (h0 + h1);
    for (int w = 0; w < wave; ++w) before += wtot[w];
    if (before <= kk && kk < before + h0 + h1) {  // exactly one thread
        const unsigned int d = (kk < before + h0) ? 2u * tid : 2u * tid + 1u;
        const unsigned int np = prefix | (d << shift);
        if (pass == 2) {
            const unsigned int u = (np & 0x80000000u) ? (np & 0x7fffffffu) : ~np;
            st[kThreshold] = static_cast<int>(u);
            st[kLastCalcPos] = total;
            ts[2048] = 0;
            ts[2049] = 0;
            ts[2050] = 0;
        } else {
            ts[2048] = np;
            ts[2049] = mask | (dm << shift);
            ts[2050] = kk - before - (d & 1u ? h0 : 0u);
        }
    }
}

struct RouteArgs {
    int* st;
    const float* k_new;
    const float* v_new;
    float* rw_k;
    float* rw_v;
    float* hh_k;
    float* hh_v;
    float* wr_k;
    float* wr_v;
    float* ev_k;
    float* ev_v;
    int64_t* hh_ids;
    int64_t* wr_ids;
    int64_t* pbs_ids;
    float* hh_scores;
    const float* g;
    int32_t* kp;
    void* ks;
    void* kz;
    int32_t* vp;
    void* vs;
    void* vz;
    int kvs, H, D, kgs, chunk, max_hh, max_seq_len, fp16;
    int slot;
    long long evicted_id;
    int thr_zero;
    int new_head;
};

enum RouteCase : int { kToHH = 0, kReplace = 1, kToWR = 2 };
constexpr int kRouteRegs = 8;  // row elements per thread kept in registers by the route kernel

template <typename MetaT>
__device__ void flush_waiting_room(const RouteArgs& a, int blocks) {
    // cache_engine.cpp:148-207: quantise the waiting room (slot order) into
    // block `blocks`.
    const int kvs = a.kvs;
    const int words = a.kgs / 16;
    MetaT* ks = static_cast<MetaT*>(a.ks);
    MetaT* kz = static_cast<MetaT*>(a.kz);
    MetaT* vs = static_cast<MetaT*>(a.vs);
    MetaT* vz = static_cast<MetaT*>(a.vz);
    for (int hc = threadIdx.x; hc < kvs; hc += blockDim.x) {
        const int c = hc % a.D;
        const size_t mi = static_cast<size_t>(blocks) * kvs + hc;
        quant_k_channel<MetaT>(a.wr_k + hc, kvs, a.kgs, c < (a.D / 8) * 8, ks + mi, kz + mi,
                               reinterpret_cast<uint32_t*>(a.kp) + static_cast<size_t>(blocks) * words * kvs + hc,
                               kvs);
    }
    // V rows: one lane per packed word, a row's D / 16 words on an aligned
    // group of lanes padded to a power of two (head_dim a multiple of 16, at
    // most 256: at most 16 lanes, a group that divides blockDim), so a row's
    // lanes are never split between iterations.
    const int wpr = a.D / 16;
    const int group = quant_v_group(wpr);
    for (int th = threadIdx.x; th < a.chunk * a.H * group; th += blockDim.x) {
        const int r = th / group, w = th % group;
        const int t = r / a.H, h = r % a.H;
        const size_t mi = (static_cast<size_t>(blocks) * a.chunk + t) * a.H + h;
        quant_v_row_lanes<MetaT>(a.wr_v + static_cast<size_t>(t) * kvs + static_cast<size_t>(h) * a.D, w, wpr, group,
                                 vs + mi, vz + mi, a.vp + mi * wpr);
    }
    for (int t = threadIdx.x; t < a.chunk; t += blockDim.x)
        a.pbs_ids[static_cast<size_t>(blocks) * a.chunk + t] = a.wr_ids[t];
}

// Ring eviction + route_evicted_token (+ flush) for one step, in one
// workgroup (cache_engine.cpp:414-430, 209-269, 148-207).
// Order-preserving key of a heavy-hitter score for the argmin: the float's
// total order in the high word (-0 folded onto +0, which '<' does not tell
// apart), the slot in the low word, so the smallest key is the first slot
// of the minimum; NaNs get the largest key and never win.
__device__ __forceinline__ unsigned long long hh_key(const float v, const int i) {
    if (v != v) return ~0ull;
    const unsigned u = __float_as_uint(v + 0.0f);
    const unsigned o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(o) << 32) | static_cast<unsigned>(i);
}
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long k) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const unsigned long long o = __shfl_xor(k, m, 64);
        k = o < k ? o : k;
    }
    return k;
}
constexpr int kArgminBatch = 8;  // heavy-hitter scores per thread with their loads in flight together

__global__ void __launch_bounds__(1024) route_kernel(RouteArgs a) {
    __shared__ int s_case, s_min_idx;
    __shared__ float s_score;
    __shared__ unsigned long long red_k[16];
    const int tid = threadIdx.x;
    const int kvs = a.kvs;
    int* st = a.st;
    const int hh = st[kHhCount];
    const int wr = st[kWrCount];
    const int blocks = st[kBlocksUsed];
    const int evictions = st[kTotalEvictions], total = st[kTotal];
    const int logical = st[kLogicalAlloc], pbs_count = st[kPbsCount];

    // Score and threshold (cache_engine.cpp:216-218).
    // (read without a branch around it, so that the kernel arguments it needs
    // come in the first batch of argument loads: g holds max_seq_len >= 1 scores)
    const long long eid = a.evicted_id;
    const bool eid_ok = eid >= 0 && eid < a.max_seq_len;
    const float g_ev = a.g[eid_ok ? eid : 0];
    const float score = eid_ok ? g_ev : 0.0f;
    const float thr = a.thr_zero ? 0.0f : __int_as_float(st[kThreshold]);

    // Evicted row out of the ring slot, new token in (each thread owns the
    // same elements for the read and the write). Rows of up to
    // 1024 kRouteRegs elements stay in registers until they are written to
    // their tier; longer rows go through the EV buffers. The loads of the
    // exchange, the scores of the argmin below and the score / threshold
    // above all go out before the first store.
    float* rk = a.rw_k + static_cast<size_t>(a.slot) * kvs;
    float* rv = a.rw_v + static_cast<size_t>(a.slot) * kvs;
    const bool in_regs = kvs <= 1024 * kRouteRegs;
    float evk[kRouteRegs], evv[kRouteRegs], kn[kRouteRegs], vn[kRouteRegs];
    if (in_regs) {
#pragma unroll
        for (int j = 0; j < kRouteRegs; ++j) {
            const int e = tid + 1024 * j;
            if (e < kvs) {
                evk[j] = rk[e];
                evv[j] = rv[e];
                kn[j] = a.k_new[e];
                vn[j] = a.v_new[e];
            }
        }
    }

    // Argmin over HH_scores[0..hh) with the sequential scan's semantics
    // (cache_engine.cpp:224-232): first index of the minimum under '<'; NaNs
    // never win unless at slot 0, which the decision below handles. Each
    // thread keeps kArgminBatch loads in flight, then a min over the keys.
    // The decision reads it only when the heavy hitters are full and the
    // score passes the threshold, so it runs only then (most evicted tokens
    // go to the waiting room without it).
    const bool need_min = (hh >= a.max_hh) && hh > 0 && score >= thr;
    float h0 = 0.0f;  // slot 0's score, read by the decision
    if (tid == 0 && need_min) h0 = a.hh_scores[0];
    unsigned long long best = ~0ull;
    if (need_min) {
        for (int i0 = 0; i0 < hh; i0 += 1024 * kArgminBatch) {
            float v[kArgminBatch];
#pragma unroll
            for (int u = 0; u < kArgminBatch; ++u) {
                const int i = i0 + tid + 1024 * u;
                v[u] = i < hh ? a.hh_scores[i] : __int_as_float(0x7fc00000);
            }
#pragma unroll
            for (int u = 0; u < kArgminBatch; ++u) {
                const unsigned long long k = hh_key(v[u], i0 + tid + 1024 * u);
                best = k < best ? k : best;
            }
        }
    }

    if (in_regs) {
#pragma unroll
        for (int j = 0; j < kRouteRegs; ++j) {
            const int e = tid + 1024 * j;
            if (e < kvs) {
                rk[e] = kn[j];
                rv[e] = vn[j];
            }
        }
    } else {
        for (int e = tid; e < kvs; e += blockDim.x) {
            a.ev_k[e] = rk[e];
            a.ev_v[e] = rv[e];
            rk[e] = a.k_new[e];
            rv[e] = a.v_new[e];
        }
    }
    if (need_min) {
        best = wave_min_u64(best);
        if ((tid & 63) == 0) red_k[tid >> 6] = best;
        __syncthreads();
        if (tid < 64) {
            best = wave_min_u64(tid < static_cast<int>(blockDim.x >> 6) ? red_k[tid] : ~0ull);
            if (tid == 0) red_k[0] = best;
        }
    }
    // The evicted row into `dk` / `dv` (row layout [kvs]).
    auto put_evicted = [&](float* dk, float* dv) {
        if (in_regs) {
#pragma unroll
            for (int j = 0; j < kRouteRegs; ++j) {
                const int e = tid + 1024 * j;
                if (e < kvs) {
                    dk[e] = evk[j];
                    dv[e] = evv[j];
                }
            }
        } else {
            for (int e = tid; e < kvs; e += blockDim.x) {
                dk[e] = a.ev_k[e];
                dv[e] = a.ev_v[e];
            }
        }
    };

    if (tid == 0) {
        int c = kToWR, mi = 0;
        if (score >= thr) {
            if (hh < a.max_hh) {
                c = kToHH;
            } else {
                float mv;
                const unsigned long long best = need_min ? red_k[0] : ~0ull;
                if (h0 != h0 || best == ~0ull) {
                    mi = 0;
                    mv = h0;
                } else {
                    // the value back from its key (a zero comes back as +0,
                    // which compares like -0)
                    mi = static_cast<int>(best & 0xffffffffu);
                    const unsigned o = static_cast<unsigned>(best >> 32);
                    mv = __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
                }
                if (score > mv) c = kReplace;
            }
        }
        s_case = c;
        s_min_idx = mi;
        s_score = score;
        if (a.thr_zero) st[kThreshold] = __float_as_int(0.0f);
    }
    __syncthreads();
    const int c = s_case;
    const int mi = s_min_idx;

    if (c == kToHH) {
        put_evicted(a.hh_k + static_cast<size_t>(hh) * kvs, a.hh_v + static_cast<size_t>(hh) * kvs);
        if (tid == 0) {
            a.hh_ids[hh] = eid;
            a.hh_scores[hh] = s_score;
        }
    } else if (c == kReplace) {
        float* hk = a.hh_k + static_cast<size_t>(mi) * kvs;
        float* hv = a.hh_v + static_cast<size_t>(mi) * kvs;
        float* wk = a.wr_k + static_cast<size_t>(wr) * kvs;
        float* wv = a.wr_v + static_cast<size_t>(wr) * kvs;
        for (int e = tid; e < kvs; e += blockDim.x) {
            const float x = hk[e], y = hv[e];  // both loads before either store
            wk[e] = x;
            wv[e] = y;
        }
        put_evicted(hk, hv);  // each thread overwrites only elements it has read
        if (tid == 0) {
            a.wr_ids[wr] = a.hh_ids[mi];
            a.hh_ids[mi] = eid;
            a.hh_scores[mi] = s_score;
        }
    } else {
        put_evicted(a.wr_k + static_cast<size_t>(wr) * kvs, a.wr_v + static_cast<size_t>(wr) * kvs);
        if (tid == 0) a.wr_ids[wr] = eid;
    }
    const int new_hh = hh + (c == kToHH ? 1 : 0);
    const int new_wr = wr + (c == kToHH ? 0 : 1);

    // The counters (read at the start, written by thread 0 only) need no
    // barrier; the flush reads waiting-room rows other threads just wrote.
    if (tid == 0) {
        st[kHhCount] = new_hh;
        st[kTotalEvictions] = evictions + 1;
        st[kRwHead] = a.new_head;
        st[kTotal] = total + 1;
        if (new_wr == a.chunk) {
            if (blocks + 1 > logical) st[kLogicalAlloc] = max(logical + 64, blocks + 1);
            st[kBlocksUsed] = blocks + 1;
            st[kPbsCount] = pbs_count + a.chunk;
            st[kWrCount] = 0;
        } else {
            st[kWrCount] = new_wr;
        }
    }
    if (new_wr == a.chunk) {  // uniform
        __syncthreads();
        if (a.fp16)
            flush_waiting_room<uint16_t>(a, blocks);
        else
            flush_waiting_room<float>(a, blocks);
    }
}

// Prefill bookkeeping after the bulk copies / quantisation
// (cache_engine.cpp:271-395).
struct PrefillArgs {
    int* st;
    int64_t* pbs_ids;
    int64_t* wr_ids;
    int chunk, sink, nbq, rem, q_len, short_path, s, r;
};

__global__ void prefill_state_kernel(PrefillArgs a) {
    int* st = a.st;
    const int used = st[kBlocksUsed];
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < a.nbq * a.chunk; i += blockDim.x * gridDim.x)
        a.pbs_ids[static_cast<size_t>(used) * a.chunk + i] = a.sink + i;
    const int rs = a.sink + a.nbq * a.chunk;
    for (int t = threadIdx.x + blockIdx.x * blockDim.x; t < a.rem; t += blockDim.x * gridDim.x) a.wr_ids[t] = rs + t;
    // Every thread has read `used` before thread 0 of block 0 rewrites it.
    __syncthreads();
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (a.short_path) {
            if (a.s > 0) st[kSCount] = a.s;
            if (a.r > 0) {
                st[kRwCount] = a.r;
                st[kRwHead] = 0;
            }
        } else {
            st[kSCount] = a.sink;
            st[kRwCount] = a.r;
            st[kRwHead] = 0;
            if (a.nbq > 0) {
                const int la = st[kLogicalAlloc];
                const int need = used + a.nbq;
                if (need > la) st[kLogicalAlloc] = max(la + 64, need);
                st[kBlocksUsed] = used + a.nbq;
                st[kPbsCount] += a.nbq * a.chunk;
                st[kTotalEvictions] += a.nbq * a.chunk;
            }
            st[kWrCount] = a.rem;
        }
        st[kTotal] = a.q_len;
    }
}

__global__ void init_state_kernel(int* st, float* g, int msl, int64_t* hh_ids, int max_hh, int64_t* wr_ids, int chunk,
                                  int64_t* pbs_ids, size_t pbs_slots) {
    const size_t i0 = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = i0; i < static_cast<size_t>(msl); i += stride) g[i] = 0.0f;
    for (size_t i = i0; i < static_cast<size_t>(max_hh); i += stride) hh_ids[i] = -1;
    for (size_t i = i0; i < static_cast<size_t>(chunk); i += stride) wr_ids[i] = -1;
    for (size_t i = i0; i < pbs_slots; i += stride) pbs_ids[i] = -1;
    if (i0 < kStateSlots) st[i0] = (i0 == kLastCalcPos) ? -1 : 0;
}

__global__ void fill_ids_kernel(int64_t* ids, size_t from, size_t to) {
    for (size_t i = from + blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < to;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        ids[i] = -1;
}

// Score feedback with caller-supplied mean weights (cache_engine.cpp:511-540).
__global__ void __launch_bounds__(256) feedback_kernel(const int* st, const float* __restrict__ mw, Feedback fb,
                                                       int kgs) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = st[kSCount], hh = st[kHhCount], rw = st[kRwCount], total = st[kTotal];
    const int Nd = s + hh + rw;
    const int n = Nd + st[kBlocksUsed] * kgs;
    if (i >= n) return;
    long long tid;
    int hh_slot = -1;
    if (i < s) {
        tid = i;
    } else if (i < s + hh) {
        hh_slot = i - s;
        tid = fb.hh_ids[hh_slot];
    } else if (i < Nd) {
        tid = static_cast<long long>(total) - rw + (i - s - hh);
    } else {
        tid = fb.pbs_ids[i - Nd];
    }
    if (tid >= 0 && tid < fb.max_seq_len) {
        const float gn = __builtin_fmaf(fb.decay, fb.g[tid], mw[i]);
        fb.g[tid] = gn;
        if (hh_slot >= 0) fb.hh_scores[hh_slot] = gn;
    }
}

template <typename T>
int dev_alloc(T** p, size_t n) {
    void* v = nullptr;
    TT_HIP_CHECK(hipMalloc(&v, std::max<size_t>(n, 1) * sizeof(T)));
    *p = static_cast<T*>(v);
    return TT_OK;
}

}  // namespace
}  // namespace tt

using namespace tt;

struct tt_engine {
    int device = 0;
    int Hq, Hkv, D, msl, S, R, interval, kgs, chunk, qhd, max_hh, fp16;
    float h_ratio, decay;
    size_t kvs;
    // tiers
    float *S_K = nullptr, *S_V = nullptr, *RW_K = nullptr, *RW_V = nullptr, *HH_K = nullptr, *HH_V = nullptr;
    float *HH_scores = nullptr, *WR_K = nullptr, *WR_V = nullptr, *EV_K = nullptr, *EV_V = nullptr, *g = nullptr;
    int64_t *HH_ids = nullptr, *WR_ids = nullptr, *PBS_ids = nullptr;
    int32_t *PBS_KP = nullptr, *PBS_VP = nullptr;
    void *PBS_KS = nullptr, *PBS_KZ = nullptr, *PBS_VS = nullptr, *PBS_VZ = nullptr;
    int cap_blocks = 0;
    int* st = nullptr;
    unsigned int* ts = nullptr;  // threshold selection state (kThrStateWords)
    // host mirror of the data-independent counters
    int h_s = 0, h_rw = 0, h_head = 0, h_total = 0, h_ev = 0, h_last = -1;
    // Heavy hitters grow by at most one per routed eviction (prefill routes
    // none), so this count, capped at max_hh, bounds the tier without a
    // device read.
    int h_routed = 0;
    int blocks_ub = 0, wr_ub = 0;
    // attention workspace
    void* ws = nullptr;
    size_t ws_bytes = 0;
    float* mw = nullptr;
    size_t mw_cap = 0;
    int* host_state = nullptr;  // pinned
    // A step whose mean weights and score feedback are still to run (its
    // partials, logits and row statistics are in ws): tt_engine_step_deferred
    // leaves it for the next engine's finalize launch or a flush.
    bool fb_pending = false;
    AttnInputs pend_in{};
    AttnPlan pend_plan{};

    size_t msz() const { return fp16 ? 2 : 4; }
};

namespace {

int engine_free_pbs(tt_engine* e) {
    (void)hipFree(e->PBS_KP);
    (void)hipFree(e->PBS_VP);
    (void)hipFree(e->PBS_KS);
    (void)hipFree(e->PBS_KZ);
    (void)hipFree(e->PBS_VS);
    (void)hipFree(e->PBS_VZ);
    (void)hipFree(e->PBS_ids);
    return TT_OK;
}

int engine_reserve_ws(tt_engine* e, const AttnPlan& p, hipStream_t s);

constexpr int kLogicalSlack = 64;

// Physical packed-store capacity. Buffers are reallocated (and copied) only
// when the upper bound on used blocks, plus the logical allocation's slack,
// exceeds the allocation.
int engine_reserve_blocks(tt_engine* e, int need, hipStream_t s) {
    // The reference's logical allocation (pbs_allocated_blocks, which sizes the
    // PBS getters) runs up to kLogicalSlack - 1 blocks past the used count
    // (cache_engine.cpp:84-116: +64 at a time); the store covers it.
    need += kLogicalSlack;
    if (need <= e->cap_blocks) return TT_OK;
    const int nc = std::max(need, e->cap_blocks + std::max(64, e->cap_blocks / 2));
    const size_t kvs = e->kvs, ch = e->chunk, msz = e->msz(), W = e->kgs / 16;
    int32_t *kp, *vp;
    char *ks, *kz, *vs, *vz;
    int64_t* ids;
    int rc;
    if ((rc = dev_alloc(&kp, nc * W * kvs)) || (rc = dev_alloc(&vp, nc * ch * e->Hkv * e->qhd)) ||
        (rc = dev_alloc(&ks, nc * kvs * msz)) || (rc = dev_alloc(&kz, nc * kvs * msz)) ||
        (rc = dev_alloc(&vs, nc * ch * e->Hkv * msz)) || (rc = dev_alloc(&vz, nc * ch * e->Hkv * msz)) ||
        (rc = dev_alloc(&ids, nc * ch)))
        return rc;
    const size_t ob = e->cap_blocks;
    if (ob > 0) {
        TT_HIP_CHECK(hipMemcpyAsync(kp, e->PBS_KP, ob * W * kvs * 4, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(vp, e->PBS_VP, ob * ch * e->Hkv * e->qhd * 4, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(ks, e->PBS_KS, ob * kvs * msz, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(kz, e->PBS_KZ, ob * kvs * msz, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(vs, e->PBS_VS, ob * ch * e->Hkv * msz, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(vz, e->PBS_VZ, ob * ch * e->Hkv * msz, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(ids, e->PBS_ids, ob * ch * 8, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipStreamSynchronize(s));
        engine_free_pbs(e);
    }
    TT_HIP_CHECK(hipMemsetAsync(kp + ob * W * kvs, 0, (nc - ob) * W * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(vp + ob * ch * e->Hkv * e->qhd, 0, (nc - ob) * ch * e->Hkv * e->qhd * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(ks + ob * kvs * msz, 0, (nc - ob) * kvs * msz, s));
    TT_HIP_CHECK(hipMemsetAsync(kz + ob * kvs * msz, 0, (nc - ob) * kvs * msz, s));
    TT_HIP_CHECK(hipMemsetAsync(vs + ob * ch * e->Hkv * msz, 0, (nc - ob) * ch * e->Hkv * msz, s));
    TT_HIP_CHECK(hipMemsetAsync(vz + ob * ch * e->Hkv * msz, 0, (nc - ob) * ch * e->Hkv * msz, s));
    hipLaunchKernelGGL(fill_ids_kernel, dim3(64), dim3(256), 0, s, ids, ob * ch, static_cast<size_t>(nc) * ch);
    TT_LAUNCH_CHECK();
    e->PBS_KP = kp;
    e->PBS_VP = vp;
    e->PBS_KS = ks;
    e->PBS_KZ = kz;
    e->PBS_VS = vs;
    e->PBS_VZ = vz;
    e->PBS_ids = ids;
    e->cap_blocks = nc;
    // Attention workspace follows the capacity.
    return engine_reserve_ws(e, attn_plan(e->S + e->max_hh + e->R, nc, e->Hq, e->Hkv, e->D, e->kgs, true, e->fp16), s);
}

// Grows the attention workspace and the mean-weight buffer to what plan `p`
// needs (plans for smaller bounds are not always smaller).
int engine_reserve_ws(tt_engine* e, const AttnPlan& p, hipStream_t s) {
    if (p.bytes > e->ws_bytes) {
        if (e->ws) {
            TT_HIP_CHECK(hipStreamSynchronize(s));
            (void)hipFree(e->ws);
        }
        e->ws = nullptr;
        TT_HIP_CHECK(hipMalloc(&e->ws, p.bytes));
        e->ws_bytes = p.bytes;
    }
    const size_t tok = static_cast<size_t>(p.token_ub) + 16;
    if (tok > e->mw_cap) {
        if (e->mw) {
            TT_HIP_CHECK(hipStreamSynchronize(s));
            (void)hipFree(e->mw);
        }
        e->mw = nullptr;
        TT_HIP_CHECK(hipMalloc(&e->mw, tok * sizeof(float)));
        e->mw_cap = tok;
    }
    return TT_OK;
}

AttnInputs engine_inputs(const tt_engine* e, const float* Q) {
    AttnInputs in;
    in.Q = Q;
    in.k0 = e->S_K;
    in.v0 = e->S_V;
    in.k1 = e->HH_K;
    in.v1 = e->HH_V;
    in.k2 = e->RW_K;
    in.v2 = e->RW_V;
    in.ring_size = e->R > 0 ? e->R : 1;
    in.state = e->st;
    in.kp = e->PBS_KP;
    in.ks = e->PBS_KS;
    in.kz = e->PBS_KZ;
    in.vp = e->PBS_VP;
    in.vs = e->PBS_VS;
    in.vz = e->PBS_VZ;
    in.ids = e->PBS_ids;
    in.Hq = e->Hq;
    in.Hkv = e->Hkv;
    in.D = e->D;
    in.kgs = e->kgs;
    in.meta_fp16 = e->fp16;
    return in;
}

Feedback engine_feedback_args(tt_engine* e) {
    Feedback fb;
    fb.g = e->g;
    fb.hh_scores = e->HH_scores;
    fb.hh_ids = e->HH_ids;
    fb.pbs_ids = e->PBS_ids;
    fb.max_seq_len = e->msl;
    fb.decay = e->decay;
    return fb;
}

// The deferred mean weights and score feedback of e's last step, if any, on
// stream s (before anything that reads or changes the scores or tiers).
int engine_flush(tt_engine* e, hipStream_t s) {
    if (!e->fb_pending) return TT_OK;
    const Feedback fb = engine_feedback_args(e);
    const int rc =
        attn_launch_finalize(e->pend_in, e->pend_plan, e->ws, nullptr, e->mw, &fb, nullptr, 0, s, FinRoles::kMean);
    if (rc == TT_OK) e->fb_pending = false;
    return rc;
}

int engine_sync_state(tt_engine* e, hipStream_t s) {
    int rc = engine_flush(e, s);
    if (rc) return rc;
    TT_HIP_CHECK(hipMemcpyAsync(e->host_state, e->st, kStateSlots * sizeof(int), hipMemcpyDeviceToHost, s));
    TT_HIP_CHECK(hipStreamSynchronize(s));
    return TT_OK;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

}  // namespace

extern "C" {

int tt_engine_create(tt_engine** out, int num_q_heads, int num_kv_heads, int head_dim, int max_seq_len, int sink_size,
                     int rw_size, float h_ratio, float score_decay, int update_interval, int k_group_size,
                     const char* pbs_metadata_dtype, void* stream) {
    clear_error();
    if (!out) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine output pointer is NULL.");
    *out = nullptr;
    const int kgs = (k_group_size == 32) ? 32 : 16;
    int rc = attn_check_shapes(num_q_heads, num_kv_heads, head_dim, kgs);
    if (rc) return rc;
    if (max_seq_len <= 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "max_seq_len must be positive.");
    if (sink_size < 0 || rw_size < 1)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "sink_size must be >= 0 and rw_size must be >= 1.");
    {
        // the attention's tokens at most: sinks, heavy hitters, ring, every block
        const long long hh = std::max(1LL, static_cast<long long>(std::ceil(static_cast<float>(max_seq_len) * h_ratio)));
        const long long tokens = static_cast<long long>(sink_size) + hh + rw_size +
                                 (static_cast<long long>(max_seq_len) / kgs + 2) * kgs;
        if (!logits_fit(num_q_heads, (tokens + 3) & ~3LL))
            TT_FAIL(TT_ERR_INVALID_ARGUMENT,
                    "num_q_heads x max_seq_len exceeds the 4 GiB logits buffer of the mean weights.");
    }
    hipStream_t s = as_stream(stream);
    tt_engine* e = new tt_engine();
    TT_HIP_CHECK(hipGetDevice(&e->device));
    e->Hq = num_q_heads;
    e->Hkv = num_kv_heads;
    e->D = head_dim;
    e->msl = max_seq_len;
    e->S = sink_size;
    e->R = rw_size;
    e->h_ratio = h_ratio;
    e->decay = score_decay;
    e->interval = update_interval;
    e->kgs = kgs;
    e->chunk = kgs;
    e->qhd = (head_dim + 15) / 16;
    e->fp16 = (pbs_metadata_dtype && std::string(pbs_metadata_dtype) == "fp16") ? 1 : 0;
    // cache_engine.cpp:47-48: ceil in float.
    e->max_hh = static_cast<int>(std::ceil(static_cast<float>(max_seq_len) * h_ratio));
    if (e->max_hh < 1) e->max_hh = 1;
    e->kvs = static_cast<size_t>(num_kv_heads) * head_dim;
    const size_t kvs = e->kvs;
    if ((rc = dev_alloc(&e->S_K, std::max(1, e->S) * kvs)) || (rc = dev_alloc(&e->S_V, std::max(1, e->S) * kvs)) ||
        (rc = dev_alloc(&e->RW_K, e->R * kvs)) || (rc = dev_alloc(&e->RW_V, e->R * kvs)) ||
        (rc = dev_alloc(&e->HH_K, e->max_hh * kvs)) || (rc = dev_alloc(&e->HH_V, e->max_hh * kvs)) ||
        (rc = dev_alloc(&e->HH_scores, e->max_hh)) || (rc = dev_alloc(&e->HH_ids, e->max_hh)) ||
        (rc = dev_alloc(&e->WR_K, e->chunk * kvs)) || (rc = dev_alloc(&e->WR_V, e->chunk * kvs)) ||
        (rc = dev_alloc(&e->WR_ids, e->chunk)) || (rc = dev_alloc(&e->EV_K, kvs)) || (rc = dev_alloc(&e->EV_V, kvs)) ||
        (rc = dev_alloc(&e->g, e->msl)) || (rc = dev_alloc(&e->st, kStateSlots)) ||
        (rc = dev_alloc(&e->ts, kThrStateWords))) {
        tt_engine_destroy(e);
        return rc;
    }
    TT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&e->host_state), kStateSlots * sizeof(int)));
    TT_HIP_CHECK(hipMemsetAsync(e->S_K, 0, std::max(1, e->S) * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->S_V, 0, std::max(1, e->S) * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->RW_K, 0, e->R * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->RW_V, 0, e->R * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->HH_K, 0, e->max_hh * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->HH_V, 0, e->max_hh * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->HH_scores, 0, e->max_hh * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->WR_K, 0, e->chunk * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->WR_V, 0, e->chunk * kvs * 4, s));
    TT_HIP_CHECK(hipMemsetAsync(e->ts, 0, kThrStateWords * sizeof(unsigned int), s));
    const int want_blocks = (e->msl + e->chunk - 1) / e->chunk + 1;
    if ((rc = engine_reserve_blocks(e, want_blocks, s))) {
        tt_engine_destroy(e);
        return rc;
    }
    hipLaunchKernelGGL(init_state_kernel, dim3(256), dim3(256), 0, s, e->st, e->g, e->msl, e->HH_ids, e->max_hh,
                       e->WR_ids, e->chunk, e->PBS_ids, static_cast<size_t>(e->cap_blocks) * e->chunk);
    TT_LAUNCH_CHECK();
    TT_HIP_CHECK(hipStreamSynchronize(s));
    *out = e;
    return TT_OK;
}

int tt_engine_destroy(tt_engine* e) {
    clear_error();
    if (!e) return TT_OK;
    DeviceGuard dg(e->device);
    (void)hipDeviceSynchronize();
    float* fb[] = {e->S_K, e->S_V, e->RW_K, e->RW_V, e->HH_K, e->HH_V, e->HH_scores, e->WR_K, e->WR_V, e->EV_K,
                   e->EV_V, e->g, e->mw};
    for (float* p : fb) (void)hipFree(p);
    (void)hipFree(e->HH_ids);
    (void)hipFree(e->WR_ids);
    (void)hipFree(e->st);
    (void)hipFree(e->ts);
    (void)hipFree(e->ws);
    engine_free_pbs(e);
    if (e->host_state) (void)hipHostFree(e->host_state);
    delete e;
    return TT_OK;
}

int tt_engine_ingest(tt_engine* e, const float* K_new, const float* V_new, void* stream) {
    clear_error();
    if (!e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine is NULL.");
    if (!K_new || !V_new) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'K_new'/'V_new' pointer address is NULL.");
    DeviceGuard dg(e->device);
    hipStream_t s = as_stream(stream);
    {
        const int frc = engine_flush(e, s);  // the last step's scores before this step's routing
        if (frc) return frc;
    }
    const int kvs = static_cast<int>(e->kvs);
    const int blocks = (kvs + 255) / 256;
    if (e->h_s < e->S) {
        hipLaunchKernelGGL(append_row_kernel, dim3(blocks), dim3(256), 0, s, K_new, V_new,
                           e->S_K + static_cast<size_t>(e->h_s) * kvs, e->S_V + static_cast<size_t>(e->h_s) * kvs, kvs,
                           e->st, static_cast<int>(kSCount));
        TT_LAUNCH_CHECK();
        e->h_s++;
    } else if (e->h_rw < e->R) {
        hipLaunchKernelGGL(append_row_kernel, dim3(blocks), dim3(256), 0, s, K_new, V_new,
                           e->RW_K + static_cast<size_t>(e->h_rw) * kvs, e->RW_V + static_cast<size_t>(e->h_rw) * kvs,
                           kvs, e->st, static_cast<int>(kRwCount));
        TT_LAUNCH_CHECK();
        e->h_rw++;
    } else {
        // Threshold cadence (cache_engine.cpp:118-146), decided on the host.
        const int cs = e->S;
        const int ce = std::min(e->h_total - e->R, e->msl);
        const int thr_zero = (ce <= cs) ? 1 : 0;
        if (!thr_zero && (e->h_last == -1 || e->h_total - e->h_last >= e->interval)) {
            const size_t n = static_cast<size_t>(ce - cs);
            float q = 1.0f - e->h_ratio;
            if (q < 0.0f) q = 0.0f;
            if (q > 1.0f) q = 1.0f;
            const size_t k = static_cast<size_t>(q * static_cast<float>(n - 1));
            if (n < kThrMultiMin) {
                hipLaunchKernelGGL(threshold_kernel, dim3(1), dim3(1024), 0, s, e->g + cs, static_cast<int>(n),
                                   static_cast<long long>(k), e->st, e->h_total);
                TT_LAUNCH_CHECK();
            } else {
                const int per = 256 * kThrHistPer;
                const int wgs = static_cast<int>(std::min<size_t>(kThrHistWgs, (n + per - 1) / per));
                for (int pass = 0; pass < 3; ++pass) {
                    hipLaunchKernelGGL(thr_hist_kernel, dim3(wgs), dim3(256), 0, s, e->g + cs, static_cast<int>(n),
                                       pass, e->ts);
                    TT_LAUNCH_CHECK();
                    hipLaunchKernelGGL(thr_select_kernel, dim3(1), dim3(1024), 0, s, pass, static_cast<long long>(k),
                                       e->ts, e->st, e->h_total);
                    TT_LAUNCH_CHECK();
                }
            }
            e->h_last = e->h_total;
        }
        // A flush may need one more block than the current upper bound.
        int rc = engine_reserve_blocks(e, e->blocks_ub + 1, s);
        if (rc) return rc;
        RouteArgs a;
        a.st = e->st;
        a.k_new = K_new;
        a.v_new = V_new;
        a.rw_k = e->RW_K;
        a.rw_v = e->RW_V;
        a.hh_k = e->HH_K;
        a.hh_v = e->HH_V;
        a.wr_k = e->WR_K;
        a.wr_v = e->WR_V;
        a.ev_k = e->EV_K;
        a.ev_v = e->EV_V;
        a.hh_ids = e->HH_ids;
        a.wr_ids = e->WR_ids;
        a.pbs_ids = e->PBS_ids;
        a.hh_scores = e->HH_scores;
        a.g = e->g;
        a.kp = e->PBS_KP;
        a.ks = e->PBS_KS;
        a.kz = e->PBS_KZ;
        a.vp = e->PBS_VP;
        a.vs = e->PBS_VS;
        a.vz = e->PBS_VZ;
        a.kvs = kvs;
        a.H = e->Hkv;
        a.D = e->D;
        a.kgs = e->kgs;
        a.chunk = e->chunk;
        a.max_hh = e->max_hh;
        a.max_seq_len = e->msl;
        a.fp16 = e->fp16;
        a.slot = e->h_head;
        a.evicted_id = static_cast<long long>(e->h_total) - e->R;
        a.thr_zero = thr_zero;
        a.new_head = (e->h_head + 1) % e->R;
        hipLaunchKernelGGL(route_kernel, dim3(1), dim3(1024), 0, s, a);
        TT_LAUNCH_CHECK();
        e->h_head = a.new_head;
        e->h_ev++;
        if (e->h_routed < e->max_hh) e->h_routed++;
        if (++e->wr_ub >= e->chunk) {
            e->wr_ub -= e->chunk;
            e->blocks_ub++;
        }
        e->h_total++;
        return TT_OK;
    }
    e->h_total++;
    return TT_OK;
}

static int engine_attend(tt_engine* e, const float* Q, float* out, float* head_w, int head_w_ld, bool feedback,
                         hipStream_t s) {
    int rc = engine_reserve_blocks(e, e->blocks_ub, s);
    if (rc) return rc;
    const int dense_ub = e->h_s + e->h_routed + e->h_rw;
    const AttnPlan p = attn_plan(dense_ub, e->blocks_ub, e->Hq, e->Hkv, e->D, e->kgs, true, e->fp16);
    rc = engine_reserve_ws(e, p, s);
    if (rc) return rc;
    AttnInputs in = engine_inputs(e, Q);
    Feedback fb = engine_feedback_args(e);
    return attn_launch(in, p, e->ws, out, e->mw, feedback ? &fb : nullptr, head_w, head_w_ld, s);
}

int tt_engine_step(tt_engine* e, const float* Q, const float* K_new, const float* V_new, float* attn_output,
                   void* stream) {
    clear_error();
    if (!e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine is NULL.");
    if (!Q || !attn_output) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'Q'/'attn_output' pointer address is NULL.");
    int rc = tt_engine_ingest(e, K_new, V_new, stream);
    if (rc) return rc;
    DeviceGuard dg(e->device);
    return engine_attend(e, Q, attn_output, nullptr, 0, true, as_stream(stream));
}

int tt_engine_step_deferred(tt_engine* e, const float* Q, const float* K_new, const float* V_new, float* attn_output,
                            tt_engine* prev, void* stream) {
    clear_error();
    if (!e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine is NULL.");
    if (!Q || !attn_output) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'Q'/'attn_output' pointer address is NULL.");
    if (prev == e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "prev must be another engine.");
    if (prev && prev->device != e->device) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "prev lives on another device.");
    int rc = tt_engine_ingest(e, K_new, V_new, stream);  // flushes e's own pending step first
    if (rc) return rc;
    DeviceGuard dg(e->device);
    hipStream_t s = as_stream(stream);
    rc = engine_reserve_blocks(e, e->blocks_ub, s);
    if (rc) return rc;
    const int dense_ub = e->h_s + e->h_routed + e->h_rw;
    const AttnPlan p = attn_plan(dense_ub, e->blocks_ub, e->Hq, e->Hkv, e->D, e->kgs, true, e->fp16);
    rc = engine_reserve_ws(e, p, s);
    if (rc) return rc;
    const AttnInputs in = engine_inputs(e, Q);
    rc = attn_launch_split(in, p, e->ws, s);
    if (rc) return rc;
    if (prev && prev->fb_pending) {
        const Feedback fb = engine_feedback_args(prev);
        rc = attn_launch_finalize_deferred(in, p, e->ws, attn_output, prev->pend_in, prev->pend_plan, prev->ws,
                                           prev->mw, &fb, s);
        if (rc == TT_OK) prev->fb_pending = false;
    } else {
        rc = attn_launch_finalize(in, p, e->ws, attn_output, nullptr, nullptr, nullptr, 0, s, FinRoles::kMerge);
    }
    if (rc) return rc;
    e->pend_in = in;
    e->pend_plan = p;
    e->fb_pending = true;
    return TT_OK;
}

int tt_engine_flush_feedback(tt_engine* e, void* stream) {
    clear_error();
    if (!e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine is NULL.");
    DeviceGuard dg(e->device);
    return engine_flush(e, as_stream(stream));
}

// Upper bound on the visible token count after the next ingest, from the
// host-side tier bounds alone (no device read): the new token lands in the
// sinks or the ring, or an eviction routes one token into the heavy hitters
// (up to max_hh) or the waiting room, whose flush adds one block.
static long long visible_ub_after_ingest(const tt_engine* e) {
    long long s = e->h_s, rw = e->h_rw, hh = e->h_routed, blocks = e->blocks_ub;
    if (s < e->S) {
        ++s;
    } else if (rw < e->R) {
        ++rw;
    } else {
        if (hh < e->max_hh) ++hh;
        if (e->wr_ub + 1 >= e->chunk) ++blocks;
    }
    return s + hh + rw + blocks * static_cast<long long>(e->chunk);
}

int tt_engine_step_weights(tt_engine* e, const float* Q, const float* K_new, const float* V_new, float* attn_output,
                           float* head_weights, int head_weights_capacity, int* visible_out, void* stream) {
    clear_error();
    if (!e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine is NULL.");
    if (!Q || !attn_output || !head_weights)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'Q'/'attn_output'/'head_weights' pointer address is NULL.");
    if (!K_new || !V_new) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'K_new'/'V_new' pointer address is NULL.");
    DeviceGuard dg(e->device);
    hipStream_t s = as_stream(stream);
    // The capacity is validated before the step is enqueued, so a rejected call
    // leaves the tiers as they were (bindings.cpp:120-128 validates before
    // computing). The host-side bound needs no device read; when it does not
    // fit, the device counters give the exact bound: one step adds at most one
    // visible token, or one block of `chunk` tokens when the waiting room
    // flushes.
    if (visible_ub_after_ingest(e) > head_weights_capacity) {
        int rc = engine_sync_state(e, s);
        if (rc) return rc;
        const int* st = e->host_state;
        const long long vis_now = static_cast<long long>(st[kSCount]) + st[kHhCount] + st[kRwCount] +
                                  static_cast<long long>(st[kBlocksUsed]) * e->chunk;
        if (vis_now + std::max(1, e->chunk) > head_weights_capacity)
            TT_FAIL(TT_ERR_OUT_OF_RANGE, "head_weights capacity is smaller than the step's visible token bound "
                                         "(the visible tokens before the step plus one block).");
    }
    int rc = tt_engine_ingest(e, K_new, V_new, stream);
    if (rc) return rc;
    rc = engine_attend(e, Q, attn_output, head_weights, head_weights_capacity, true, s);
    if (rc) return rc;
    rc = engine_sync_state(e, s);
    if (rc) return rc;
    const int* st = e->host_state;
    const int vis = st[kSCount] + st[kHhCount] + st[kRwCount] + st[kBlocksUsed] * e->chunk;
    if (visible_out) *visible_out = vis;
    if (vis > head_weights_capacity)
        TT_FAIL(TT_ERR_OUT_OF_RANGE, "head_weights capacity is smaller than the visible token count.");
    return TT_OK;
}

int tt_engine_feedback(tt_engine* e, const float* mean_attn_weights, void* stream) {
    clear_error();
    if (!e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine is NULL.");
    if (!mean_attn_weights) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "mean_attn_weights is NULL.");
    DeviceGuard dg(e->device);
    hipStream_t s = as_stream(stream);
    int rc = engine_flush(e, s);
    if (rc) return rc;
    const int n = e->S + e->max_hh + e->R + e->blocks_ub * e->chunk;
    hipLaunchKernelGGL(feedback_kernel, dim3((n + 255) / 256), dim3(256), 0, s, e->st, mean_attn_weights,
                       engine_feedback_args(e), e->kgs);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

int tt_engine_prefill(tt_engine* e, const float* K_all, const float* V_all, int q_len, void* stream) {
    clear_error();
    if (!e) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine is NULL.");
    if (q_len < 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "q_len must be non-negative.");
    if (q_len > 0 && (!K_all || !V_all))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'K_all'/'V_all' pointer address is NULL.");
    DeviceGuard dg(e->device);
    hipStream_t s = as_stream(stream);
    int frc = engine_flush(e, s);
    if (frc) return frc;
    const size_t kvs = e->kvs;
    PrefillArgs pa{};
    pa.st = e->st;
    pa.pbs_ids = e->PBS_ids;
    pa.wr_ids = e->WR_ids;
    pa.chunk = e->chunk;
    pa.sink = e->S;
    pa.q_len = q_len;
    if (q_len <= e->S + e->R) {
        const int sc = std::min(e->S, q_len);
        const int r = q_len - sc;
        if (sc > 0) {
            TT_HIP_CHECK(hipMemcpyAsync(e->S_K, K_all, sc * kvs * 4, hipMemcpyDeviceToDevice, s));
            TT_HIP_CHECK(hipMemcpyAsync(e->S_V, V_all, sc * kvs * 4, hipMemcpyDeviceToDevice, s));
            e->h_s = sc;
        }
        if (r > 0) {
            TT_HIP_CHECK(hipMemcpyAsync(e->RW_K, K_all + sc * kvs, r * kvs * 4, hipMemcpyDeviceToDevice, s));
            TT_HIP_CHECK(hipMemcpyAsync(e->RW_V, V_all + sc * kvs, r * kvs * 4, hipMemcpyDeviceToDevice, s));
            e->h_rw = r;
            e->h_head = 0;
        }
        pa.short_path = 1;
        pa.s = sc;
        pa.r = r;
    } else {
        TT_HIP_CHECK(hipMemcpyAsync(e->S_K, K_all, e->S * kvs * 4, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(e->S_V, V_all, e->S * kvs * 4, hipMemcpyDeviceToDevice, s));
        const int rw_start = q_len - e->R;
        TT_HIP_CHECK(hipMemcpyAsync(e->RW_K, K_all + rw_start * kvs, e->R * kvs * 4, hipMemcpyDeviceToDevice, s));
        TT_HIP_CHECK(hipMemcpyAsync(e->RW_V, V_all + rw_start * kvs, e->R * kvs * 4, hipMemcpyDeviceToDevice, s));
        const int n_inter = rw_start - e->S;
        const int nbq = n_inter / e->chunk;
        const int rem = n_inter % e->chunk;
        if (nbq > 0) {
            int rc = engine_reserve_blocks(e, e->blocks_ub + nbq + 1, s);
            if (rc) return rc;
            const float* ksrc = K_all + e->S * kvs;
            const float* vsrc = V_all + e->S * kvs;
            rc = launch_quantize_k(ksrc, reinterpret_cast<uint32_t*>(e->PBS_KP), e->PBS_KS, e->PBS_KZ, nbq, e->Hkv, e->D,
                                   e->kgs, e->fp16, e->st + kBlocksUsed, s);
            if (rc) return rc;
            rc = launch_quantize_v(vsrc, e->PBS_VP, e->PBS_VS, e->PBS_VZ, nbq * e->chunk, e->Hkv, e->D, e->fp16,
                                   e->st + kBlocksUsed, e->chunk, s);
            if (rc) return rc;
        }
        if (rem > 0) {
            const size_t rs = e->S + static_cast<size_t>(nbq) * e->chunk;
            TT_HIP_CHECK(hipMemcpyAsync(e->WR_K, K_all + rs * kvs, rem * kvs * 4, hipMemcpyDeviceToDevice, s));
            TT_HIP_CHECK(hipMemcpyAsync(e->WR_V, V_all + rs * kvs, rem * kvs * 4, hipMemcpyDeviceToDevice, s));
        }
        pa.short_path = 0;
        pa.nbq = nbq;
        pa.rem = rem;
        pa.r = e->R;
        e->h_s = e->S;
        e->h_rw = e->R;
        e->h_head = 0;
        e->h_ev += nbq * e->chunk;
        e->blocks_ub += nbq;
        e->wr_ub = rem;
    }
    const int work = std::max(pa.nbq * pa.chunk, pa.rem);
    // One workgroup: the state update must follow every read of the old
    // block count, which a block-wide barrier guarantees.
    (void)work;
    hipLaunchKernelGGL(prefill_state_kernel, dim3(1), dim3(1024), 0, s, pa);
    TT_LAUNCH_CHECK();
    e->h_total = q_len;
    return TT_OK;
}

int tt_engine_counters(tt_engine* e, int64_t* o, void* stream) {
    clear_error();
    if (!e || !o) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine or output is NULL.");
    DeviceGuard dg(e->device);
    int rc = engine_sync_state(e, as_stream(stream));
    if (rc) return rc;
    const int* st = e->host_state;
    const int64_t v[TT_ENGINE_N_COUNTERS] = {e->Hq, e->Hkv, e->D, e->msl, e->S, e->R, e->interval, e->kgs, e->chunk,
                                             e->qhd, e->max_hh, e->fp16, st[kSCount], st[kRwCount], st[kRwHead],
                                             st[kHhCount], st[kWrCount], st[kLogicalAlloc], st[kBlocksUsed],
                                             st[kPbsCount], st[kTotal], st[kLastCalcPos], st[kTotalEvictions]};
    std::memcpy(o, v, sizeof(v));
    return TT_OK;
}

const char* tt_engine_counter_names(void) {
    return "num_q_heads num_kv_heads head_dim max_seq_len sink_size rw_size update_interval k_group_size "
           "chunk_size quant_head_dim max_hh use_fp16_meta s_count rw_count rw_head_index hh_count wr_count "
           "pbs_allocated_blocks pbs_blocks_used pbs_count total_processed_tokens last_calc_pos total_evictions";
}

int tt_engine_buffer_bytes(tt_engine* e, size_t* out, void* stream) {
    clear_error();
    if (!e || !out) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine or output is NULL.");
    DeviceGuard dg(e->device);
    int rc = engine_sync_state(e, as_stream(stream));
    if (rc) return rc;
    const size_t kvs = e->kvs, nb = e->host_state[kLogicalAlloc], msz = e->msz(), ch = e->chunk;
    size_t b = 0;
    b += 2 * static_cast<size_t>(e->S) * kvs * 4;
    b += 2 * static_cast<size_t>(e->R) * kvs * 4;
    b += 2 * static_cast<size_t>(e->max_hh) * kvs * 4 + static_cast<size_t>(e->max_hh) * 12;
    b += 2 * ch * kvs * 4 + ch * 8;
    b += nb * (e->kgs / 16) * kvs * 4;
    b += 2 * nb * kvs * msz;
    b += 2 * nb * ch * e->Hkv * msz;
    b += nb * ch * e->Hkv * e->qhd * 4;
    b += nb * ch * 8;
    b += static_cast<size_t>(e->msl) * 4;
    *out = b;
    return TT_OK;
}

int tt_engine_buffer(tt_engine* e, int which, void** p, int64_t* numel, int* es, void* stream) {
    clear_error();
    if (!e || !p || !numel || !es) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine or output is NULL.");
    DeviceGuard dg(e->device);
    int rc = engine_sync_state(e, as_stream(stream));
    if (rc) return rc;
    const int64_t kvs = static_cast<int64_t>(e->kvs), nb = e->host_state[kLogicalAlloc], ch = e->chunk;
    const int msz = static_cast<int>(e->msz());
    if (nb > e->cap_blocks) TT_FAIL(TT_ERR_RUNTIME, "packed store smaller than its logical allocation.");
    switch (which) {
    case 0: *p = e->S_K; *numel = e->S * kvs; *es = 4; break;
    case 1: *p = e->S_V; *numel = e->S * kvs; *es = 4; break;
    case 2: *p = e->RW_K; *numel = e->R * kvs; *es = 4; break;
    case 3: *p = e->RW_V; *numel = e->R * kvs; *es = 4; break;
    case 4: *p = e->HH_K; *numel = e->max_hh * kvs; *es = 4; break;
    case 5: *p = e->HH_V; *numel = e->max_hh * kvs; *es = 4; break;
    case 6: *p = e->HH_ids; *numel = e->max_hh; *es = 8; break;
    case 7: *p = e->HH_scores; *numel = e->max_hh; *es = 4; break;
    case 8: *p = e->WR_K; *numel = ch * kvs; *es = 4; break;
    case 9: *p = e->WR_V; *numel = ch * kvs; *es = 4; break;
    case 10: *p = e->WR_ids; *numel = ch; *es = 8; break;
    case 11: *p = e->PBS_KP; *numel = nb * (e->kgs / 16) * kvs; *es = 4; break;
    case 12: *p = e->PBS_KS; *numel = nb * kvs; *es = msz; break;
    case 13: *p = e->PBS_KZ; *numel = nb * kvs; *es = msz; break;
    case 14: *p = e->PBS_VP; *numel = nb * ch * e->Hkv * e->qhd; *es = 4; break;
    case 15: *p = e->PBS_VS; *numel = nb * ch * e->Hkv; *es = msz; break;
    case 16: *p = e->PBS_VZ; *numel = nb * ch * e->Hkv; *es = msz; break;
    case 17: *p = e->PBS_ids; *numel = nb * ch; *es = 8; break;
    case 18: *p = e->g; *numel = e->msl; *es = 4; break;
    case 19:
        *p = e->mw;
        *numel = e->host_state[kSCount] + e->host_state[kHhCount] + e->host_state[kRwCount] +
                 static_cast<int64_t>(e->host_state[kBlocksUsed]) * e->chunk;
        *es = 4;
        break;
    default: TT_FAIL(TT_ERR_OUT_OF_RANGE, "buffer index out of range.");
    }
    return TT_OK;
}

int tt_engine_visible(tt_engine* e, int* out, void* stream) {
    clear_error();
    if (!e || !out) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "engine or output is NULL.");
    DeviceGuard dg(e->device);
    int rc = engine_sync_state(e, as_stream(stream));
    if (rc) return rc;
    const int* st = e->host_state;
    *out = st[kSCount] + st[kHhCount] + st[kRwCount] + st[kBlocksUsed] * e->chunk;
    return TT_OK;
}

}  // extern "C"
