// tt_common.h -- shared host/device helpers for the gfx950 TriTierCache kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <climits>
#include <cstdint>
#include <cstring>
#include <string>

#include "../../include/tritiercache_amd.h"

namespace tt {

// ---------------------------------------------------------------------------
// Error handling: a status code plus a thread-local message.
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();

struct Status {
    int code = TT_OK;
    static Status ok() { return Status{}; }
};

#define TT_FAIL(code_, msg_)        \
    do {                            \
        ::tt::set_error(msg_);      \
        return (code_);             \
    } while (0)

#define TT_HIP_CHECK(expr)                                                                        \
    do {                                                                                          \
        hipError_t _e = (expr);                                                                   \
        if (_e != hipSuccess) {                                                                   \
            ::tt::set_error(std::string("HIP error in " #expr ": ") + hipGetErrorString(_e));     \
            return (_e == hipErrorOutOfMemory) ? TT_ERR_NO_MEMORY : TT_ERR_HIP;                   \
        }                                                                                         \
    } while (0)

#define TT_LAUNCH_CHECK() TT_HIP_CHECK(hipGetLastError())

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------
// Bit-exact scalar models of the reference's x86 primitives (device side).
// The reference quantisers run AVX2 code (csrc/cpu/quantize_{k,v}_avx2.cpp);
// these reproduce its semantics lane for lane, including the NaN and signed
// zero behaviour of the operand order.
// ---------------------------------------------------------------------------

// MINPS/MAXPS: (a < b) ? a : b -- the second operand wins on ties and NaN.
__device__ __forceinline__ float x86_minps(float a, float b) { return (a < b) ? a : b; }
__device__ __forceinline__ float x86_maxps(float a, float b) { return (a > b) ? a : b; }
// std::min / std::max of the scalar code paths.
__device__ __forceinline__ float std_min(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ float std_max(float a, float b) { return (a < b) ? b : a; }

// vcvtps2dq under the default MXCSR: round to nearest even, and the integer
// indefinite value 0x80000000 for NaN / out of range.
__device__ __forceinline__ int cvt_rne_i32(float x) {
    if (!(x >= -2147483648.0f && x < 2147483648.0f)) return INT_MIN;
    return static_cast<int>(__builtin_rintf(x));
}

// float -> IEEE binary16 with F16C vcvtps2ph(imm8=0) semantics: round to
// nearest even, half denormals produced, overflow to inf, NaN quieted with the
// top payload bits kept. Integer-only so it is exact on every device.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t mant = u & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    if (exp == 0) return (uint16_t)sign;
    int e = (int)exp - 112;  // rebias 127 -> 15
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        uint32_t full = mant | 0x800000u;
        int shift = 126 - (int)exp;
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

// binary16 -> float, exact (the hardware conversion keeps half denormals).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return static_cast<float>(v);
}

template <typename MetaT>
struct Meta;
template <>
struct Meta<float> {
    __device__ __forceinline__ static float load(const float* p, size_t i) { return p[i]; }
    __device__ __forceinline__ static void store(float* p, size_t i, float v) { p[i] = v; }
};
template <>
struct Meta<uint16_t> {
    __device__ __forceinline__ static float load(const uint16_t* p, size_t i) { return f16_to_f32(p[i]); }
    __device__ __forceinline__ static void store(uint16_t* p, size_t i, float v) { p[i] = f32_to_f16_rne(v); }
};

// ---------------------------------------------------------------------------
// Launchers implemented in the .hip files.
// ---------------------------------------------------------------------------
int launch_quantize_k(const float* K, uint32_t* packed, void* scale, void* zero, int num_blocks,
                      int num_heads, int head_dim, int k_group_size, int meta_fp16,
                      const int* block_base_dev, hipStream_t stream);
int launch_quantize_v(const float* V, int32_t* packed, void* scale, void* zero, int tokens,
                      int num_heads, int head_dim, int meta_fp16, const int* block_base_dev,
                      int tokens_per_block, hipStream_t stream);
int launch_dequantize_k(const int32_t* packed, const void* scale, const void* zero, float* out,
                        int num_blocks, int num_heads, int head_dim, int k_group_size, int meta_fp16,
                        hipStream_t stream);
int launch_dequantize_v(const int32_t* packed, const void* scale, const void* zero, float* out,
                        int total_tokens, int num_heads, int head_dim, int meta_fp16,
                        hipStream_t stream);

}  // namespace tt
