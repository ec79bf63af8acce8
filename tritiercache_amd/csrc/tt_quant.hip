// tt_quant.hip -- 2-bit asymmetric quantisers and dequantisers (gfx950).
//
// Bit-exact restatements of the reference AVX2 kernels:
//   K: csrc/cpu/quantize_k_avx2.cpp:26-110   (per channel over the block's tokens)
//   V: csrc/cpu/quantize_v_avx2.cpp:44-108   (per token over the head's channels)
//   dequant: csrc/cpu/dequantize_avx2.cpp:24-110 and :138-204
// They run off the decode hot path (once per 16 evictions, or in bulk at
// prefill), so each thread owns one output group and the code favours exact
// semantics over speed: explicit operand order for min/max, IEEE division,
// round-to-nearest-even conversion, software F16C-equivalent rounding.
#include "tt_quant_dev.h"

namespace tt {

namespace {

constexpr int kMaxGridY = 65535;  // largest grid y extent
// threads of a 1-D launch at most (a dispatch counts its work-items in 32 bits)
constexpr long long kMaxThreads = 0xFFFFFF00LL;

// One thread per (block, head, channel). Channels below 8*floor(D/8) follow
// the 8-wide vector body of the reference (MINPS/MAXPS operand order), the
// rest follow its scalar tail (std::min/std::max). Block b = b_off +
// blockIdx.y of the input; the output block is b + *base_dev when base_dev is
// given (engine prefill).
template <typename MetaT>
__global__ void __launch_bounds__(256) quantize_k_kernel(const float* __restrict__ K, uint32_t* __restrict__ packed,
                                                         MetaT* __restrict__ scale, MetaT* __restrict__ zero, int H,
                                                         int D, int kgs, const int* __restrict__ base_dev, int b_off) {
    const int row = H * D;
    const int hc = blockIdx.x * blockDim.x + threadIdx.x;
    if (hc >= row) return;
    const int b = b_off + static_cast<int>(blockIdx.y);
    const int ob = b + (base_dev ? *base_dev : 0);
    const int c = hc % D;
    const size_t mi = static_cast<size_t>(ob) * row + hc;
    quant_k_channel<MetaT>(K + static_cast<size_t>(b) * kgs * row + hc, row, kgs, c < (D / 8) * 8, scale + mi,
                           zero + mi, packed + static_cast<size_t>(ob) * (kgs / 16) * row + hc, row);
}

// One lane per packed word of a (token, head) row: the row's D / 16 words
// on an aligned group of `group` lanes (a power of two, at most 64, so the
// group lies in one wave; lanes past D / 16 only pad the min/max tree), the
// loads of a row coalesced. D % 16 == 0 (checked by the host).
template <typename MetaT>
__global__ void __launch_bounds__(256) quantize_v_kernel(const float* __restrict__ V, int32_t* __restrict__ packed,
                                                         MetaT* __restrict__ scale, MetaT* __restrict__ zero,
                                                         int tokens, int H, int D, int group,
                                                         const int* __restrict__ base_dev, int tokens_per_block) {
    const int wpr = D / 16;
    const long long th = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    // whole groups leave together: the total is a multiple of the group size
    if (th >= static_cast<long long>(tokens) * H * group) return;
    const int r = static_cast<int>(th / group), w = static_cast<int>(th % group);
    const int t = r / H, h = r % H;
    const int ot = t + (base_dev ? (*base_dev) * tokens_per_block : 0);
    const size_t mi = static_cast<size_t>(ot) * H + h;
    quant_v_row_lanes<MetaT>(V + static_cast<size_t>(t) * H * D + static_cast<size_t>(h) * D, w, wpr, group,
                             scale + mi, zero + mi, packed + mi * wpr);
}

// Rows of more than 64 words (D > 1024): one thread per (token, head) row.
template <typename MetaT>
__global__ void __launch_bounds__(256) quantize_v_serial_kernel(const float* __restrict__ V,
                                                                int32_t* __restrict__ packed,
                                                                MetaT* __restrict__ scale, MetaT* __restrict__ zero,
                                                                int tokens, int H, int D) {
    const int wpr = D / 16;
    const long long r = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= static_cast<long long>(tokens) * H) return;
    const size_t mi = static_cast<size_t>(r);
    quant_v_row_serial<MetaT>(V + mi * D, wpr, scale + mi, zero + mi, packed + mi * wpr);
}

// One thread per (block, head, channel): x = fmaf((float)q, scale, zero).
template <typename MetaT>
__global__ void __launch_bounds__(256) dequantize_k_kernel(const int32_t* __restrict__ packed,
                                                           const MetaT* __restrict__ scale,
                                                           const MetaT* __restrict__ zero, float* __restrict__ out,
                                                           int H, int D, int kgs, int b_off) {
    const int row = H * D;
    const int hc = blockIdx.x * blockDim.x + threadIdx.x;
    if (hc >= row) return;
    const int b = b_off + static_cast<int>(blockIdx.y);
    const float s = Meta<MetaT>::load(scale, static_cast<size_t>(b) * row + hc);
    const float z = Meta<MetaT>::load(zero, static_cast<size_t>(b) * row + hc);
    const int words = kgs / 16;
    for (int w = 0; w < words; ++w) {
        const uint32_t p = static_cast<uint32_t>(packed[(static_cast<size_t>(b) * words + w) * row + hc]);
        for (int st = 0; st < 16; ++st) {
            const size_t tok = static_cast<size_t>(b) * kgs + w * 16 + st;
            out[tok * row + hc] = __builtin_fmaf(static_cast<float>((p >> (2 * st)) & 3u), s, z);
        }
    }
}

// One thread per (token, head, 16-channel group).
template <typename MetaT>
__global__ void __launch_bounds__(256) dequantize_v_kernel(const int32_t* __restrict__ packed,
                                                           const MetaT* __restrict__ scale,
                                                           const MetaT* __restrict__ zero, float* __restrict__ out,
                                                           int tokens, int H, int D) {
    const int qhd = D / 16;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<long long>(tokens) * H * qhd) return;
    const int g = static_cast<int>(idx % qhd);
    const long long th = idx / qhd;  // token * H + head
    const float s = Meta<MetaT>::load(scale, static_cast<size_t>(th));
    const float z = Meta<MetaT>::load(zero, static_cast<size_t>(th));
    const uint32_t p = static_cast<uint32_t>(packed[idx]);
    float* o = out + static_cast<size_t>(th) * D + g * 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = __builtin_fmaf(static_cast<float>((p >> (2 * i)) & 3u), s, z);
}

}  // namespace

int launch_quantize_k(const float* K, uint32_t* packed, void* scale, void* zero, int num_blocks, int H, int D,
                      int kgs, int meta_fp16, const int* base_dev, hipStream_t stream) {
    if (num_blocks <= 0 || H * D <= 0) return TT_OK;
    // blocks in slices of at most kMaxGridY (the grid's y extent)
    for (int b0 = 0; b0 < num_blocks; b0 += kMaxGridY) {
        const dim3 grid((H * D + 255) / 256, std::min(kMaxGridY, num_blocks - b0));
        if (meta_fp16)
            hipLaunchKernelGGL(quantize_k_kernel<uint16_t>, grid, dim3(256), 0, stream, K, packed,
                               static_cast<uint16_t*>(scale), static_cast<uint16_t*>(zero), H, D, kgs, base_dev, b0);
        else
            hipLaunchKernelGGL(quantize_k_kernel<float>, grid, dim3(256), 0, stream, K, packed,
                               static_cast<float*>(scale), static_cast<float*>(zero), H, D, kgs, base_dev, b0);
        TT_LAUNCH_CHECK();
    }
    return TT_OK;
}

int launch_quantize_v(const float* V, int32_t* packed, void* scale, void* zero, int tokens, int H, int D,
                      int meta_fp16, const int* base_dev, int tokens_per_block, hipStream_t stream) {
    if (tokens <= 0 || H <= 0) return TT_OK;
    const int group = quant_v_group(D / 16);
    if (group == 0) {
        if (base_dev) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "quantize_v: head_dim above 1024 in the engine");
        const long long rows = static_cast<long long>(tokens) * H;
        if (rows > kMaxThreads) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "quantize_v: tokens x heads too large for one call");
        const dim3 grid(static_cast<unsigned>((rows + 255) / 256));
        if (meta_fp16)
            hipLaunchKernelGGL(quantize_v_serial_kernel<uint16_t>, grid, dim3(256), 0, stream, V, packed,
                               static_cast<uint16_t*>(scale), static_cast<uint16_t*>(zero), tokens, H, D);
        else
            hipLaunchKernelGGL(quantize_v_serial_kernel<float>, grid, dim3(256), 0, stream, V, packed,
                               static_cast<float*>(scale), static_cast<float*>(zero), tokens, H, D);
        TT_LAUNCH_CHECK();
        return TT_OK;
    }
    const long long n = static_cast<long long>(tokens) * H * group;
    if (n > kMaxThreads) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "quantize_v: tokens x heads too large for one call");
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    if (meta_fp16)
        hipLaunchKernelGGL(quantize_v_kernel<uint16_t>, grid, dim3(256), 0, stream, V, packed,
                           static_cast<uint16_t*>(scale), static_cast<uint16_t*>(zero), tokens, H, D, group, base_dev,
                           tokens_per_block);
    else
        hipLaunchKernelGGL(quantize_v_kernel<float>, grid, dim3(256), 0, stream, V, packed, static_cast<float*>(scale),
                           static_cast<float*>(zero), tokens, H, D, group, base_dev, tokens_per_block);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

int launch_dequantize_k(const int32_t* packed, const void* scale, const void* zero, float* out, int num_blocks,
                        int H, int D, int kgs, int meta_fp16, hipStream_t stream) {
    if (num_blocks <= 0 || H * D <= 0) return TT_OK;
    for (int b0 = 0; b0 < num_blocks; b0 += kMaxGridY) {
        const dim3 grid((H * D + 255) / 256, std::min(kMaxGridY, num_blocks - b0));
        if (meta_fp16)
            hipLaunchKernelGGL(dequantize_k_kernel<uint16_t>, grid, dim3(256), 0, stream, packed,
                               static_cast<const uint16_t*>(scale), static_cast<const uint16_t*>(zero), out, H, D,
                               kgs, b0);
        else
            hipLaunchKernelGGL(dequantize_k_kernel<float>, grid, dim3(256), 0, stream, packed,
                               static_cast<const float*>(scale), static_cast<const float*>(zero), out, H, D, kgs, b0);
        TT_LAUNCH_CHECK();
    }
    return TT_OK;
}

int launch_dequantize_v(const int32_t* packed, const void* scale, const void* zero, float* out, int tokens, int H,
                        int D, int meta_fp16, hipStream_t stream) {
    const long long n = static_cast<long long>(tokens) * H * (D / 16);
    if (n <= 0) return TT_OK;
    if (n > kMaxThreads) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "dequantize_v: tokens x heads too large for one call");
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    if (meta_fp16)
        hipLaunchKernelGGL(dequantize_v_kernel<uint16_t>, grid, dim3(256), 0, stream, packed,
                           static_cast<const uint16_t*>(scale), static_cast<const uint16_t*>(zero), out, tokens, H, D);
    else
        hipLaunchKernelGGL(dequantize_v_kernel<float>, grid, dim3(256), 0, stream, packed,
                           static_cast<const float*>(scale), static_cast<const float*>(zero), out, tokens, H, D);
    TT_LAUNCH_CHECK();
    return TT_OK;
}

}  // namespace tt
