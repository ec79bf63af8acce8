// tt_capi.hip -- extern "C" entry points for the stateless kernels, error
// reporting and device queries. The engine's entry points are in tt_engine.hip.
//
// Argument validation follows the reference binding (csrc/bindings.cpp:120-128,
// 139-147: counts non-negative, heads/dim positive, data pointers nullable
// exactly when their count is zero) and adds the shape limits of the gfx950
// kernels (GQA ratio integral, head_dim a multiple of 16 of at most 256).
#include "tt_attn.h"

#include <mutex>
#include <unordered_map>

namespace tt {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

namespace {

// Library-owned attention workspace, one per device, grown on demand.
struct DeviceWorkspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::unordered_map<int, DeviceWorkspace> g_ws;

int get_workspace(size_t bytes, void** out) {
    int dev = 0;
    TT_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    DeviceWorkspace& w = g_ws[dev];
    if (w.bytes < bytes) {
        if (w.ptr) {
            TT_HIP_CHECK(hipDeviceSynchronize());
            TT_HIP_CHECK(hipFree(w.ptr));
            w.ptr = nullptr;
            w.bytes = 0;
        }
        const size_t nb = std::max(bytes, static_cast<size_t>(1) << 20);
        TT_HIP_CHECK(hipMalloc(&w.ptr, nb));
        w.bytes = nb;
    }
    *out = w.ptr;
    return TT_OK;
}

// Allocation-free workspace: a file-scope device array that every GPU the
// library runs on holds until the process ends. In host code `scratch` only
// names the symbol; its device address on the current GPU comes from
// hipGetSymbolAddress, once per device, and only that address is passed to
// kernels. Every call on one GPU shares that GPU's copy, so calls that
// overlap on one GPU race on it.
constexpr size_t kScratchBytes = static_cast<size_t>(32) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device.
int scratch_address(void** out) {
    int dev = 0;
    TT_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxScratchDevices)
        TT_FAIL(TT_ERR_RUNTIME, "tt_fused_attention_decode_noalloc: device index beyond the scratch table.");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        TT_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) TT_FAIL(TT_ERR_RUNTIME, "tt_fused_attention_decode_noalloc: no device address for the scratch array.");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TT_OK;
}

int check_common(int dense_count, int num_blocks, int Hq, int Hkv, int D, int kgs) {
    if (dense_count < 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "dense_count must be non-negative.");
    if (num_blocks < 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_blocks must be non-negative.");
    const int rc = attn_check_shapes(Hq, Hkv, D, kgs);
    if (rc) return rc;
    // token positions and the padded logits rows are int
    if (static_cast<long long>(dense_count) + static_cast<long long>(num_blocks) * kgs > INT_MAX - 64)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "dense_count + num_blocks x k_group_size must stay below 2^31.");
    return TT_OK;
}

// Validates the stateless attention arguments and fills the kernel inputs and plan.
int prepare(const float* Q, const float* dK, const float* dV, int dense_count, const int32_t* KP, const void* KS,
            const void* KZ, const int32_t* VP, const void* VS, const void* VZ, const int64_t* ids, int num_blocks,
            int Hq, int Hkv, int D, int kgs, int meta_fp16, bool want_mw, AttnInputs* in, AttnPlan* plan) {
    int rc = check_common(dense_count, num_blocks, Hq, Hkv, D, kgs);
    if (rc) return rc;
    if (!Q) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'Q' pointer address is NULL.");
    if (dense_count > 0 && (!dK || !dV))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'dense_K'/'dense_V' pointer address is NULL.");
    if (num_blocks > 0 && (!KP || !KS || !KZ || !VP || !VS || !VZ || !ids))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "PBS arguments must be non-NULL when num_blocks > 0.");
    *plan = attn_plan(dense_count, num_blocks, Hq, Hkv, D, kgs, want_mw, meta_fp16);
    if (want_mw && !logits_fit(Hq, plan->ld))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_q_heads x tokens exceeds the 4 GiB logits buffer of the mean weights.");
    in->Q = Q;
    in->k0 = dK;
    in->v0 = dV;
    in->n0 = dense_count;
    in->kp = KP;
    in->ks = KS;
    in->kz = KZ;
    in->vp = VP;
    in->vs = VS;
    in->vz = VZ;
    in->ids = ids;
    in->num_blocks = num_blocks;
    in->Hq = Hq;
    in->Hkv = Hkv;
    in->D = D;
    in->kgs = kgs;
    in->meta_fp16 = meta_fp16 ? 1 : 0;
    return TT_OK;
}

enum Phase { kBoth, kPartials, kFinalize };

int fused_impl(const float* Q, const float* dK, const float* dV, int dense_count, const int32_t* KP, const void* KS,
               const void* KZ, const int32_t* VP, const void* VS, const void* VZ, const int64_t* ids, int num_blocks,
               int Hq, int Hkv, int D, float* out, float* mw, int kgs, int meta_fp16, void* ws, size_t ws_bytes,
               bool own_ws, Phase phase, int want_mw, hipStream_t s) {
    AttnInputs in;
    AttnPlan plan;
    const bool logits = (phase == kBoth) ? (mw != nullptr) : (want_mw != 0);
    int rc = prepare(Q, dK, dV, dense_count, KP, KS, KZ, VP, VS, VZ, ids, num_blocks, Hq, Hkv, D, kgs, meta_fp16,
                     logits, &in, &plan);
    if (rc) return rc;
    if (phase == kBoth && !out) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'attn_output' pointer address is NULL.");
    if (phase == kFinalize && !out && !mw)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "tt_attention_finalize: attn_output and mean_attn_weights are both NULL.");
    if (phase == kFinalize && mw && !logits)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "mean_attn_weights requested but the partials were planned without them.");
    if (own_ws) {
        rc = get_workspace(plan.bytes, &ws);
        if (rc) return rc;
    } else if (!ws || ws_bytes < plan.bytes) {
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "workspace is NULL or smaller than tt_fused_attention_workspace_bytes().");
    }
    if (phase == kPartials) return attn_launch_split(in, plan, ws, s);
    if (phase == kFinalize)
        return attn_launch_finalize(in, plan, ws, out, mw, nullptr, nullptr, 0, s,
                                    !mw ? FinRoles::kMerge : (!out ? FinRoles::kMean : FinRoles::kBoth));
    return attn_launch(in, plan, ws, out, mw, nullptr, nullptr, 0, s);
}

// Validates a batch: shapes, and each sequence as tt_fused_attention_decode
// validates its arguments.
int check_batch(const tt_decode_seq* seqs, int num_seqs, int Hq, int Hkv, int D, int kgs) {
    if (num_seqs < 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_seqs must be non-negative.");
    if (num_seqs > 0 && !seqs) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'seqs' pointer address is NULL.");
    int rc = attn_check_shapes(Hq, Hkv, D, kgs);
    if (rc) return rc;
    long long tokens = 0;
    for (int i = 0; i < num_seqs; ++i) {
        const tt_decode_seq& q = seqs[i];
        tokens += static_cast<long long>(q.dense_count) + static_cast<long long>(q.num_blocks) * kgs + 4;
        if (tokens > INT_MAX) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "the batch holds more than 2^31 tokens.");
        const long long tub = static_cast<long long>(q.dense_count) + static_cast<long long>(q.num_blocks) * kgs;
        if (q.mean_attn_weights && !logits_fit(Hq, (tub + 3) & ~3LL))
            TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_q_heads x tokens exceeds the 4 GiB logits buffer of the mean weights.");
        AttnInputs in;
        AttnPlan plan;
        rc = prepare(q.Q, q.dense_K, q.dense_V, q.dense_count, q.PBS_K_Packed, q.PBS_K_Scales, q.PBS_K_Zeroes,
                     q.PBS_V_Packed, q.PBS_V_Scales, q.PBS_V_Zeroes, q.PBS_token_ids, q.num_blocks, Hq, Hkv, D, kgs, 0,
                     false, &in, &plan);
        if (rc) return rc;
        if (!q.attn_output) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'attn_output' pointer address is NULL.");
    }
    return TT_OK;
}

// Workspace of a batch: the largest launch (chunks of kMaxBatchSeqs sequences
// run one after another on the stream and share it); other head dims run the
// sequences one at a time.
size_t batch_bytes(const tt_decode_seq* seqs, int num_seqs, int Hq, int Hkv, int D, int kgs, int meta_fp16) {
    size_t b = 0;
    if (!use_packed_kernel(D)) {
        for (int i = 0; i < num_seqs; ++i)
            b = std::max(b, attn_plan(seqs[i].dense_count, seqs[i].num_blocks, Hq, Hkv, D, kgs,
                                      seqs[i].mean_attn_weights != nullptr, meta_fp16)
                                .bytes);
        return b;
    }
    for (int c0 = 0; c0 < num_seqs; c0 += kMaxBatchSeqs)
        b = std::max(b, batch_plan(seqs + c0, std::min(kMaxBatchSeqs, num_seqs - c0), Hq, Hkv, D, kgs, meta_fp16).bytes);
    return b;
}

}  // namespace
}  // namespace tt

using namespace tt;

extern "C" {

const char* tt_last_error(void) { return g_last_error.c_str(); }

const char* tt_version(void) { return "tritiercache_amd 0.1.0 gfx950"; }

int tt_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int tt_pointer_kind(const void* ptr) {
    if (!ptr) return 0;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged) return 1;
    if (attr.type == hipMemoryTypeHost) return 2;
    return 0;
}

int tt_quantize_k_block(const float* K, uint32_t* packed, void* scale, void* zero, int num_blocks, int num_heads,
                        int head_dim, int k_group_size, int meta_fp16, void* stream) {
    clear_error();
    if (num_blocks < 0 || num_heads <= 0 || head_dim <= 0)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_blocks must be >= 0; num_heads and head_dim must be positive.");
    if (k_group_size != 16 && k_group_size != 32) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "k_group_size must be 16 or 32.");
    if (!K || !packed || !scale || !zero) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "quantize_k_block: NULL pointer argument.");
    return launch_quantize_k(K, packed, scale, zero, num_blocks, num_heads, head_dim, k_group_size, meta_fp16, nullptr,
                             as_stream(stream));
}

int tt_quantize_v_block(const float* V, int32_t* packed, void* scale, void* zero, int tokens, int num_heads,
                        int head_dim, int meta_fp16, void* stream) {
    clear_error();
    if (tokens < 0 || num_heads <= 0 || head_dim <= 0)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "tokens must be >= 0; num_heads and head_dim must be positive.");
    if (head_dim % 16 != 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "quantize_v_block: head_dim must be a multiple of 16.");
    if (!V || !packed || !scale || !zero) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "quantize_v_block: NULL pointer argument.");
    return launch_quantize_v(V, packed, scale, zero, tokens, num_heads, head_dim, meta_fp16, nullptr, 0,
                             as_stream(stream));
}

int tt_dequantize_k(const int32_t* packed, const void* scale, const void* zero, float* out, int num_blocks,
                    int num_heads, int head_dim, int k_group_size, int meta_fp16, void* stream) {
    clear_error();
    if (num_blocks < 0 || num_heads <= 0 || head_dim <= 0)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "num_blocks must be >= 0; num_heads and head_dim must be positive.");
    if (k_group_size != 16 && k_group_size != 32) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "k_group_size must be 16 or 32.");
    if (num_blocks > 0 && (!packed || !scale || !zero || !out))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "dequantize_k: NULL pointer argument.");
    return launch_dequantize_k(packed, scale, zero, out, num_blocks, num_heads, head_dim, k_group_size, meta_fp16,
                               as_stream(stream));
}

int tt_dequantize_v(const int32_t* packed, const void* scale, const void* zero, float* out, int total_tokens,
                    int num_heads, int head_dim, int meta_fp16, void* stream) {
    clear_error();
    if (total_tokens < 0 || num_heads <= 0 || head_dim <= 0)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "total_tokens must be >= 0; num_heads and head_dim must be positive.");
    if (head_dim % 16 != 0) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "dequantize_v: head_dim must be a multiple of 16.");
    if (total_tokens > 0 && (!packed || !scale || !zero || !out))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "dequantize_v: NULL pointer argument.");
    return launch_dequantize_v(packed, scale, zero, out, total_tokens, num_heads, head_dim, meta_fp16,
                               as_stream(stream));
}

int tt_fused_attention_decode(const float* Q, const float* dense_K, const float* dense_V, int dense_count,
                              const int32_t* PBS_K_Packed, const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                              const int32_t* PBS_V_Packed, const void* PBS_V_Scales, const void* PBS_V_Zeroes,
                              const int64_t* PBS_token_ids, int num_blocks, int num_q_heads, int num_kv_heads,
                              int head_dim, float* attn_output, float* mean_attn_weights, int k_group_size,
                              int meta_fp16, void* stream) {
    clear_error();
    return fused_impl(Q, dense_K, dense_V, dense_count, PBS_K_Packed, PBS_K_Scales, PBS_K_Zeroes, PBS_V_Packed,
                      PBS_V_Scales, PBS_V_Zeroes, PBS_token_ids, num_blocks, num_q_heads, num_kv_heads, head_dim,
                      attn_output, mean_attn_weights, k_group_size, meta_fp16, nullptr, 0, true, kBoth, 0,
                      as_stream(stream));
}

int tt_fused_attention_decode_noalloc(const float* Q, const float* dense_K, const float* dense_V, int dense_count,
                                      const int32_t* PBS_K_Packed, const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                                      const int32_t* PBS_V_Packed, const void* PBS_V_Scales, const void* PBS_V_Zeroes,
                                      const int64_t* PBS_token_ids, int num_blocks, int num_q_heads, int num_kv_heads,
                                      int head_dim, float* attn_output, float* mean_attn_weights, int k_group_size,
                                      int meta_fp16, void* stream) {
    clear_error();
    AttnInputs in;
    AttnPlan plan;
    int rc = prepare(Q, dense_K, dense_V, dense_count, PBS_K_Packed, PBS_K_Scales, PBS_K_Zeroes, PBS_V_Packed,
                     PBS_V_Scales, PBS_V_Zeroes, PBS_token_ids, num_blocks, num_q_heads, num_kv_heads, head_dim,
                     k_group_size, meta_fp16, mean_attn_weights != nullptr, &in, &plan);
    if (rc) return rc;
    if (plan.bytes > kScratchBytes)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "tt_fused_attention_decode_noalloc: the call needs " +
                                             std::to_string(plan.bytes) + " bytes of scratch; the static scratch holds " +
                                             std::to_string(kScratchBytes) +
                                             " (use tt_fused_attention_decode_ws with a larger workspace).");
    void* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc) return rc;
    return fused_impl(Q, dense_K, dense_V, dense_count, PBS_K_Packed, PBS_K_Scales, PBS_K_Zeroes, PBS_V_Packed,
                      PBS_V_Scales, PBS_V_Zeroes, PBS_token_ids, num_blocks, num_q_heads, num_kv_heads, head_dim,
                      attn_output, mean_attn_weights, k_group_size, meta_fp16, ws, kScratchBytes, false, kBoth, 0,
                      as_stream(stream));
}

size_t tt_fused_attention_workspace_bytes(int dense_count, int num_blocks, int num_q_heads, int num_kv_heads,
                                          int head_dim, int k_group_size, int want_mean_weights) {
    clear_error();
    if (check_common(dense_count, num_blocks, num_q_heads, num_kv_heads, head_dim, k_group_size) != TT_OK) return 0;
    // The largest plan over both metadata types (their split counts can differ).
    size_t b = 0;
    for (int f = 0; f < 2; ++f) {
        const AttnPlan p = attn_plan(dense_count, num_blocks, num_q_heads, num_kv_heads, head_dim, k_group_size,
                                     want_mean_weights != 0, f);
        if (want_mean_weights && !logits_fit(num_q_heads, p.ld)) {
            set_error("num_q_heads x tokens exceeds the 4 GiB logits buffer of the mean weights.");
            return 0;
        }
        b = std::max(b, p.bytes);
    }
    return b;
}

int tt_fused_attention_decode_ws(const float* Q, const float* dense_K, const float* dense_V, int dense_count,
                                 const int32_t* PBS_K_Packed, const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                                 const int32_t* PBS_V_Packed, const void* PBS_V_Scales, const void* PBS_V_Zeroes,
                                 const int64_t* PBS_token_ids, int num_blocks, int num_q_heads, int num_kv_heads,
                                 int head_dim, float* attn_output, float* mean_attn_weights, int k_group_size,
                                 int meta_fp16, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    return fused_impl(Q, dense_K, dense_V, dense_count, PBS_K_Packed, PBS_K_Scales, PBS_K_Zeroes, PBS_V_Packed,
                      PBS_V_Scales, PBS_V_Zeroes, PBS_token_ids, num_blocks, num_q_heads, num_kv_heads, head_dim,
                      attn_output, mean_attn_weights, k_group_size, meta_fp16, workspace, workspace_bytes, false,
                      kBoth, 0, as_stream(stream));
}

int tt_attention_partials(const float* Q, const float* dense_K, const float* dense_V, int dense_count,
                          const int32_t* PBS_K_Packed, const void* PBS_K_Scales, const void* PBS_K_Zeroes,
                          const int32_t* PBS_V_Packed, const void* PBS_V_Scales, const void* PBS_V_Zeroes,
                          const int64_t* PBS_token_ids, int num_blocks, int num_q_heads, int num_kv_heads, int head_dim,
                          int k_group_size, int meta_fp16, int want_mean_weights, void* workspace,
                          size_t workspace_bytes, void* stream) {
    clear_error();
    return fused_impl(Q, dense_K, dense_V, dense_count, PBS_K_Packed, PBS_K_Scales, PBS_K_Zeroes, PBS_V_Packed,
                      PBS_V_Scales, PBS_V_Zeroes, PBS_token_ids, num_blocks, num_q_heads, num_kv_heads, head_dim,
                      nullptr, nullptr, k_group_size, meta_fp16, workspace, workspace_bytes, false, kPartials,
                      want_mean_weights, as_stream(stream));
}

int tt_attention_finalize(const float* Q, int dense_count, int num_blocks, int num_q_heads, int num_kv_heads,
                          int head_dim, float* attn_output, float* mean_attn_weights, int k_group_size, int meta_fp16,
                          int want_mean_weights, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    // The finalize phase reads only the workspace; the tier pointers are not
    // dereferenced, so placeholders satisfy the shared validation.
    const void* ph = workspace;
    return fused_impl(Q, static_cast<const float*>(ph), static_cast<const float*>(ph), dense_count,
                      static_cast<const int32_t*>(ph), ph, ph, static_cast<const int32_t*>(ph), ph, ph,
                      static_cast<const int64_t*>(ph), num_blocks, num_q_heads, num_kv_heads, head_dim, attn_output,
                      mean_attn_weights, k_group_size, meta_fp16, workspace, workspace_bytes, false, kFinalize,
                      want_mean_weights, as_stream(stream));
}

int tt_attention_finalize_deferred(const float* Q, int dense_count, int num_blocks, int num_q_heads,
                                   int num_kv_heads, int head_dim, float* attn_output, int k_group_size,
                                   int meta_fp16, void* workspace, size_t workspace_bytes, int prev_dense_count,
                                   int prev_num_blocks, float* prev_mean_attn_weights, void* prev_workspace,
                                   size_t prev_workspace_bytes, void* stream) {
    clear_error();
    if (!attn_output) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'attn_output' pointer address is NULL.");
    if (!prev_mean_attn_weights)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'prev_mean_attn_weights' pointer address is NULL.");
    if (!workspace || !prev_workspace)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "workspace or prev_workspace is NULL.");
    const char* w0 = static_cast<const char*>(workspace);
    const char* w1 = static_cast<const char*>(prev_workspace);
    if (w0 < w1 + prev_workspace_bytes && w1 < w0 + workspace_bytes)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "workspace and prev_workspace overlap.");
    // Only the workspaces are read; the tier pointers are placeholders for the
    // shared validation.
    AttnInputs in, prev_in;
    AttnPlan plan, prev_plan;
    const void* ph = workspace;
    int rc = prepare(Q, static_cast<const float*>(ph), static_cast<const float*>(ph), dense_count,
                     static_cast<const int32_t*>(ph), ph, ph, static_cast<const int32_t*>(ph), ph, ph,
                     static_cast<const int64_t*>(ph), num_blocks, num_q_heads, num_kv_heads, head_dim, k_group_size,
                     meta_fp16, true, &in, &plan);
    if (rc) return rc;
    rc = prepare(Q, static_cast<const float*>(ph), static_cast<const float*>(ph), prev_dense_count,
                 static_cast<const int32_t*>(ph), ph, ph, static_cast<const int32_t*>(ph), ph, ph,
                 static_cast<const int64_t*>(ph), prev_num_blocks, num_q_heads, num_kv_heads, head_dim, k_group_size,
                 meta_fp16, true, &prev_in, &prev_plan);
    if (rc) return rc;
    if (workspace_bytes < plan.bytes || prev_workspace_bytes < prev_plan.bytes)
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "workspace is NULL or smaller than tt_fused_attention_workspace_bytes().");
    return attn_launch_finalize_deferred(in, plan, workspace, attn_output, prev_in, prev_plan, prev_workspace,
                                         prev_mean_attn_weights, nullptr, as_stream(stream));
}

size_t tt_batched_decode_workspace_bytes(const tt_decode_seq* seqs, int num_seqs, int num_q_heads, int num_kv_heads,
                                         int head_dim, int k_group_size) {
    clear_error();
    if (check_batch(seqs, num_seqs, num_q_heads, num_kv_heads, head_dim, k_group_size) != TT_OK) return 0;
    if (num_seqs == 0) return 256;
    // The largest plan over both metadata types (their split counts can differ).
    return std::max(batch_bytes(seqs, num_seqs, num_q_heads, num_kv_heads, head_dim, k_group_size, 0),
                    batch_bytes(seqs, num_seqs, num_q_heads, num_kv_heads, head_dim, k_group_size, 1));
}

int tt_fused_attention_decode_batched(const tt_decode_seq* seqs, const tt_decode_seq* seqs_device, int num_seqs,
                                      int num_q_heads, int num_kv_heads, int head_dim, int k_group_size, int meta_fp16,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    const int Hq = num_q_heads, Hkv = num_kv_heads, D = head_dim, kgs = k_group_size;
    int rc = check_batch(seqs, num_seqs, Hq, Hkv, D, kgs);
    if (rc) return rc;
    if (num_seqs == 0) return TT_OK;
    if (!workspace || workspace_bytes < batch_bytes(seqs, num_seqs, Hq, Hkv, D, kgs, meta_fp16))
        TT_FAIL(TT_ERR_INVALID_ARGUMENT, "workspace is NULL or smaller than tt_batched_decode_workspace_bytes().");
    const hipStream_t s = as_stream(stream);
    if (!use_packed_kernel(D)) {
        for (int i = 0; i < num_seqs; ++i) {
            const tt_decode_seq& q = seqs[i];
            AttnInputs in;
            AttnPlan plan;
            rc = prepare(q.Q, q.dense_K, q.dense_V, q.dense_count, q.PBS_K_Packed, q.PBS_K_Scales, q.PBS_K_Zeroes,
                         q.PBS_V_Packed, q.PBS_V_Scales, q.PBS_V_Zeroes, q.PBS_token_ids, q.num_blocks, Hq, Hkv, D, kgs,
                         meta_fp16, q.mean_attn_weights != nullptr, &in, &plan);
            if (rc) return rc;
            rc = attn_launch(in, plan, workspace, q.attn_output, q.mean_attn_weights, nullptr, nullptr, 0, s);
            if (rc) return rc;
        }
        return TT_OK;
    }
    if (!seqs_device) TT_FAIL(TT_ERR_INVALID_ARGUMENT, "Argument 'seqs_device' pointer address is NULL.");
    for (int c0 = 0; c0 < num_seqs; c0 += kMaxBatchSeqs) {
        const int n = std::min(kMaxBatchSeqs, num_seqs - c0);
        const BatchPlan plan = batch_plan(seqs + c0, n, Hq, Hkv, D, kgs, meta_fp16);
        rc = batch_launch(plan, seqs_device + c0, Hq, Hkv, kgs, meta_fp16, workspace, s);
        if (rc) return rc;
    }
    return TT_OK;
}

}  // extern "C"
