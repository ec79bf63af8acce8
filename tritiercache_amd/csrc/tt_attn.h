// tt_attn.h -- host interface of the fused decode attention kernels.
#pragma once
#include "tt_common.h"

namespace tt {

// Engine counters kept in device memory (int32 slots; the threshold is a
// float stored in slot kThreshold). Kernels index this array directly.
enum StateSlot : int {
    kSCount = 0,
    kRwCount = 1,
    kRwHead = 2,
    kHhCount = 3,
    kWrCount = 4,
    kBlocksUsed = 5,
    kPbsCount = 6,
    kTotal = 7,
    kLastCalcPos = 8,
    kTotalEvictions = 9,
    kLogicalAlloc = 10,
    kThreshold = 11,
    kStateSlots = 16,
};

// Where the attended tokens live. Dense tokens are, in logical order,
// seg0 rows [0, n0), seg1 rows [0, n1), then seg2 read as a ring of
// `ring_size` rows starting at `ring_head` for n2 rows. Rows are
// [num_kv_heads, head_dim] f32. For the stateless entry point seg0 is the
// caller's dense_K/V and n1 = n2 = 0. When `state` is set (engine), n0/n1/n2,
// ring_head and num_blocks are read from device memory instead.
struct AttnInputs {
    const float* Q = nullptr;
    const float* k0 = nullptr; const float* v0 = nullptr;
    const float* k1 = nullptr; const float* v1 = nullptr;
    const float* k2 = nullptr; const float* v2 = nullptr;
    int n0 = 0, n1 = 0, n2 = 0;
    int ring_size = 1, ring_head = 0;
    const int* state = nullptr;
    const int32_t* kp = nullptr; const void* ks = nullptr; const void* kz = nullptr;
    const int32_t* vp = nullptr; const void* vs = nullptr; const void* vz = nullptr;
    const int64_t* ids = nullptr;
    int num_blocks = 0;
    int Hq = 0, Hkv = 0, D = 0, kgs = 16;
    int meta_fp16 = 0;
};

// Score feedback applied by the mean-weight kernel (engine only):
// g[tid] = fmaf(decay, g[tid], mw[i]) for every visible token i, and
// HH_scores[slot] = g[tid] for heavy-hitter slots (cache_engine.cpp:511-540).
struct Feedback {
    float* g = nullptr;
    float* hh_scores = nullptr;
    const int64_t* hh_ids = nullptr;
    const int64_t* pbs_ids = nullptr;
    int max_seq_len = 0;
    float decay = 1.0f;
};

struct AttnPlan {
    int nsplit = 1;      // partial slots per query head = nsplit_p + nsplit_d
    int nsplit_p = 0;    // matrix-core workgroups over the packed store (head_dim 128)
    int nsplit_d = 1;    // VALU workgroups
    int ld = 0;          // logits row stride (floats)
    int token_ub = 0;    // upper bound on attended tokens
    int dense_delay = 0; // wait of the FP32-tier workgroups before their first load (10 ns ticks)
    // head_dim 64 with an even KV head count: KV heads 2j and 2j + 1 run as one
    // head of head_dim 128 on the matrix-core kernel (the plan is that of
    // num_kv_heads / 2 heads of 128 channels; partials hold 128 channels)
    bool pair64 = false;
    size_t off_ml = 0, off_acc = 0, off_rowstat = 0, off_logits = 0, bytes = 0;
    bool logits = false;
};

// Plans the split-K launch for an upper bound of dense tokens / blocks.
AttnPlan attn_plan(int dense_ub, int blocks_ub, int Hq, int Hkv, int D, int kgs, bool need_logits, int meta_fp16);

// Enqueues split + merge (+ mean weights / feedback / per-head weights).
// mean_w: [token count] or null; head_w: [Hq, head_w_ld] or null.
int attn_launch(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out, float* mean_w,
                const Feedback* fb, float* head_w, int head_w_ld, hipStream_t stream);
// The two phases of attn_launch: per-split partials (+ logits) into `ws`,
// then the merge / mean weights / feedback that read them.
int attn_launch_split(const AttnInputs& in, const AttnPlan& plan, void* ws, hipStream_t stream);
// Which parts of the finalize a launch runs: both in one launch (the merge
// workgroups next to the mean-weight ones, which rebuild the per-head row
// statistics themselves), the merge alone (it publishes the row statistics in
// the workspace), or the mean weights / feedback / per-head weights alone,
// reading the row statistics a merge-only launch left there.
enum class FinRoles { kBoth, kMerge, kMean };
int attn_launch_finalize(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out, float* mean_w,
                         const Feedback* fb, float* head_w, int head_w_ld, hipStream_t stream,
                         FinRoles roles = FinRoles::kBoth);
// One launch: the merge of (in, plan, ws) into out, and the mean weights (and
// score feedback, when prev_fb is given) of an earlier merge-only finalize
// whose partials, logits and row statistics are in prev_ws (planned with
// logits), into prev_mean_w.
int attn_launch_finalize_deferred(const AttnInputs& in, const AttnPlan& plan, void* ws, float* out,
                                  const AttnInputs& prev_in, const AttnPlan& prev_plan, void* prev_ws,
                                  float* prev_mean_w, const Feedback* prev_fb, hipStream_t stream);

// Validates shapes the kernels support.
int attn_check_shapes(int Hq, int Hkv, int D, int kgs);

// Whether head_dim D runs on the matrix-core split kernel (and the batched one).
bool use_packed_kernel(int D);

// Whether a logits buffer of Hq rows of ld floats stays within 4 GiB: the
// kernels store it through buffer resources, whose byte range is 32-bit.
inline bool logits_fit(long long Hq, long long ld) { return Hq * ld * 4LL <= 0xFFFFFFFFLL; }

// Batched ragged decode (head_dim 128): sequences per launch; their plan
// travels in the kernel arguments.
constexpr int kMaxBatchSeqs = 64;

// Split-K plan of one batched launch over seqs[0, nseq). Every sequence gets
// packed and FP32-tier partial slots under one cap on the work a slot
// carries (packed pairs, or 4 units per FP32 tile); the slots of all
// sequences together make one round of resident workgroups, the FP32-tier
// ones a whole number of dispatch rounds after all packed ones.
// Workspace: part_ml [slot][Hq][2] and part_acc [slot][Hq][128] in per-sequence
// runs ([Hq][nsplit_i] each), row statistics [nseq][Hq][2], logits [Hq][ld_i]
// per sequence that wants mean weights.
struct BatchPlan {
    int nseq = 0;
    int total_slots = 0;
    int slot_base[kMaxBatchSeqs + 1] = {};  // prefix of per-sequence slot counts
    int tok_base[kMaxBatchSeqs + 1] = {};   // prefix of per-sequence logits row strides
    int mean_base[kMaxBatchSeqs + 1] = {};  // prefix of per-sequence mean-weight workgroups
    // Launch order: the packed slots of all sequences (prefix pk_base), then
    // their FP32-tier slots (prefix dn_base), so that the FP32 workgroups
    // come in whole dispatch rounds, one per CU, as for one sequence.
    // Sequence i's packed slots are the first pk_base[i + 1] - pk_base[i] of
    // its slot_base run.
    int pk_base[kMaxBatchSeqs + 1] = {};
    int dn_base[kMaxBatchSeqs + 1] = {};
    size_t off_ml = 0, off_acc = 0, off_rowstat = 0, off_logits = 0, bytes = 0;
};

BatchPlan batch_plan(const tt_decode_seq* seqs, int nseq, int Hq, int Hkv, int D, int kgs, int meta_fp16);
// Enqueues the batched partials and the batched merge / mean weights.
int batch_launch(const BatchPlan& plan, const tt_decode_seq* seqs_dev, int Hq, int Hkv, int kgs, int meta_fp16,
                 void* ws, hipStream_t stream);

}  // namespace tt
