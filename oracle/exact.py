"""Float64 softmax attention over a tiered layer's exact values (test infrastructure only:
the parity tests and bench.py's baseline leg compare results against it).

The FP32 dense rows are taken as they are and the packed rows as the oracle's
bit-exact dequantisation (x = fmaf(q, scale, zero), csrc/cpu/dequantize_avx2.cpp
of the reference), so the only rounding left is float64's. This is the textbook
computation the reference's fused_attention_decode approximates in float32
(csrc/cpu/fused_attn_avx2.cpp:145-301): scores q.k / sqrt(D), softmax over the
valid tokens (ids of -1 excluded), GQA head h reading KV head h / (Hq / Hkv),
mean weights = the per-head softmax weights averaged over query heads.

Also the elementwise error measures the parity tests bound.
"""
from __future__ import annotations

import numpy as np


def exact_attention(oracle, Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs=16, fp16=False,
                    per_head=False):
    """(out [Hq, D], mean weights [nd + nb * kgs]) in float64; with per_head also the
    per-head softmax weights [Hq, nd + nb * kgs] (0 at masked tokens), the weights
    the reference's torch path returns for output_attentions
    (src/tri_tier/integration/patch_model.py:33-51)."""
    G = Hq // Hkv
    parts_k, parts_v = [], []
    if nd:
        parts_k.append(np.asarray(dK, np.float32).reshape(nd, Hkv, D)[:nd])
        parts_v.append(np.asarray(dV, np.float32).reshape(nd, Hkv, D)[:nd])
    valid = [np.ones(nd, bool)]
    if nb:
        parts_k.append(oracle.dequantize_k(KP, KS, KZ, nb, Hkv, D, kgs, fp16))
        parts_v.append(oracle.dequantize_v(VP, VS, VZ, nb * kgs, Hkv, D, fp16))
        valid.append(np.asarray(ids).reshape(-1)[: nb * kgs] != -1)
    valid = np.concatenate(valid)
    n = valid.size
    out = np.zeros((Hq, D))
    mw = np.zeros(n)
    W = np.zeros((Hq, n))
    if n == 0:
        return (out, mw, W) if per_head else (out, mw)
    K = np.concatenate(parts_k)
    V = np.concatenate(parts_v)
    q = np.asarray(Q, np.float32).reshape(Hq, D).astype(np.float64)
    for h in range(Hkv):
        kh = np.ascontiguousarray(K[:, h, :]).astype(np.float64)  # [n, D]
        s = (q[h * G:(h + 1) * G] @ kh.T) / np.sqrt(D)            # [G, n]
        s[:, ~valid] = -np.inf
        m = s.max(axis=1, keepdims=True)
        m[~np.isfinite(m)] = 0.0
        p = np.exp(s - m)
        L = p.sum(axis=1, keepdims=True)
        L[L == 0] = 1.0
        w = p / L
        W[h * G:(h + 1) * G] = w
        out[h * G:(h + 1) * G] = w @ np.ascontiguousarray(V[:, h, :]).astype(np.float64)
        mw += w.sum(axis=0)
    return (out, mw / Hq, W) if per_head else (out, mw / Hq)


def elementwise_ratio(got, want, rtol=1e-4, atol_frac=1e-6) -> float:
    """max_i |got_i - want_i| / (rtol |want_i| + atol_frac max|want|): <= 1 passes."""
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    bound = rtol * np.abs(want) + atol_frac * max(float(np.abs(want).max()), 1e-30)
    return float((np.abs(got - want) / bound).max()) if want.size else 0.0


def weights_rel_err(got, want, floor=1e-8) -> float:
    """Max elementwise relative error of attention weights over the weights >= floor."""
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    m = want >= floor
    return float((np.abs(got[m] - want[m]) / want[m]).max()) if m.any() else 0.0


def engine_exact_attention(oracle, state, Q, Hq, Hkv, D, kgs, fp16, per_head=False):
    """exact_attention over an engine's visible tokens, from a state dict (counters
    plus flat tier buffers, as oracle.binding.CpuEngine.state() returns): sinks,
    heavy-hitter slots, the recent window oldest first, then the used packed
    blocks -- the engine's attention order (cache_engine.cpp:433-462)."""
    c = state["counters"]
    s, hh, rw, head, nb = c["s_count"], c["hh_count"], c["rw_count"], c["rw_head_index"], c["pbs_blocks_used"]
    kvs = Hkv * D
    rows = lambda name: np.asarray(state[name]).reshape(-1, Hkv, D)  # noqa: E731
    R = rows("RW_K").shape[0]
    ring = (head + np.arange(rw)) % max(R, 1)
    dK = np.concatenate([rows("S_K")[:s], rows("HH_K")[:hh], rows("RW_K")[ring]])
    dV = np.concatenate([rows("S_V")[:s], rows("HH_V")[:hh], rows("RW_V")[ring]])
    W = kgs // 16
    KP = np.asarray(state["PBS_K_Packed"]).reshape(-1, W, Hkv, D)[:nb]
    KS = np.asarray(state["PBS_K_Scales"]).reshape(-1, Hkv, D)[:nb]
    KZ = np.asarray(state["PBS_K_Zeroes"]).reshape(-1, Hkv, D)[:nb]
    VP = np.asarray(state["PBS_V_Packed"]).reshape(-1, Hkv, (D + 15) // 16)[: nb * kgs]
    VS = np.asarray(state["PBS_V_Scales"]).reshape(-1, Hkv)[: nb * kgs]
    VZ = np.asarray(state["PBS_V_Zeroes"]).reshape(-1, Hkv)[: nb * kgs]
    ids = np.asarray(state["PBS_token_ids"]).reshape(-1)[: nb * kgs]
    assert dK.size == (s + hh + rw) * kvs
    return exact_attention(oracle, Q, dK, dV, s + hh + rw, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16,
                           per_head)


def engine_visible_ids(state):
    """Token id of every column of the engine's attention order (sinks, heavy-hitter
    slots, recent window oldest first, packed slots), from a state dict."""
    c = state["counters"]
    s, hh, rw, nb, total = (c["s_count"], c["hh_count"], c["rw_count"], c["pbs_blocks_used"],
                            c["total_processed_tokens"])
    kgs = c["k_group_size"]
    return np.concatenate([np.arange(s, dtype=np.int64), np.asarray(state["HH_token_ids"]).reshape(-1)[:hh],
                           np.arange(total - rw, total, dtype=np.int64),
                           np.asarray(state["PBS_token_ids"]).reshape(-1)[: nb * kgs]])


def reconstruct_order(state):
    """The permutation of the engine's attention order into the order of the
    reference's reconstruct_full_cache (src/tri_tier/cache.py:326-372): sinks, then
    heavy hitters and valid packed tokens sorted by token id, then the recent window
    oldest first. Packed slots with id -1 are dropped."""
    c = state["counters"]
    s, hh, rw = c["s_count"], c["hh_count"], c["rw_count"]
    ids = engine_visible_ids(state)
    nd = s + hh + rw
    middle = np.concatenate([np.arange(s, s + hh), np.arange(nd, ids.size)])
    middle = middle[ids[middle] != -1]
    middle = middle[np.argsort(ids[middle], kind="stable")]
    return np.concatenate([np.arange(s), middle, np.arange(s + hh, nd)]).astype(np.int64)


def reconstruct_full_cache(oracle, state, Hkv, D, fp16):
    """(K, V, ids) in reconstruct_order, the packed rows through the oracle's
    bit-exact dequantisers (csrc/cpu/dequantize_avx2.cpp)."""
    c = state["counters"]
    s, hh, rw, head, nb = c["s_count"], c["hh_count"], c["rw_count"], c["rw_head_index"], c["pbs_blocks_used"]
    kgs = c["k_group_size"]
    rows = lambda name: np.asarray(state[name]).reshape(-1, Hkv, D)  # noqa: E731
    R = rows("RW_K").shape[0]
    ring = (head + np.arange(rw)) % max(R, 1)
    W = kgs // 16
    parts_k = [rows("S_K")[:s], rows("HH_K")[:hh], rows("RW_K")[ring]]
    parts_v = [rows("S_V")[:s], rows("HH_V")[:hh], rows("RW_V")[ring]]
    if nb:
        parts_k.append(oracle.dequantize_k(np.asarray(state["PBS_K_Packed"]).reshape(-1, W, Hkv, D)[:nb],
                                           np.asarray(state["PBS_K_Scales"]).reshape(-1, Hkv, D)[:nb],
                                           np.asarray(state["PBS_K_Zeroes"]).reshape(-1, Hkv, D)[:nb],
                                           nb, Hkv, D, kgs, fp16))
        parts_v.append(oracle.dequantize_v(np.asarray(state["PBS_V_Packed"]).reshape(-1, Hkv, (D + 15) // 16)[: nb * kgs],
                                           np.asarray(state["PBS_V_Scales"]).reshape(-1, Hkv)[: nb * kgs],
                                           np.asarray(state["PBS_V_Zeroes"]).reshape(-1, Hkv)[: nb * kgs],
                                           nb * kgs, Hkv, D, fp16))
    K = np.concatenate(parts_k)
    V = np.concatenate(parts_v)
    perm = reconstruct_order(state)
    return K[perm], V[perm], engine_visible_ids(state)[perm]
