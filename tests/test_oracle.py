"""Pins the oracle (oracle/tt_oracle.c) before the parity tests trust it.

* the reference's own known-answer vectors (tests/test_quantize_v.cpp,
  tests/tie_test_v.cpp), via tests/golden/*.json;
* fixtures written by the compiled reference (tests/golden/make_golden.py):
  kernel outputs and engine state digests, bit for bit;
* what the mathematics fixes: dequantisation error bounds, field layout under
  permutation, float64 softmax attention, mean weights summing to one.
"""
import numpy as np
import pytest

from oracle import synth
import engine_runs


def same_bits(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


# ---------------------------------------------------------------- reference KATs
def test_quantize_v_reference_kat(oracle, golden):
    k = golden["qv_kat"]
    V = np.array(k["V"], np.float32).reshape(k["chunk_size"], k["num_heads"], k["head_dim"])
    p, s, z = oracle.quantize_v(V, fp16=False)
    assert np.all(np.abs(z.reshape(-1) - np.array(k["expected_min"], np.float32)) <= k["tolerance_min_scale"])
    assert np.all(np.abs(s.reshape(-1) - np.array(k["expected_scale"], np.float32)) <= k["tolerance_min_scale"])
    assert np.array_equal(p.reshape(-1).view(np.uint32), np.array(k["expected_packed"], np.uint32))
    # one (token, head) row is constant -1.5: the 1e-9 scale floor and all-zero words
    row = int(np.flatnonzero(np.array(k["expected_min"], np.float32) == np.float32(-1.5))[0])
    assert s.reshape(-1)[row] == np.float32(1e-9)
    assert np.all(p.reshape(-1, 2)[row] == 0)


def test_round_half_even_kat(oracle, golden):
    k = golden["tie_kat"]
    V = np.array(k["V"], np.float32).reshape(16, 1, 16)
    p, s, z = oracle.quantize_v(V, fp16=False)
    w = int(p.reshape(-1).view(np.uint32)[0])
    for ch, want in k["expected_q"].items():
        assert (w >> (2 * int(ch))) & 3 == want
    assert s[0, 0] == k["expected_scale0"]
    assert np.array_equal(p.reshape(-1).view(np.uint32), np.array(k["reference_packed"], np.uint32))


# ------------------------------------------------------- compiled-reference fixtures
def test_quantize_k_fixtures(oracle, golden):
    K = golden["kernels"]
    for i, c in enumerate(golden["kernels_index"]["qk"]):
        p, s, z = oracle.quantize_k(K[f"qk{i}_K"], c["kgs"], c["fp16"])
        assert same_bits(p, K[f"qk{i}_packed"]), i
        assert same_bits(s, K[f"qk{i}_scale"]) and same_bits(z, K[f"qk{i}_zero"]), i
        d = oracle.dequantize_k(p, s, z, 1, c["H"], c["D"], c["kgs"], c["fp16"])
        assert same_bits(d, K[f"qk{i}_deq"]), i


def test_quantize_v_fixtures(oracle, golden):
    K = golden["kernels"]
    for i, c in enumerate(golden["kernels_index"]["qv"]):
        p, s, z = oracle.quantize_v(K[f"qv{i}_V"], c["fp16"])
        assert same_bits(p, K[f"qv{i}_packed"]), i
        assert same_bits(s, K[f"qv{i}_scale"]) and same_bits(z, K[f"qv{i}_zero"]), i
        d = oracle.dequantize_v(p, s, z, c["chunk"], c["H"], c["D"], c["fp16"])
        assert same_bits(d, K[f"qv{i}_deq"]), i


def _fa_args(K, i, c):
    return (K[f"fa{i}_Q"], K[f"fa{i}_dK"], K[f"fa{i}_dV"], c["nd"], K[f"fa{i}_KP"], K[f"fa{i}_KS"], K[f"fa{i}_KZ"],
            K[f"fa{i}_VP"], K[f"fa{i}_VS"], K[f"fa{i}_VZ"], K[f"fa{i}_ids"], c["nb"], c["Hq"], c["Hkv"], c["D"],
            c["kgs"], c["fp16"])


def test_fused_attention_fixtures(oracle, golden):
    """Same glibc expf, same summation order as the AVX2 kernel: bit-exact on this host."""
    K = golden["kernels"]
    for i, c in enumerate(golden["kernels_index"]["fa"]):
        out, mw = oracle.fused_attention_decode(*_fa_args(K, i, c))
        np.testing.assert_allclose(out, K[f"fa{i}_out"], rtol=0, atol=2e-6 * max(1.0, np.abs(out).max()))
        np.testing.assert_allclose(mw, K[f"fa{i}_mw"], rtol=0, atol=1e-7)


# ------------------------------------------------------------ closed-form checks
@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("kgs", [16, 32])
def test_quantize_k_error_bound_and_layout(oracle, kgs, fp16):
    """Each dequantised value lies within half a quantisation step of the input,
    and permuting the tokens of a block permutes their 2-bit fields."""
    H, D = 3, 32
    K = synth.normal(7, kgs, (kgs, H, D), std=2.0)
    p, s, z = oracle.quantize_k(K, kgs, fp16)
    d = oracle.dequantize_k(p, s, z, 1, H, D, kgs, fp16)
    sf = (s.view(np.float16).astype(np.float32) if fp16 else s)[None]
    zf = (z.view(np.float16).astype(np.float32) if fp16 else z)[None]
    # half-step rounding, plus the binary16 rounding of scale and zero (2^-11 relative each)
    bound = sf * 0.5 + 1e-6 + ((3 * sf + np.abs(zf)) * 2.0 ** -10 if fp16 else 0)
    assert np.all(np.abs(d - K) <= bound)
    perm = np.random.default_rng(0).permutation(kgs)
    p2, s2, z2 = oracle.quantize_k(K[perm], kgs, fp16)
    assert same_bits(s2, s) and same_bits(z2, z)
    f1 = np.stack([(p.reshape(kgs // 16, H, D)[t // 16].view(np.uint32) >> (2 * (t % 16))) & 3 for t in range(kgs)])
    f2 = np.stack([(p2.reshape(kgs // 16, H, D)[t // 16].view(np.uint32) >> (2 * (t % 16))) & 3 for t in range(kgs)])
    assert np.array_equal(f2, f1[perm])


def test_quantize_v_error_bound_and_layout(oracle):
    H, D = 2, 64
    V = synth.normal(8, 0, (16, H, D), std=1.5)
    p, s, z = oracle.quantize_v(V, fp16=False)
    d = oracle.dequantize_v(p, s, z, 16, H, D, False)
    assert np.all(np.abs(d - V) <= s[:, :, None] * 0.5 + 1e-6)
    perm = np.random.default_rng(1).permutation(D)
    p2, s2, z2 = oracle.quantize_v(V[:, :, perm], fp16=False)
    assert same_bits(s2, s) and same_bits(z2, z)

    def fields(pk):
        w = pk.view(np.uint32)
        return np.stack([(w[:, :, c // 16] >> (2 * (c % 16))) & 3 for c in range(D)], axis=-1)

    assert np.array_equal(fields(p2), fields(p)[:, :, perm])


def test_f16_conversion_against_numpy(oracle):
    """RNE float -> half against numpy's IEEE conversion (normals, denormals, overflow)."""
    xs = np.concatenate([synth.normal(9, 0, (4000,), std=1e3), synth.normal(9, 1, (4000,), std=1e-5),
                         np.array([65504.0, 65519.0, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, -0.0, 1e-9], np.float32)])
    import ctypes as C

    f = oracle.lib.orc_f32_to_f16
    f.argtypes = [C.c_float]
    f.restype = C.c_uint16
    got = np.array([f(float(x)) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def _f64_attention(Q, dK, dV, nd, deqK, deqV, ids, Hq, Hkv, D):
    G = Hq // Hkv
    K = np.concatenate([dK, deqK]).astype(np.float64)
    V = np.concatenate([dV, deqV]).astype(np.float64)
    valid = np.concatenate([np.ones(nd, bool), ids != -1])
    out = np.zeros((Hq, D))
    w = np.zeros((Hq, K.shape[0]))
    for h in range(Hq):
        s = K[:, h // G, :] @ Q[h].astype(np.float64) / np.sqrt(D)
        s[~valid] = -np.inf
        e = np.exp(s - s.max())
        w[h] = e / e.sum()
        out[h] = w[h] @ V[:, h // G, :]
    return out, w.mean(axis=0)


def test_fused_attention_float64_brute_force(oracle):
    """Softmax attention over the dequantised tiers, in float64, within 1e-5."""
    Hq, Hkv, D, nd, nb, kgs = 8, 2, 64, 37, 6, 16
    Q = synth.normal(21, 0, (Hq, D))
    dK, dV = synth.normal(21, 1, (nd, Hkv, D)), synth.normal(21, 2, (nd, Hkv, D))
    Kp, Vp = synth.normal(21, 3, (nb * kgs, Hkv, D)), synth.normal(21, 4, (nb * kgs, Hkv, D))
    blocks = [[], [], [], [], [], []]
    for b in range(nb):
        for j, x in enumerate(oracle.quantize_k(Kp[b * kgs:(b + 1) * kgs], kgs, False)):
            blocks[j].append(x)
        for j, x in enumerate(oracle.quantize_v(Vp[b * kgs:(b + 1) * kgs], False)):
            blocks[3 + j].append(x)
    KP, KS, KZ = (np.stack(x) for x in blocks[:3])
    VP, VS, VZ = (np.concatenate(x) for x in blocks[3:])
    ids = np.arange(nb * kgs, dtype=np.int64)
    ids[-5:] = -1
    out, mw = oracle.fused_attention_decode(Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, False)
    deqK = oracle.dequantize_k(KP, KS, KZ, nb, Hkv, D, kgs, False)
    deqV = oracle.dequantize_v(VP, VS, VZ, nb * kgs, Hkv, D, False)
    ref_out, ref_mw = _f64_attention(Q, dK, dV, nd, deqK, deqV, ids, Hq, Hkv, D)
    assert np.abs(out - ref_out).max() <= 1e-5 * np.abs(ref_out).max()
    assert np.abs(mw - ref_mw).max() <= 1e-6
    assert abs(float(mw.sum(dtype=np.float64)) - 1.0) < 1e-5
    assert np.all(mw[nd + nb * kgs - 5:] == 0)


# ---------------------------------------------------------------- engine digests
@pytest.mark.parametrize("run", sorted(engine_runs.RUNS))
def test_engine_matches_reference_digests(oracle, golden, run):
    """The oracle engine reproduces the compiled reference engine's full state
    (counters, tier buffers, packed store, global scores) bit for bit at every
    checkpoint, in full-step mode (reference attention included) and in
    score-injected tier-maintenance mode."""
    cfg = engine_runs.RUNS[run]
    want = golden["engine"][run]
    e = oracle.engine(*engine_runs.engine_args(cfg))
    if cfg["prefill"]:
        e.prefill(*engine_runs.prefill_inputs(cfg))
    for s in range(cfg["steps"]):
        Q, K, V = engine_runs.step_inputs(cfg, s)
        if cfg["mode"] == "step":
            e.step(Q, K, V)
        else:
            e.ingest(K, V)
            e.feedback(engine_runs.inject_weights(cfg, s, e.visible()))
        if engine_runs.is_checkpoint(cfg, s):
            st = e.state()
            assert synth.state_digest(st["counters"], st) == want["digests"][str(s)], (run, s)
    assert e.counters() == want["final_counters"]


# ------------------------------------------------- float64 exact attention helper
def _tiny_case(oracle, seed):
    Hq, Hkv, D, nd, nb, kgs = 4, 2, 16, 3, 1, 16
    Q = synth.normal(seed, 0, (Hq, D))
    dK, dV = synth.normal(seed, 1, (nd, Hkv, D)), synth.normal(seed, 2, (nd, Hkv, D))
    KP, KS, KZ = (x[None] for x in oracle.quantize_k(synth.normal(seed, 3, (kgs, Hkv, D)), kgs, False))
    VP, VS, VZ = oracle.quantize_v(synth.normal(seed, 4, (kgs, Hkv, D)), False)
    ids = np.arange(kgs, dtype=np.int64) + nd
    ids[[2, 9]] = -1
    return (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, False)


def test_exact_attention_helper_brute_force(oracle):
    """oracle.exact.exact_attention (the float64 bar of the GPU tests) against
    scalar Python loops over the same dequantised values, on a tiny layer with
    masked slots: equal to 1e-12."""
    import math

    from oracle.exact import exact_attention

    args = _tiny_case(oracle, 41)
    Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, _ = args
    out, mw = exact_attention(oracle, *args)
    K = np.concatenate([dK, oracle.dequantize_k(KP, KS, KZ, nb, Hkv, D, kgs, False)])
    V = np.concatenate([dV, oracle.dequantize_v(VP, VS, VZ, nb * kgs, Hkv, D, False)])
    keep = [True] * nd + [bool(i != -1) for i in ids]
    n = len(keep)
    want_mw = [0.0] * n
    for h in range(Hq):
        kv = h // (Hq // Hkv)
        s = [sum(float(Q[h, c]) * float(K[t, kv, c]) for c in range(D)) / math.sqrt(D) if keep[t] else None
             for t in range(n)]
        m = max(x for x in s if x is not None)
        e = [math.exp(x - m) if x is not None else 0.0 for x in s]
        tot = sum(e)
        for c in range(D):
            o = sum(e[t] / tot * float(V[t, kv, c]) for t in range(n))
            assert abs(out[h, c] - o) <= 1e-12 * max(1.0, abs(o))
        for t in range(n):
            want_mw[t] += e[t] / tot / Hq
    assert np.allclose(mw, want_mw, rtol=0, atol=1e-14)
    assert mw[nd + 2] == 0.0 and mw[nd + 9] == 0.0


def test_engine_exact_attention_matches_oracle_engine(oracle):
    """oracle.exact.engine_exact_attention assembles the engine's visible tokens in the
    engine's order (sinks, heavy hitters, recent window oldest first, packed
    blocks): its result agrees with the oracle engine's own attention to float32
    accuracy after a run with a wrapped ring, heavy hitters and flushed blocks."""
    from oracle.exact import elementwise_ratio, engine_exact_attention

    cfg = engine_runs.RUNS["step_gqa_d128_fp16"]
    e = oracle.engine(*engine_runs.engine_args(cfg))
    e.prefill(*engine_runs.prefill_inputs(cfg))
    for s in range(150):
        Q, K, V = engine_runs.step_inputs(cfg, s)
        e.step(Q, K, V)
    Q, K, V = engine_runs.step_inputs(cfg, 150)
    e.ingest(K, V)
    c = e.counters()
    assert c["hh_count"] > 0 and c["pbs_blocks_used"] > 0 and c["rw_head_index"] > 0
    xo, xmw = engine_exact_attention(oracle, e.state(), Q, cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["kgs"], cfg["fp16"])
    ro, rmw = e.attend(Q)
    assert elementwise_ratio(ro, xo.reshape(-1), rtol=1e-5, atol_frac=1e-6) <= 1.0
    assert np.abs(rmw - xmw).max() <= 1e-6 * xmw.max()


def test_reconstruct_order_and_rows_from_the_inputs(oracle):
    """oracle.exact.reconstruct_full_cache / reconstruct_order (the order of the
    reference's reconstruct_full_cache, src/tri_tier/cache.py:326-372) pinned by the
    inputs themselves, after a run with a wrapped ring, heavy hitters and flushed
    blocks: the ids are every processed token except the waiting room's, strictly
    increasing; each FP32-tier row is the K/V row that token was given, bit for bit;
    each packed row is within half a quantisation step of it; and the per-head
    weights in that order are the engine-order weights permuted (rows sum to 1)."""
    from oracle.exact import engine_exact_attention, engine_visible_ids, reconstruct_full_cache, reconstruct_order

    cfg = engine_runs.RUNS["step_gqa_d128_fp16"]
    Hq, Hkv, D, kgs, fp16 = cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["kgs"], cfg["fp16"]
    e = oracle.engine(*engine_runs.engine_args(cfg))
    K0, V0 = engine_runs.prefill_inputs(cfg)
    e.prefill(K0, V0)
    Ks, Vs = [np.asarray(K0).reshape(-1, Hkv, D)], [np.asarray(V0).reshape(-1, Hkv, D)]
    for s in range(150):
        Q, K, V = engine_runs.step_inputs(cfg, s)
        e.step(Q, K, V)
        Ks.append(np.asarray(K).reshape(1, Hkv, D))
        Vs.append(np.asarray(V).reshape(1, Hkv, D))
    Kin, Vin = np.concatenate(Ks), np.concatenate(Vs)
    st = e.state()
    c = st["counters"]
    assert c["hh_count"] > 0 and c["pbs_blocks_used"] > 0 and c["rw_head_index"] > 0 and c["wr_count"] > 0
    K, V, ids = reconstruct_full_cache(oracle, st, Hkv, D, fp16)
    wr = set(np.asarray(st["WR_token_ids"]).reshape(-1)[: c["wr_count"]].tolist())
    total = c["total_processed_tokens"]
    assert total == Kin.shape[0]
    assert ids.tolist() == [t for t in range(total) if t not in wr]
    hh = set(np.asarray(st["HH_token_ids"]).reshape(-1)[: c["hh_count"]].tolist())
    nb = c["pbs_blocks_used"]
    slot = {t: j for j, t in enumerate(np.asarray(st["PBS_token_ids"]).reshape(-1)[: nb * kgs].tolist())}
    meta = (lambda a: np.asarray(a).view(np.float16).astype(np.float32)) if fp16 else np.asarray  # noqa: E731
    KS, KZ = meta(st["PBS_K_Scales"]).reshape(-1, Hkv, D), meta(st["PBS_K_Zeroes"]).reshape(-1, Hkv, D)
    VS, VZ = meta(st["PBS_V_Scales"]).reshape(-1, Hkv, 1), meta(st["PBS_V_Zeroes"]).reshape(-1, Hkv, 1)

    def half_step(sc, z):
        # codes are chosen with the float32 scale/min; f16 metadata rounds both
        return 0.5 * sc + 2.0 ** -10 * (3 * sc + np.abs(z)) + 1e-6

    n_packed = 0
    for i, t in enumerate(ids.tolist()):
        if t in slot:
            assert t not in hh
            j = slot[t]
            assert np.all(np.abs(K[i] - Kin[t]) <= half_step(KS[j // kgs], KZ[j // kgs])), t
            assert np.all(np.abs(V[i] - Vin[t]) <= half_step(VS[j], VZ[j])), t
            n_packed += 1
        else:
            assert np.array_equal(K[i], Kin[t]) and np.array_equal(V[i], Vin[t]), t
    assert n_packed == nb * kgs
    Q, _, _ = engine_runs.step_inputs(cfg, 150)
    _, _, W = engine_exact_attention(oracle, st, Q, Hq, Hkv, D, kgs, fp16, per_head=True)
    perm = reconstruct_order(st)
    assert np.array_equal(engine_visible_ids(st)[perm], ids)
    assert np.allclose(W[:, perm].sum(axis=1), 1.0, atol=1e-12)


@pytest.mark.parametrize("fp16,kgs,Hq,Hkv,D,msl,R,hr", [(True, 16, 4, 2, 64, 256, 16, 0.1),
                                                       (False, 16, 32, 8, 128, 4096, 256, 0.05),
                                                       (True, 32, 28, 4, 128, 2000, 64, 0.02),
                                                       (False, 32, 8, 8, 32, 512, 32, 0.3)])
def test_engine_buffer_bytes_matches_reference(oracle, reference, fp16, kgs, Hq, Hkv, D, msl, R, hr):
    """The oracle's get_buffer_bytes accounting (cache_engine.cpp:543-568) equals the
    compiled reference's, before any token, after a prefill that grows the packed
    store past its first allocation, and after decode steps."""
    o = oracle.engine(Hq, Hkv, D, msl, 4, R, hr, 0.999, 32, kgs, fp16)
    r = reference.engine(Hq, Hkv, D, msl, 4, R, hr, 0.999, 32, kgs, fp16)
    assert o.buffer_bytes() == r.buffer_bytes()
    n = min(msl - 8, 64 * kgs + 3 * R)
    K, V = synth.normal(61, 0, (n, Hkv, D)), synth.normal(61, 1, (n, Hkv, D))
    o.prefill(K, V)
    r.prefill(K, V)
    assert o.counters()["pbs_allocated_blocks"] == r.counters()["pbs_allocated_blocks"] > 0
    assert o.buffer_bytes() == r.buffer_bytes()
    for s in range(5):
        q, k, v = synth.normal(62, s, (Hq * D,)), synth.normal(63, s, (Hkv * D,)), synth.normal(64, s, (Hkv * D,))
        o.step(q, k, v)
        r.step(q, k, v)
    assert o.buffer_bytes() == r.buffer_bytes()


# ------------------------------------------- heavy-hitter argmin with tied scores
@pytest.mark.parametrize("run,fp16", [("small", False), ("small", True), ("large", False)])
def test_engine_route_ties_match_reference(oracle, reference, run, fp16):
    """Routing with tied heavy-hitter scores (engine_runs.TIE_RUNS): the oracle
    engine's state equals the compiled reference engine's, bit for bit, through
    the fill of the heavy-hitter tier and the replacements of its first minimal
    slot, for a 60-slot tier and an 8750-slot one."""
    cfg = engine_runs.TIE_RUNS[run]
    o, r = oracle.engine(*cfg["args"], fp16), reference.engine(*cfg["args"], fp16)
    replaced = 0
    prev = None
    for s in range(cfg["steps"]):
        k, v = engine_runs.tie_kv(s)
        o.ingest(k, v)
        r.ingest(k, v)
        c = o.counters()
        if c["hh_count"] == c["max_hh"] and (s % 10 == 0 or run == "small"):
            ids = o.buffer("HH_token_ids")[: c["hh_count"]]
            if prev is not None and (prev != ids).any():
                replaced += 1
            prev = ids
        w = engine_runs.tie_weights(run, c, o.visible(), s)
        o.feedback(w)
        r.feedback(w)
        if s in cfg["checkpoints"]:
            so, sr = o.state(), r.state()
            assert so["counters"] == sr["counters"], s
            for name in sr:
                if name != "counters":
                    assert np.array_equal(so[name].view(np.uint8), sr[name].view(np.uint8)), (s, name)
    c = o.counters()
    hs = o.buffer("HH_scores")[: c["hh_count"]]
    assert c["hh_count"] == c["max_hh"] and replaced >= 3 and (hs == hs.min()).sum() > 1, (replaced, c["hh_count"])
