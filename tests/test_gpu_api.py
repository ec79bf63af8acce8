"""Python API and HF patch on the GPU, mirroring the reference's own tests:
tests/test_cache_init.py (TriTierCache construction), tests/test_wiring_verification.py
(k_group_size / metadata-dtype wiring through _C), tests/test_patch_llama.py and
tests/test_multi_model_patch.py (the attention patch on tiny offline configs).
Here every module and tensor lives on the ROCm device and the engine runs on it.

TriTierCache.prefill/step and the patched attention of LLaMA, Mistral, Qwen2
and Qwen3 layers (head_dim 128, GQA) also run in score-injected lockstep with
the oracle engine: the post-RoPE Q/K/V each call hands the engine are fed to
the oracle, the GPU's mean attention weights are its score feedback, the tier
state must stay bit-exact and the context vector before o_proj must match the
oracle's. The Q/K/V the patch hands the engine are checked against those the
family's own unpatched forward computes for the same hidden states.
"""
import math
import sys

import numpy as np
import pytest
import torch

from gpu_helpers import Lockstep, attention_ok, dev, host, same_bits
from oracle import synth

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU test on a machine without a GPU"


# ---------------------------------------------------------------------------
# TriTierCache construction (reference tests/test_cache_init.py)
# ---------------------------------------------------------------------------
MAX_SEQ_LEN, HEAD_DIM, NUM_HEADS, R_SIZE, H_RATIO = 128, 16, 4, 32, 0.05


@pytest.fixture
def cache():
    from tritiercache_amd.cache import TriTierCache

    return TriTierCache(max_seq_len=MAX_SEQ_LEN, head_dim=HEAD_DIM, num_heads=NUM_HEADS, R_size=R_SIZE,
                        H_ratio=H_RATIO)


def test_cache_constructs_on_the_engine(cache):
    assert cache._engine is not None
    assert cache.RW_K_Buffer.device.type == "cuda"


def test_cache_sizing(cache):
    from tritiercache_amd.constants import CHUNK_SIZE

    assert cache.R_size + cache.max_heavy_hitters + cache.max_background_tokens == MAX_SEQ_LEN
    assert cache.num_blocks == math.ceil(cache.max_background_tokens / CHUNK_SIZE)
    assert cache.quant_head_dim == math.ceil(HEAD_DIM / 16)


def test_cache_tier_buffers(cache):
    from tritiercache_amd.constants import CHUNK_SIZE

    assert cache.RW_K_Buffer.shape == (R_SIZE, NUM_HEADS, HEAD_DIM)
    assert cache.RW_V_Buffer.shape == (R_SIZE, NUM_HEADS, HEAD_DIM)
    assert cache.RW_K_Buffer.dtype == torch.float32
    assert cache.RW_count == 0 and cache.RW_head_index == 0
    n = cache.max_heavy_hitters
    assert cache.HH_K_Buffer.shape == (n, NUM_HEADS, HEAD_DIM)
    assert cache.HH_token_ids.shape == (n,) and cache.HH_token_ids.dtype == torch.int64
    assert cache.HH_scores.shape == (n,) and cache.HH_scores.dtype == torch.float32
    assert torch.all(cache.HH_token_ids == -1)
    assert cache.HH_count == 0
    assert cache.WR_K_Buffer.shape == (CHUNK_SIZE, NUM_HEADS, HEAD_DIM)
    assert cache.WR_token_ids.shape == (CHUNK_SIZE,)
    assert torch.all(cache.WR_token_ids == -1)
    assert cache.WR_count == 0
    assert cache.Global_Attn_Scr.shape == (MAX_SEQ_LEN,)
    assert torch.all(cache.Global_Attn_Scr == 0.0)
    assert cache.current_threshold == 0.0
    assert cache.PBS_count == 0


def test_cache_counters_are_read_only_with_the_engine(cache):
    with pytest.raises(AttributeError):
        cache.Total_Processed_Tokens = 3


# ---------------------------------------------------------------------------
# _C wiring (reference tests/test_wiring_verification.py)
# ---------------------------------------------------------------------------
def test_k_group_size_wiring():
    from tritiercache_amd import _C

    H, D, T = 4, 64, 32
    rng = np.random.default_rng(42)
    K = np.zeros((T, H, D), np.float32)
    K[:16] = rng.uniform(-1.0, 1.0, (16, H, D))
    K[16:] = rng.uniform(5.0, 10.0, (16, H, D))
    p16 = np.zeros((2, H, D), np.int32)
    s16 = np.zeros((2, H, D), np.float32)
    z16 = np.zeros((2, H, D), np.float32)
    _C.quantize_k_block(K[:16], p16[0], s16[0], z16[0], H, D, 16, "fp32")
    _C.quantize_k_block(K[16:], p16[1], s16[1], z16[1], H, D, 16, "fp32")
    d16 = np.zeros((T, H, D), np.float32)
    _C.dequantize_k(p16, s16, z16, d16, 2, H, D, 16, "fp32")
    p32 = np.zeros((2, H, D), np.int32)
    s32 = np.zeros((1, H, D), np.float32)
    z32 = np.zeros((1, H, D), np.float32)
    _C.quantize_k_block(K, p32, s32, z32, H, D, 32, "fp32")
    d32 = np.zeros((T, H, D), np.float32)
    _C.dequantize_k(p32, s32, z32, d32, 1, H, D, 32, "fp32")
    assert not np.array_equal(p16, p32)
    assert np.max(np.abs(d16 - d32)) > 0.1
    # each block size reconstructs its own tokens within half a step
    assert np.all(np.abs(d16[:16] - K[:16]) <= s16[0] * 0.5 + 1e-6)
    assert np.all(np.abs(d32 - K) <= s32 * 0.5 + 1e-5)


def test_pbs_metadata_dtype_wiring():
    from tritiercache_amd import _C

    H, D, T = 4, 64, 16
    K = (np.random.default_rng(42).standard_normal((T, H, D)) * 2.5 + 1.2345).astype(np.float32)
    out = {}
    for meta, mdt in (("fp32", np.float32), ("fp16", np.uint16)):
        p = np.zeros((1, H, D), np.int32)
        s = np.zeros((1, H, D), mdt)
        z = np.zeros((1, H, D), mdt)
        _C.quantize_k_block(K, p, s, z, H, D, 16, meta)
        d = np.zeros((T, H, D), np.float32)
        _C.dequantize_k(p, s, z, d, 1, H, D, 16, meta)
        out[meta] = (s, d)
    assert out["fp16"][0].itemsize == 2 and out["fp32"][0].itemsize == 4
    diff = np.max(np.abs(out["fp32"][1] - out["fp16"][1]))
    assert 0 < diff < 0.05


def _engines():
    from tritiercache_amd import _C

    args = (4, 2, 64, 256, 4, 16, 0.1, 0.999, 16)
    return {"16/fp16": _C.TriTierCacheEngine(*args, 16, "fp16"), "16/fp32": _C.TriTierCacheEngine(*args, 16, "fp32"),
            "32/fp16": _C.TriTierCacheEngine(*args, 32, "fp16")}


def test_engine_properties_and_memory_sensitivity():
    eng = _engines()
    assert eng["16/fp16"].k_group_size == 16 and eng["16/fp16"].pbs_metadata_dtype == "fp16"
    assert eng["16/fp16"].use_fp16_meta is True
    assert eng["16/fp32"].use_fp16_meta is False and eng["16/fp32"].pbs_metadata_dtype == "fp32"
    assert eng["32/fp16"].k_group_size == 32
    rng = np.random.default_rng(123)
    Kp = rng.standard_normal((96, 2, 64)).astype(np.float32)
    Vp = rng.standard_normal((96, 2, 64)).astype(np.float32)
    for e in eng.values():
        e.prefill(Kp, Vp, 96)
        assert e.pbs_count > 0
    assert eng["16/fp16"].get_buffer_bytes() < eng["16/fp32"].get_buffer_bytes()


def test_engine_attention_step_differs_across_configurations():
    eng = _engines()
    rng = np.random.default_rng(999)
    Kp = rng.standard_normal((96, 2, 64)).astype(np.float32)
    Vp = rng.standard_normal((96, 2, 64)).astype(np.float32)
    Q = rng.standard_normal(4 * 64).astype(np.float32)
    Kn = rng.standard_normal(2 * 64).astype(np.float32)
    Vn = rng.standard_normal(2 * 64).astype(np.float32)
    outs = {}
    for k, e in eng.items():
        e.prefill(Kp, Vp, 96)
        o = np.zeros(4 * 64, np.float32)
        e.step(Q, Kn, Vn, o)
        assert np.all(np.isfinite(o)) and np.any(o != 0.0)
        outs[k] = o
    assert np.max(np.abs(outs["16/fp16"] - outs["32/fp16"])) > 0
    assert np.max(np.abs(outs["16/fp16"] - outs["16/fp32"])) > 0


# ---------------------------------------------------------------------------
# Engine decode against float32 attention over the reconstructed tiers
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("Hq,Hkv,D,kgs,meta", [(8, 2, 128, 16, "fp16"), (8, 8, 64, 32, "fp32"),
                                               (12, 4, 128, 32, "fp32")])
def test_decode_matches_attention_over_reconstructed_cache(Hq, Hkv, D, kgs, meta):
    from tritiercache_amd.cache import TriTierCache

    torch.manual_seed(Hq * 1000 + D + kgs)
    c = TriTierCache(max_seq_len=1024, head_dim=D, num_heads=Hkv, R_size=64, H_ratio=0.05, num_q_heads=Hq,
                     k_group_size=kgs, pbs_metadata_dtype=meta)
    c.prefill(torch.randn(300, Hkv, D, device=DEV), torch.randn(300, Hkv, D, device=DEV))
    out = torch.empty(Hq * D, device=DEV)
    for step in range(40):  # past ring overflow, routing and at least one waiting-room flush
        Q = torch.randn(Hq * D, device=DEV)
        Kn, Vn = torch.randn(Hkv * D, device=DEV), torch.randn(Hkv * D, device=DEV)
        c.step(Q, Kn, Vn, out)
        Kf, Vf, ids = c.reconstruct_full_cache()
        assert Kf.shape[0] == c.Total_Processed_Tokens - c.WR_count
        rep = Hq // Hkv
        Kh = Kf.permute(1, 0, 2).repeat_interleave(rep, dim=0)  # [Hq, N, D]
        Vh = Vf.permute(1, 0, 2).repeat_interleave(rep, dim=0)
        q = Q.view(Hq, 1, D)
        w = torch.softmax(torch.matmul(q, Kh.transpose(1, 2).contiguous()) / math.sqrt(D), dim=-1)
        ref = torch.matmul(w, Vh).reshape(-1)
        err = (out - ref).abs().max() / ref.abs().max()
        assert err <= 1e-4, (step, float(err))
    assert c.PBS_count > 300 - 4 - 64 - c.max_heavy_hitters - kgs


# ---------------------------------------------------------------------------
# TriTierCache.prefill / step in lockstep with the oracle engine
# ---------------------------------------------------------------------------
def _lockstep_for(oracle, cache):
    from tritiercache_amd.constants import SINK_SIZE, UPDATE_THRESHOLD

    e = cache._engine
    return Lockstep(oracle, cache.num_q_heads, cache.num_heads, cache.head_dim, cache.max_seq_len, SINK_SIZE,
                    cache.R_size, cache.H_ratio, cache.score_decay, UPDATE_THRESHOLD, e.k_group_size,
                    cache.pbs_metadata_dtype == "fp16")


@pytest.mark.parametrize("Hq,Hkv,kgs,meta", [(28, 4, 16, "fp32"), (8, 2, 32, "fp16")])
def test_cache_prefill_and_steps_lockstep_with_oracle(oracle, Hq, Hkv, kgs, meta):
    """600-token prefill, then 320 decode steps through TriTierCache: past the heavy
    hitters filling up (41 slots), demotions into the waiting room and flushes."""
    from tritiercache_amd.cache import TriTierCache

    D, msl, R, hr = 128, 2048, 64, 0.02
    c = TriTierCache(max_seq_len=msl, head_dim=D, num_heads=Hkv, R_size=R, H_ratio=hr, num_q_heads=Hq,
                     k_group_size=kgs, pbs_metadata_dtype=meta)
    ls = _lockstep_for(oracle, c)
    seed = 300 + Hq
    Kp, Vp = synth.normal(seed, 1, (600, Hkv, D)), synth.normal(seed, 2, (600, Hkv, D))
    c.prefill(dev(Kp), dev(Vp))
    ls.prefill(Kp, Vp)
    ls.check_state(c._engine, "prefill")
    blocks0 = c._engine.counters()["pbs_blocks_used"]
    for s in range(320):
        q = synth.normal(seed, 10 + 3 * s, (Hq * D,))
        k, v = synth.normal(seed, 11 + 3 * s, (Hkv * D,)), synth.normal(seed, 12 + 3 * s, (Hkv * D,))
        out = torch.empty(Hq * D, dtype=torch.float32, device=DEV)
        c.step(dev(q), dev(k), dev(v), out)
        r = ls.step(q, k, v, host(out), host(c._engine.get_mean_attn_weights()))
        assert attention_ok(r), (s, r)
        if (s + 1) % 40 == 0:
            ls.check_state(c._engine, s)
    assert c.HH_count == c.max_heavy_hitters
    assert c._engine.counters()["pbs_blocks_used"] >= blocks0 + 2


# ---------------------------------------------------------------------------
# Per-head weights and reconstruct_full_cache in lockstep with the oracle
# (the reference's torch path, src/tri_tier/integration/patch_model.py:33-51,
# returned at :162-169; src/tri_tier/cache.py:326-372)
# ---------------------------------------------------------------------------
def _check_weights_against_oracle(oracle, ls, q, w, ids, Hq, Hkv, D, kgs, fp16, tag):
    """w [Hq, visible] and ids [visible] as step_with_weights returns them, against
    float64 per-head softmax weights over the oracle engine's tiers (the tiers the
    step attended: the score feedback changes no membership), permuted into
    reconstruct order."""
    from oracle.exact import engine_exact_attention, engine_visible_ids, reconstruct_order, weights_rel_err

    st = ls.oe.state()
    _, _, W = engine_exact_attention(oracle, st, q, Hq, Hkv, D, kgs, fp16, per_head=True)
    perm = reconstruct_order(st)
    assert np.array_equal(host(ids), engine_visible_ids(st)[perm]), tag
    got = host(w).astype(np.float64)
    want = W[:, perm]
    assert got.shape == want.shape, (tag, got.shape, want.shape)
    err = weights_rel_err(got, want)
    assert err <= 1e-4, (tag, err)
    assert np.abs(got.sum(axis=1) - 1.0).max() <= 1e-5, tag
    return err


def _check_reconstruct_against_oracle(oracle, ls, cache, fp16, tag):
    from oracle.exact import reconstruct_full_cache

    K, V, ids = cache.reconstruct_full_cache()
    oK, oV, oids = reconstruct_full_cache(oracle, ls.oe.state(), cache.num_heads, cache.head_dim, fp16)
    assert np.array_equal(host(ids), oids), tag
    assert same_bits(host(K), oK) and same_bits(host(V), oV), tag
    # every visible token in id order, and nothing but the waiting room left out
    assert np.all(np.diff(oids) > 0), tag
    assert oids.size == cache.Total_Processed_Tokens - cache.WR_count, tag


@pytest.mark.parametrize("Hq,Hkv,D,kgs,meta", [(8, 2, 128, 16, "fp16"), (12, 4, 64, 32, "fp32"),
                                               (28, 4, 128, 16, "fp32")])
def test_step_with_weights_and_reconstruct_lockstep_with_oracle(oracle, Hq, Hkv, D, kgs, meta):
    """A 400-token prefill and 200 decode steps through TriTierCache in score-injected
    lockstep with the oracle engine (heavy hitters filling and demoting, waiting-room
    flushes): every fifth step through step_with_weights, whose per-head weights
    (reconstruct order) must equal float64 softmax weights over the oracle's tiers
    within 1e-4 relative for every weight >= 1e-8, with the same token ids; every
    40 steps reconstruct_full_cache() must equal the oracle's dequantised tiers bit
    for bit."""
    from tritiercache_amd.cache import TriTierCache

    fp16 = meta == "fp16"
    c = TriTierCache(max_seq_len=1024, head_dim=D, num_heads=Hkv, R_size=64, H_ratio=0.05, num_q_heads=Hq,
                     k_group_size=kgs, pbs_metadata_dtype=meta)
    ls = _lockstep_for(oracle, c)
    seed = 700 + Hq + D
    Kp, Vp = synth.normal(seed, 1, (400, Hkv, D)), synth.normal(seed, 2, (400, Hkv, D))
    c.prefill(dev(Kp), dev(Vp))
    ls.prefill(Kp, Vp)
    _check_reconstruct_against_oracle(oracle, ls, c, fp16, "prefill")
    worst, checked = 0.0, 0
    for s in range(200):
        q = synth.normal(seed, 10 + 3 * s, (Hq * D,))
        k, v = synth.normal(seed, 11 + 3 * s, (Hkv * D,)), synth.normal(seed, 12 + 3 * s, (Hkv * D,))
        out = torch.empty(Hq * D, dtype=torch.float32, device=DEV)
        with_w = s % 5 == 0 or s == 199
        if with_w:
            w, ids = c.step_with_weights(dev(q), dev(k), dev(v), out)
        else:
            c.step(dev(q), dev(k), dev(v), out)
        r = ls.step(q, k, v, host(out), host(c._engine.get_mean_attn_weights()))
        assert attention_ok(r), (s, r)
        if with_w:
            worst = max(worst, _check_weights_against_oracle(oracle, ls, q, w, ids, Hq, Hkv, D, kgs, fp16, s))
            checked += 1
        if (s + 1) % 40 == 0:
            _check_reconstruct_against_oracle(oracle, ls, c, fp16, s)
            ls.check_state(c._engine, s)
    assert checked == 41
    assert c.HH_count == c.max_heavy_hitters and c.PBS_count > 0
    print(f"per-head weights worst rel err {worst:.3g} over {checked} steps", flush=True)


@pytest.mark.parametrize("kgs,meta", [(16, "fp16"), (32, "fp32")])
def test_live_cache_bytes_equal_the_engine_buffers_in_use(kgs, meta):
    """accounting.live_cache_bytes prices the tiers from the engine's counters; each
    tier's figure equals the bytes of the device buffers that tier occupies (sinks,
    ring, heavy-hitter rows + ids + scores, packed words, scales/zeros + ids, the
    waiting room's rows), and the canonical measure_cache_bytes of the same cache
    object takes its shapes from it."""
    from tritiercache_amd.accounting import live_cache_bytes, measure_cache_bytes
    from tritiercache_amd.cache import TriTierCache

    Hq, Hkv, D = 8, 2, 128
    c = TriTierCache(max_seq_len=2048, head_dim=D, num_heads=Hkv, R_size=64, H_ratio=0.05, num_q_heads=Hq,
                     k_group_size=kgs, pbs_metadata_dtype=meta)
    c.prefill(torch.randn(500, Hkv, D, device=DEV), torch.randn(500, Hkv, D, device=DEV))
    out = torch.empty(Hq * D, device=DEV)
    for _ in range(150):
        c.step(torch.randn(Hq * D, device=DEV), torch.randn(Hkv * D, device=DEV), torch.randn(Hkv * D, device=DEV),
               out)
    cnt = c._engine.counters()
    s, rw, hh, wr, nb, npk = (cnt[k] for k in ("s_count", "rw_count", "hh_count", "wr_count", "pbs_blocks_used",
                                               "pbs_count"))
    assert hh > 0 and nb > 0 and wr > 0 and npk == nb * kgs
    nbytes = lambda t: t.numel() * t.element_size()  # noqa: E731
    r = live_cache_bytes(c, num_layers=3)
    assert r["sink_bytes"] == 3 * (nbytes(c.S_K_Buffer[:s]) + nbytes(c.S_V_Buffer[:s]))
    assert r["rw_bytes"] == 3 * (nbytes(c.RW_K_Buffer[:rw]) + nbytes(c.RW_V_Buffer[:rw]))
    assert r["hh_bytes"] == 3 * (nbytes(c.HH_K_Buffer[:hh]) + nbytes(c.HH_V_Buffer[:hh]) +
                                 nbytes(c.HH_token_ids[:hh]) + nbytes(c.HH_scores[:hh]))
    assert r["pbs_payload_bytes"] == 3 * (nbytes(c.PBS_K_Packed[:nb]) + nbytes(c.PBS_V_Packed[:npk]))
    assert r["pbs_metadata_bytes"] == 3 * (nbytes(c.PBS_K_Scales[:nb]) + nbytes(c.PBS_K_Zeroes[:nb]) +
                                           nbytes(c.PBS_V_Scales[:npk]) + nbytes(c.PBS_V_Zeroes[:npk]) +
                                           nbytes(c.PBS_token_ids[:npk]))
    assert r["wr_bytes"] == 3 * (nbytes(c.WR_K_Buffer[:wr]) + nbytes(c.WR_V_Buffer[:wr]))
    assert r["actual_sinks"] + r["actual_rw"] + r["actual_hh"] + r["actual_pbs"] + r["actual_wr"] == 650
    canon = measure_cache_bytes(cache_obj=c, num_layers=3, k_group_size=kgs, pbs_metadata_dtype=meta)
    assert (canon["num_kv_heads"], canon["head_dim"], canon["total_tokens"]) == (Hkv, D, 650)


def test_step_with_weights_rejects_small_capacity_before_the_step():
    """A head-weights capacity the step could exceed is rejected (IndexError in
    Python) before anything is enqueued: the engine's state is unchanged. A capacity
    of the visible count plus one block is always accepted."""
    import ctypes as C

    from gpu_helpers import gpu_engine_state
    from tritiercache_amd import _C, _lib

    Hq, Hkv, D = 8, 2, 64
    eng = _C.TriTierCacheEngine(Hq, Hkv, D, 512, 4, 16, 0.1, 0.999, 32, 16, "fp16")
    eng.prefill(torch.randn(100, Hkv, D, device=DEV), torch.randn(100, Hkv, D, device=DEV), 100)
    for _ in range(5):
        eng.step(torch.randn(Hq * D, device=DEV), torch.randn(Hkv * D, device=DEV),
                 torch.randn(Hkv * D, device=DEV), torch.empty(Hq * D, device=DEV))
    before = gpu_engine_state(eng)
    vis = eng.visible()
    q, k, v = (torch.randn(n, device=DEV) for n in (Hq * D, Hkv * D, Hkv * D))
    out = torch.full((Hq * D,), 7.0, device=DEV)
    w = torch.zeros((Hq, vis + 16), device=DEV)
    got = C.c_int(-1)
    for cap in (1, vis):  # below every bound of the step's visible count
        rc = _lib.load().tt_engine_step_weights(eng._h, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                                w.data_ptr(), cap, C.byref(got), None)
        assert rc == _lib.TT_ERR_OUT_OF_RANGE, rc
        assert "capacity" in _lib.last_error()
    torch.cuda.synchronize()
    assert got.value == -1 and torch.all(out == 7.0) and torch.all(w == 0)
    after = gpu_engine_state(eng)
    assert after["counters"] == before["counters"]
    for name in before:
        if name != "counters":
            assert same_bits(after[name], before[name]), name
    # the bound itself is accepted
    rc = _lib.load().tt_engine_step_weights(eng._h, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                            w.data_ptr(), vis + 16, C.byref(got), None)
    assert rc == _lib.TT_OK and 0 < got.value <= vis + 16
    torch.cuda.synchronize()
    assert torch.allclose(w[:, : got.value].sum(dim=1), torch.ones(Hq, device=DEV), atol=1e-5)


# ---------------------------------------------------------------------------
# HF patch (reference tests/test_patch_llama.py, tests/test_multi_model_patch.py)
# ---------------------------------------------------------------------------
transformers = pytest.importorskip("transformers")


@pytest.fixture
def patched():
    from tritiercache_amd.integration import patch_model

    patch_model.apply_patch()
    yield patch_model
    patch_model.remove_patch()


def _llama_attention(num_q_heads=4, num_kv_heads=4, hidden_size=64, head_dim=16):
    from transformers.models.llama.configuration_llama import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaAttention, LlamaRotaryEmbedding

    cfg = LlamaConfig(hidden_size=hidden_size, num_attention_heads=num_q_heads, num_key_value_heads=num_kv_heads,
                      head_dim=head_dim, max_position_embeddings=4096, attention_bias=False)
    return LlamaAttention(cfg, layer_idx=0).to(DEV), LlamaRotaryEmbedding(config=cfg).to(DEV), cfg


def _pos(rotary, h, positions):
    return rotary(h, torch.tensor([positions], device=DEV))


def test_patch_replaces_and_restores_forwards(patched):
    from transformers.models.llama.modeling_llama import LlamaAttention
    from transformers.models.mistral.modeling_mistral import MistralAttention
    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    assert patched.is_patched()
    for cls in (LlamaAttention, MistralAttention, Qwen2Attention):
        assert cls.forward == patched.patched_forward
    patched.remove_patch()
    assert not patched.is_patched()
    for cls in (LlamaAttention, MistralAttention, Qwen2Attention):
        assert cls.forward != patched.patched_forward
    patched.apply_patch()


def test_batch_size_above_one_is_rejected(patched):
    layer, rot, cfg = _llama_attention()
    h = torch.randn(2, 1, cfg.hidden_size, device=DEV)
    cos, sin = rot(h, torch.tensor([[0], [0]], device=DEV))
    with pytest.raises(AssertionError, match="TriTierCache only supports batch_size=1"):
        layer(h, position_embeddings=(cos, sin))


def test_prefill_then_decode_creates_engine_cache(patched):
    from tritiercache_amd.cache import TriTierCache

    layer, rot, cfg = _llama_attention(num_q_heads=4, num_kv_heads=2)
    assert not hasattr(layer, "tri_tier_cache")
    h = torch.randn(1, 4, cfg.hidden_size, device=DEV)
    out, w = layer(h, position_embeddings=_pos(rot, h, [0, 1, 2, 3]))
    assert out.shape == (1, 4, cfg.hidden_size) and not torch.isnan(out).any()
    c = layer.tri_tier_cache
    assert isinstance(c, TriTierCache) and c._engine is not None
    assert c.num_heads == cfg.num_key_value_heads and c.head_dim == 16 and c.R_size == patched.R_SIZE
    assert c.Total_Processed_Tokens == 4
    h1 = torch.randn(1, 1, cfg.hidden_size, device=DEV)
    out, w = layer(h1, position_embeddings=_pos(rot, h1, [4]))
    assert out.shape == (1, 1, cfg.hidden_size) and out.device.type == "cuda" and w is None
    assert c.Total_Processed_Tokens == 5


@pytest.mark.parametrize("nq,nkv,hid,hd", [(4, 4, 64, 16), (8, 2, 128, 16)])
def test_decode_with_attention_weights(patched, nq, nkv, hid, hd):
    layer, rot, cfg = _llama_attention(nq, nkv, hid, hd)
    h = torch.randn(1, 1, hid, device=DEV)
    out, w = layer(h, position_embeddings=_pos(rot, h, [0]))
    assert out.shape == (1, 1, hid) and w is None
    h = torch.randn(1, 1, hid, device=DEV)
    out, w = layer(h, position_embeddings=_pos(rot, h, [1]), output_attentions=True)
    assert out.shape == (1, 1, hid) and not torch.isnan(out).any()
    assert w.shape == (1, nq, 1, 2)
    assert torch.allclose(w.float().sum(dim=-1), torch.ones(1, nq, 1, device=DEV), atol=1e-5)


def test_multi_step_decode_across_eviction_and_quantization(patched):
    from tritiercache_amd.constants import CHUNK_SIZE, SINK_SIZE

    layer, rot, cfg = _llama_attention(4, 4, 64, 16)
    steps = SINK_SIZE + patched.R_SIZE + CHUNK_SIZE + 10
    for s in range(steps):
        h = torch.randn(1, 1, 64, device=DEV)
        out, w = layer(h, position_embeddings=_pos(rot, h, [s]), output_attentions=True)
        assert out.shape == (1, 1, 64) and torch.isfinite(out).all()
        c = layer.tri_tier_cache
        assert w.shape == (1, 4, 1, (s + 1) - c.WR_count)
        assert torch.allclose(w.float().sum(dim=-1), torch.ones(1, 4, 1, device=DEV), atol=1e-4)
    c = layer.tri_tier_cache
    assert c.Total_Processed_Tokens == steps and c.S_count == SINK_SIZE and c.RW_count == patched.R_SIZE
    assert c.PBS_count >= CHUNK_SIZE or c.HH_count > 0


def test_end_to_end_causal_lm_generate(patched):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=100, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=256,
                      pad_token_id=0, bos_token_id=1, eos_token_id=2)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(DEV).eval()
    with torch.no_grad():
        out = model.generate(torch.tensor([[1]], device=DEV), max_new_tokens=15, use_cache=True, eos_token_id=None,
                             do_sample=False)
    assert out.shape == (1, 16)
    c0 = model.model.layers[0].self_attn.tri_tier_cache
    c1 = model.model.layers[1].self_attn.tri_tier_cache
    assert c0 is not c1
    assert c0.Total_Processed_Tokens == 15 and c1.Total_Processed_Tokens == 15
    assert float(c0.Global_Attn_Scr[:15].sum()) > 0
    patched.reset_caches(model)
    assert not hasattr(model.model.layers[0].self_attn, "tri_tier_cache")


def test_causal_lm_logits_match_unpatched_model_while_tiers_are_fp32(patched):
    """A two-layer LLaMA (8 q / 2 KV heads, head_dim 128), teacher-forced over a
    40-token prompt and 200 decode tokens: with sinks + ring = 260 slots nothing is
    evicted or quantised yet, so the engine's attention is exact float32
    attention over every token, and the patched model's next-token logits must
    match the unpatched model's (HF DynamicCache, SDPA) at every position."""
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=512, hidden_size=1024, intermediate_size=2048, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=1024,
                      pad_token_id=0, bos_token_id=1, eos_token_id=2)
    torch.manual_seed(11)
    model = LlamaForCausalLM(cfg).to(DEV).eval()
    n0, n_dec = 40, 200
    assert n0 + n_dec <= 4 + patched.R_SIZE  # every token stays in the FP32 sinks and ring
    ids = torch.randint(3, cfg.vocab_size, (1, n0 + n_dec), device=DEV)

    def run():
        past = DynamicCache()
        logits = [model(input_ids=ids[:, :n0], past_key_values=past, use_cache=True).logits[0, -1]]
        for t in range(n0, n0 + n_dec - 1):
            out = model(input_ids=ids[:, t:t + 1], position_ids=torch.tensor([[t]], device=DEV),
                        past_key_values=past, use_cache=True)
            logits.append(out.logits[0, -1])
        return torch.stack(logits)

    with torch.no_grad():
        patched.remove_patch()
        try:
            want = run()
        finally:
            patched.apply_patch()
        got = run()
    c0 = model.model.layers[0].self_attn.tri_tier_cache
    assert c0.Total_Processed_Tokens == n0 + n_dec - 1 and c0.PBS_count == 0 and c0.HH_count == 0
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)
    assert torch.equal(got.argmax(-1), want.argmax(-1))


@pytest.mark.parametrize("arch", ["mistral", "qwen2", "qwen3"])
def test_other_architectures_prefill_and_decode(patched, arch):
    import transformers as tf

    if arch == "mistral":
        cfg = tf.MistralConfig(hidden_size=256, num_attention_heads=8, num_key_value_heads=4, head_dim=64)
        from transformers.models.mistral.modeling_mistral import MistralAttention as A
        q_len = 32
    elif arch == "qwen2":
        cfg = tf.Qwen2Config(hidden_size=512, num_attention_heads=4, num_key_value_heads=2, head_dim=128)
        from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention as A
        q_len = 20
    else:
        if not hasattr(tf, "Qwen3Config"):
            pytest.skip("Qwen3 not in the installed transformers")
        cfg = tf.Qwen3Config(hidden_size=256, num_attention_heads=4, num_key_value_heads=2, head_dim=64)
        from transformers.models.qwen3.modeling_qwen3 import Qwen3Attention as A
        q_len = 24
    layer = A(cfg, layer_idx=0).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(7)
    h = torch.randn(1, q_len, cfg.hidden_size, device=DEV, generator=g)
    cos = torch.randn(1, q_len, cfg.head_dim, device=DEV, generator=g)
    sin = torch.randn(1, q_len, cfg.head_dim, device=DEV, generator=g)
    out, _ = layer(h, position_embeddings=(cos, sin))
    assert out.shape == (1, q_len, cfg.hidden_size)
    assert layer.tri_tier_cache.head_dim == cfg.head_dim
    assert layer.tri_tier_cache.Total_Processed_Tokens == q_len
    ht = torch.randn(1, 1, cfg.hidden_size, device=DEV, generator=g)
    out, _ = layer(ht, position_embeddings=(torch.randn(1, 1, cfg.head_dim, device=DEV, generator=g),
                                            torch.randn(1, 1, cfg.head_dim, device=DEV, generator=g)))
    assert out.shape == (1, 1, cfg.hidden_size) and torch.isfinite(out).all()
    assert layer.tri_tier_cache.Total_Processed_Tokens == q_len + 1


def _spy_lockstep(oracle, cache, every=50):
    """Wraps the cache's prefill/step so every call the patched layer makes is
    replayed on the oracle engine (same post-RoPE K/V and Q), with the GPU's mean
    weights as score feedback; collects the attention errors of each step."""
    ls = _lockstep_for(oracle, cache)
    log = {"steps": 0, "errors": []}
    prefill, step = cache.prefill, cache.step_deferred

    def spy_prefill(K, V):
        log["prefill_kv"] = (K.clone(), V.clone())
        prefill(K, V)
        ls.prefill(host(K.float()), host(V.float()))
        ls.check_state(cache._engine, "prefill")

    def spy_step(Q, K, V, out, prev=None):
        # the patch chains its decode steps (step_deferred); reading the mean
        # weights runs this step's pending feedback first
        log["step_qkv"] = (Q.clone(), K.clone(), V.clone())
        step(Q, K, V, out, prev=prev)
        r = ls.step(host(Q), host(K), host(V), host(out), host(cache._engine.get_mean_attn_weights()))
        log["errors"].append(r)
        log["steps"] += 1
        if log["steps"] % every == 0:
            ls.check_state(cache._engine, log["steps"])

    cache.prefill, cache.step_deferred = spy_prefill, spy_step
    return ls, log


@pytest.mark.parametrize("arch", ["llama", "qwen2", "mistral", "qwen3"])
def test_patched_attention_lockstep_with_oracle(patched, oracle, arch):
    """A patched LLaMA layer (8 q / 2 KV heads, head_dim 128, the patch's own lazily
    created cache: 32k capacity, 256-token ring, f16 metadata), likewise a Mistral
    layer (16 q / 4 KV heads) and a Qwen3 layer (8 q / 2 KV heads, RMS-normed
    queries and keys before the rotation), and a patched Qwen2 layer (14 q / 2 KV
    heads, head_dim 128, a 1024-token cache set on the module so that its 52
    heavy-hitter slots fill and demote): a 700-token prompt, then 300 decode
    steps, each in lockstep with the oracle engine. The prompt's output (causal
    attention) and K/V and every 50th step's Q/K/V, as handed to the engine,
    equal the family's own unpatched forward's."""
    import transformers as tf

    from tritiercache_amd.cache import TriTierCache

    torch.manual_seed(5)
    if arch == "llama":
        from transformers.models.llama.modeling_llama import LlamaAttention as A, LlamaRotaryEmbedding as Rot

        cfg = tf.LlamaConfig(hidden_size=1024, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                             max_position_embeddings=4096)
    elif arch == "mistral":
        from transformers.models.mistral.modeling_mistral import MistralAttention as A, MistralRotaryEmbedding as Rot

        cfg = tf.MistralConfig(hidden_size=1024, num_attention_heads=16, num_key_value_heads=4, head_dim=128,
                               max_position_embeddings=4096)
    elif arch == "qwen3":
        if not hasattr(tf, "Qwen3Config"):
            pytest.skip("Qwen3 not in the installed transformers")
        from transformers.models.qwen3.modeling_qwen3 import Qwen3Attention as A, Qwen3RotaryEmbedding as Rot

        cfg = tf.Qwen3Config(hidden_size=1024, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                             max_position_embeddings=4096)
    else:
        from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention as A, Qwen2RotaryEmbedding as Rot

        cfg = tf.Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2, head_dim=128,
                             max_position_embeddings=4096)
    layer, rot = A(cfg, layer_idx=0).to(DEV).eval(), Rot(config=cfg).to(DEV)
    if arch == "qwen3":
        # non-trivial norm weights, so that a patch that skipped the q/k norms would diverge
        with torch.no_grad():
            layer.q_norm.weight.uniform_(0.5, 1.5)
            layer.k_norm.weight.uniform_(0.5, 1.5)
    if arch == "qwen2":
        layer.tri_tier_cache = TriTierCache(max_seq_len=1024, head_dim=128, num_heads=2, R_size=64, H_ratio=0.05,
                                            num_q_heads=14, score_decay=patched.SCORE_DECAY,
                                            k_group_size=patched.K_GROUP_SIZE,
                                            pbs_metadata_dtype=patched.PBS_METADATA_DTYPE)
    else:
        # the patch's own cache: create it exactly as the first forward would
        h0 = torch.randn(1, 1, cfg.hidden_size, device=DEV)
        patched._layer_cache(layer, h0.device)
    cache = layer.tri_tier_cache
    ls, log = _spy_lockstep(oracle, cache)
    family = sys.modules[A.__module__]
    unpatched = patched._ORIGINAL_FORWARDS[A]

    def family_qkv(h, pe):
        """Post-RoPE Q/K/V [1, heads, tokens, D] as the family's own unpatched
        forward computes them, taken at its call of the eager attention."""
        got, eager, impl = {}, family.eager_attention_forward, cfg._attn_implementation

        def capture(module, q, k, v, mask, **kw):
            got["q"], got["k"], got["v"] = q, k, v
            return eager(module, q, k, v, mask, **kw)

        family.eager_attention_forward, cfg._attn_implementation = capture, "eager"
        try:
            unpatched(layer, h, position_embeddings=pe, attention_mask=None)
        finally:
            family.eager_attention_forward, cfg._attn_implementation = eager, impl
        return got

    def same(mine, theirs, what):
        torch.testing.assert_close(mine, theirs.float(), rtol=1e-6, atol=1e-6, msg=lambda m: f"{arch} {what}: {m}")

    n0 = 700
    with torch.no_grad():
        h = torch.randn(1, n0, cfg.hidden_size, device=DEV)
        pe = rot(h, torch.arange(n0, device=DEV)[None])
        out, _ = layer(h, position_embeddings=pe)
        # the prompt's output: causal attention, as the family's own SDPA path computes it
        impl = cfg._attn_implementation
        cfg._attn_implementation = "sdpa"
        try:
            want, _ = unpatched(layer, h, position_embeddings=pe, attention_mask=None)
        finally:
            cfg._attn_implementation = impl
        torch.testing.assert_close(out, want, rtol=1e-5, atol=1e-5, msg=lambda m: f"{arch} prompt output: {m}")
        ref = family_qkv(h, pe)
        K, V = log["prefill_kv"]
        same(K, ref["k"][0].transpose(0, 1), "prefill K")
        same(V, ref["v"][0].transpose(0, 1), "prefill V")
        for s in range(300):
            h = torch.randn(1, 1, cfg.hidden_size, device=DEV)
            pe = rot(h, torch.tensor([[n0 + s]], device=DEV))
            out, _ = layer(h, position_embeddings=pe)
            r = log["errors"][-1]
            assert attention_ok(r), (arch, s, r)
            if s % 50 == 0:
                ref = family_qkv(h, pe)
                for mine, name in zip(log["step_qkv"], "qkv"):
                    same(mine, ref[name].reshape(-1), f"step {s} {name.upper()}")
    assert log["steps"] == 300 and cache.Total_Processed_Tokens == n0 + 300
    ls.check_state(cache._engine, "end")
    worst = {k: max(e[k] for e in log["errors"]) for k in log["errors"][0]}
    print(arch, "worst over 300 steps", {k: f"{v:.3g}" for k, v in worst.items()}, "hh", cache.HH_count, "blocks",
          cache._engine.counters()["pbs_blocks_used"], flush=True)
    if arch == "qwen2":
        assert cache.HH_count == cache.max_heavy_hitters


def test_patched_attention_weights_lockstep_with_oracle(patched, oracle):
    """A patched LLaMA layer (8 q / 2 KV heads, head_dim 128, a 1024-token cache with
    f16 metadata set on the module) called with output_attentions=True for every
    one of 150 decode steps after a 400-token prompt: each step's (1, Hq, 1, visible)
    weights -- the reference returns per-head softmax weights over the
    reconstructed cache there (patch_model.py:33-51, :162-169) -- equal float64
    softmax weights over the oracle engine's tiers, in reconstruct order, within
    1e-4 relative for every weight >= 1e-8; the engine runs in score-injected
    lockstep with the oracle (state bit-exact every 50 steps) and the last step's
    reconstruct_full_cache() equals the oracle's."""
    import transformers as tf
    from transformers.models.llama.modeling_llama import LlamaAttention as A, LlamaRotaryEmbedding as Rot

    from tritiercache_amd.cache import TriTierCache

    torch.manual_seed(9)
    cfg = tf.LlamaConfig(hidden_size=1024, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                         max_position_embeddings=4096)
    Hq, Hkv, D = 8, 2, 128
    layer, rot = A(cfg, layer_idx=0).to(DEV).eval(), Rot(config=cfg).to(DEV)
    layer.tri_tier_cache = TriTierCache(max_seq_len=1024, head_dim=D, num_heads=Hkv, R_size=64, H_ratio=0.05,
                                        num_q_heads=Hq, score_decay=patched.SCORE_DECAY,
                                        k_group_size=patched.K_GROUP_SIZE,
                                        pbs_metadata_dtype=patched.PBS_METADATA_DTYPE)
    cache = layer.tri_tier_cache
    fp16 = cache.pbs_metadata_dtype == "fp16"
    ls = _lockstep_for(oracle, cache)
    log = {}
    prefill, step_w = cache.prefill, cache.step_with_weights

    def spy_prefill(K, V):
        prefill(K, V)
        ls.prefill(host(K.float()), host(V.float()))

    def spy_step_w(Q, K, V, out):
        w, ids = step_w(Q, K, V, out)
        log["r"] = ls.step(host(Q), host(K), host(V), host(out), host(cache._engine.get_mean_attn_weights()))
        log["q"], log["ids"] = host(Q), ids
        return w, ids

    cache.prefill, cache.step_with_weights = spy_prefill, spy_step_w
    n0, worst = 400, 0.0
    with torch.no_grad():
        h = torch.randn(1, n0, cfg.hidden_size, device=DEV)
        layer(h, position_embeddings=rot(h, torch.arange(n0, device=DEV)[None]))
        ls.check_state(cache._engine, "prefill")
        for s in range(150):
            h = torch.randn(1, 1, cfg.hidden_size, device=DEV)
            out, w = layer(h, position_embeddings=rot(h, torch.tensor([[n0 + s]], device=DEV)),
                           output_attentions=True)
            assert out.shape == (1, 1, cfg.hidden_size)
            assert attention_ok(log["r"]), (s, log["r"])
            assert w.shape == (1, Hq, 1, cache.Total_Processed_Tokens - cache.WR_count), (s, w.shape)
            worst = max(worst, _check_weights_against_oracle(oracle, ls, log["q"], w[0, :, 0], log["ids"], Hq, Hkv,
                                                             D, cache.k_group_size, fp16, s))
            if (s + 1) % 50 == 0:
                ls.check_state(cache._engine, s)
    _check_reconstruct_against_oracle(oracle, ls, cache, fp16, "end")
    assert cache.HH_count > 0 and cache.PBS_count > 0
    print(f"patched layer per-head weights worst rel err {worst:.3g}", flush=True)


def test_patched_layers_chain_deferred_steps_lockstep_with_oracle(patched, oracle):
    """Two patched LLaMA layers (8 q / 2 KV heads, head_dim 128, 1024-token caches)
    stepped as a model steps them: every decode step of layer 1 runs layer 0's pending
    mean weights and score feedback in its finalize launch (the patch chains its steps
    with step_deferred). Each layer's engine runs in score-injected lockstep with its
    own oracle engine, fed the mean weights the GPU used -- read only after the next
    layer's step, so layer 0's come from layer 1's launch -- through a 400-token prompt
    and 250 decode steps: contexts within the attention tolerance, state bit-exact
    every 50 steps."""
    import transformers as tf
    from transformers.models.llama.modeling_llama import LlamaAttention as A, LlamaRotaryEmbedding as Rot

    from tritiercache_amd.cache import TriTierCache

    torch.manual_seed(13)
    cfg = tf.LlamaConfig(hidden_size=1024, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                         max_position_embeddings=4096)
    rot = Rot(config=cfg).to(DEV)
    layers, caches, lss, logs = [], [], [], []
    for i in range(2):
        layer = A(cfg, layer_idx=i).to(DEV).eval()
        layer.tri_tier_cache = TriTierCache(max_seq_len=1024, head_dim=128, num_heads=2, R_size=64, H_ratio=0.05,
                                            num_q_heads=8, score_decay=patched.SCORE_DECAY,
                                            k_group_size=patched.K_GROUP_SIZE,
                                            pbs_metadata_dtype=patched.PBS_METADATA_DTYPE)
        c = layer.tri_tier_cache
        ls = _lockstep_for(oracle, c)
        log = []
        prefill, step = c.prefill, c.step_deferred

        def spy_prefill(K, V, prefill=prefill, ls=ls):
            prefill(K, V)
            ls.prefill(host(K.float()), host(V.float()))

        def spy_step(Q, K, V, out, prev=None, step=step, log=log):
            step(Q, K, V, out, prev=prev)
            log.append((Q.clone(), K.clone(), V.clone(), out, prev))

        c.prefill, c.step_deferred = spy_prefill, spy_step
        layers.append(layer)
        caches.append(c)
        lss.append(ls)
        logs.append(log)
    n0 = 400
    with torch.no_grad():
        h = torch.randn(1, n0, cfg.hidden_size, device=DEV)
        pe = rot(h, torch.arange(n0, device=DEV)[None])
        for layer in layers:
            layer(h, position_embeddings=pe)
        for s in range(250):
            h = torch.randn(1, 1, cfg.hidden_size, device=DEV)
            pe = rot(h, torch.tensor([[n0 + s]], device=DEV))
            x = h
            for layer in layers:
                x, _ = layer(x, position_embeddings=pe)
                x = x / x.norm() * 32.0  # keep the next layer's input at a steady scale
            # layer 1's step ran layer 0's pending feedback in its finalize launch
            Q0, K0, V0, out0, prev0 = logs[0][-1]
            Q1, K1, V1, out1, prev1 = logs[1][-1]
            assert prev1 is caches[0] and (s == 0 or prev0 is caches[1])
            for i, (Q, K, V, out) in enumerate(((Q0, K0, V0, out0), (Q1, K1, V1, out1))):
                r = lss[i].step(host(Q), host(K), host(V), host(out), host(caches[i]._engine.get_mean_attn_weights()))
                assert attention_ok(r), (s, i, r)
            if (s + 1) % 50 == 0:
                for i in range(2):
                    lss[i].check_state(caches[i]._engine, (s, i))
    for c in caches:
        assert c.PBS_count > 0 and c.HH_count > 0
