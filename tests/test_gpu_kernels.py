"""GPU parity of the stateless kernels (through the C ABI) against the oracle and the golden fixtures.

Bar: packed words, scales and zeros bit-exact; attention outputs and mean
weights within max|gpu - ref| / max|ref| <= 1e-4 (FP32, ATTN_TOL below), and
on full-size layers also elementwise against float64 attention over the same
exact tier values (oracle.exact).
"""
import itertools

import numpy as np
import pytest
import torch

from oracle import synth
from oracle.exact import elementwise_ratio, exact_attention, weights_rel_err
from gpu_helpers import attention_errors, attention_ok, dev, host, make_case, quantize_blocks_gpu, rel_err, same_bits

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-4


@pytest.fixture(scope="module")
def C():
    assert torch.cuda.is_available(), "GPU test on a machine without a GPU"
    from tritiercache_amd import _C

    assert _C.device_count() > 0
    return _C


def _meta(fp16):
    return (torch.uint16, "fp16") if fp16 else (torch.float32, "fp32")


def gpu_quantize_k(C, K, kgs, fp16):
    kgs_, H, D = K.shape
    mdt, dt = _meta(fp16)
    p = torch.zeros((kgs // 16, H, D), dtype=torch.int32, device="cuda")
    s = torch.zeros((H, D), dtype=mdt, device="cuda")
    z = torch.zeros((H, D), dtype=mdt, device="cuda")
    C.quantize_k_block(dev(K), p, s, z, H, D, kgs, dt)
    return host(p), host(s), host(z)


def gpu_quantize_v(C, V, fp16):
    ch, H, D = V.shape
    mdt, dt = _meta(fp16)
    p = torch.zeros((ch, H, D // 16), dtype=torch.int32, device="cuda")
    s = torch.zeros((ch, H), dtype=mdt, device="cuda")
    z = torch.zeros((ch, H), dtype=mdt, device="cuda")
    C.quantize_v_block(dev(V), p, s, z, H, D, ch, dt)
    return host(p), host(s), host(z)


# ------------------------------------------------------------------ quantisers
def test_quantize_k_golden(C, golden):
    K = golden["kernels"]
    for i, c in enumerate(golden["kernels_index"]["qk"]):
        p, s, z = gpu_quantize_k(C, K[f"qk{i}_K"], c["kgs"], c["fp16"])
        assert same_bits(p, K[f"qk{i}_packed"]), i
        assert same_bits(s, K[f"qk{i}_scale"]) and same_bits(z, K[f"qk{i}_zero"]), i


def test_quantize_v_golden(C, golden):
    K = golden["kernels"]
    for i, c in enumerate(golden["kernels_index"]["qv"]):
        p, s, z = gpu_quantize_v(C, K[f"qv{i}_V"], c["fp16"])
        assert same_bits(p, K[f"qv{i}_packed"]), i
        assert same_bits(s, K[f"qv{i}_scale"]) and same_bits(z, K[f"qv{i}_zero"]), i


def test_quantize_v_reference_kat(C, golden):
    k = golden["qv_kat"]
    V = np.array(k["V"], np.float32).reshape(16, 2, 32)
    p, s, z = gpu_quantize_v(C, V, False)
    assert np.array_equal(p.reshape(-1).view(np.uint32), np.array(k["expected_packed"], np.uint32))
    assert np.all(np.abs(z.reshape(-1) - np.array(k["expected_min"], np.float32)) <= 1e-4)
    assert np.all(np.abs(s.reshape(-1) - np.array(k["expected_scale"], np.float32)) <= 1e-4)


def test_round_half_even_kat(C, golden):
    k = golden["tie_kat"]
    V = np.array(k["V"], np.float32).reshape(16, 1, 16)
    p, s, z = gpu_quantize_v(C, V, False)
    assert np.array_equal(p.reshape(-1).view(np.uint32), np.array(k["reference_packed"], np.uint32))


def _edge_values(shape, seed):
    """N(0,1) plus planted edge cases: constant runs, signed zeros, exact ties,
    huge and tiny magnitudes, fp16 overflow and denormal metadata."""
    x = synth.normal(seed, 0, shape, std=2.0).reshape(-1)
    n = x.size
    x[: n // 16] = 0.5
    x[n // 16: n // 8: 2] = -0.0
    x[n // 8: n // 8 + 64] = np.linspace(0, 3, 64, dtype=np.float32)
    x[n // 4: n // 4 + 32] *= 1e5
    x[n // 2: n // 2 + 32] *= 1e-6
    return x.reshape(shape).astype(np.float32)


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("kgs,H,D", [(16, 1, 8), (16, 3, 12), (16, 8, 128), (32, 4, 64), (16, 32, 128), (32, 2, 256)])
def test_quantize_k_random_vs_oracle(C, oracle, kgs, H, D, fp16):
    for seed in range(3):
        K = _edge_values((kgs, H, D), 1000 + seed)
        g = gpu_quantize_k(C, K, kgs, fp16)
        o = oracle.quantize_k(K, kgs, fp16)
        for a, b in zip(g, o):
            assert same_bits(a, b), (kgs, H, D, fp16, seed)


@pytest.mark.parametrize("fp16", [False, True])
# D / 16 words per row: powers of two, others (48, 80, 96, 112, 160, 192: the
# row's lane group is padded to a power of two) and more than 64 words
# (1040, 2048: one thread per row).
@pytest.mark.parametrize("ch,H,D", [(16, 1, 16), (16, 8, 128), (32, 4, 64), (16, 32, 128), (16, 2, 256),
                                    (16, 3, 48), (16, 2, 80), (32, 5, 96), (16, 4, 112), (16, 3, 160),
                                    (16, 2, 192), (16, 2, 1040), (16, 1, 2048)])
def test_quantize_v_random_vs_oracle(C, oracle, ch, H, D, fp16):
    for seed in range(3):
        V = _edge_values((ch, H, D), 2000 + seed)
        g = gpu_quantize_v(C, V, fp16)
        o = oracle.quantize_v(V, fp16)
        for a, b in zip(g, o):
            assert same_bits(a, b), (ch, H, D, fp16, seed)


@pytest.mark.parametrize("fp16", [False, True])
def test_quantize_v_unaligned_rows_vs_oracle(C, oracle, fp16):
    """V whose rows are only 4-byte aligned (a view one float into its storage)."""
    ch, H, D = 16, 4, 128
    V = _edge_values((ch, H, D), 2100)
    buf = torch.empty(V.size + 1, dtype=torch.float32, device="cuda")
    Vd = buf[1:].view(ch, H, D)
    Vd.copy_(torch.from_numpy(V))
    assert Vd.data_ptr() % 16 == 4
    mdt, dt = _meta(fp16)
    p = torch.zeros((ch, H, D // 16), dtype=torch.int32, device="cuda")
    s = torch.zeros((ch, H), dtype=mdt, device="cuda")
    z = torch.zeros((ch, H), dtype=mdt, device="cuda")
    C.quantize_v_block(Vd, p, s, z, H, D, ch, dt)
    for a, b in zip((host(p), host(s), host(z)), oracle.quantize_v(V, fp16)):
        assert same_bits(a, b), fp16


@pytest.mark.parametrize("fp16", [False, True])
def test_k_block_calls_past_the_grid_y_extent(C, oracle, fp16):
    """One quantize_k / dequantize_k call over more blocks than a grid's y extent (65535): the launches
    are sliced, and the blocks on both sides of the seam, the first and the last match the oracle."""
    import ctypes as ct
    from tritiercache_amd import _lib

    L = _lib.load()
    H, D, kgs, nb = 1, 16, 16, 65535 + 21
    mdt, _ = _meta(fp16)
    K = torch.randn((nb * kgs, H, D), generator=torch.Generator(device="cuda").manual_seed(77), device="cuda")
    p = torch.zeros((nb, H, D), dtype=torch.int32, device="cuda")
    sc = torch.zeros((nb, H, D), dtype=mdt, device="cuda")
    z = torch.zeros((nb, H, D), dtype=mdt, device="cuda")
    sp = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(L.tt_quantize_k_block(K.data_ptr(), p.data_ptr(), sc.data_ptr(), z.data_ptr(), nb, H, D, kgs,
                                     int(fp16), sp))
    out = torch.zeros((nb * kgs, H, D), dtype=torch.float32, device="cuda")
    _lib.check(L.tt_dequantize_k(p.data_ptr(), sc.data_ptr(), z.data_ptr(), out.data_ptr(), nb, H, D, kgs,
                                 int(fp16), sp))
    torch.cuda.synchronize()
    hk, hp, hs, hz, ho = host(K), host(p), host(sc), host(z), host(out)
    for b in (0, 1, 65533, 65534, 65535, 65536, nb - 1):
        op, os_, oz = oracle.quantize_k(hk[b * kgs:(b + 1) * kgs], kgs, fp16)
        assert same_bits(hp[b], op[0]) and same_bits(hs[b], os_) and same_bits(hz[b], oz), b
        od = oracle.dequantize_k(op, os_[None], oz[None], 1, H, D, kgs, fp16)
        assert same_bits(ho[b * kgs:(b + 1) * kgs], od), b


@pytest.mark.parametrize("fp16", [False, True])
def test_dequantize_vs_oracle(C, oracle, fp16):
    H, D, nb, kgs = 4, 64, 5, 32
    K = synth.normal(31, 0, (nb * kgs, H, D))
    mdt, dt = _meta(fp16)
    packs = [oracle.quantize_k(K[b * kgs:(b + 1) * kgs], kgs, fp16) for b in range(nb)]
    p, s, z = (np.stack([x[i] for x in packs]) for i in range(3))
    out = torch.zeros((nb * kgs, H, D), dtype=torch.float32, device="cuda")
    C.dequantize_k(dev(p), dev(s), dev(z), out, nb, H, D, kgs, dt)
    assert same_bits(host(out), oracle.dequantize_k(p, s, z, nb, H, D, kgs, fp16))
    p, s, z = oracle.quantize_v(K, fp16)
    out = torch.zeros((nb * kgs, H, D), dtype=torch.float32, device="cuda")
    C.dequantize_v(dev(p), dev(s), dev(z), out, nb * kgs, H, D, dt)
    assert same_bits(host(out), oracle.dequantize_v(p, s, z, nb * kgs, H, D, fp16))


def test_quantize_host_buffers_like_reference_tests(C, oracle):
    """numpy in / numpy out, as the reference's test_wiring_verification.py calls them."""
    K = synth.normal(41, 0, (16, 4, 64)) * 2.5 + 1.2345
    packed = np.zeros((1, 4, 64), np.int32)
    scale = np.zeros((1, 4, 64), np.uint16)
    zero = np.zeros((1, 4, 64), np.uint16)
    C.quantize_k_block(K, packed[0], scale[0], zero[0], 4, 64, 16, "fp16")
    p, s, z = oracle.quantize_k(K, 16, True)
    assert same_bits(packed[0], p[0]) and same_bits(scale[0], s) and same_bits(zero[0], z)
    out = np.zeros((16, 4, 64), np.float32)
    C.dequantize_k(packed, scale, zero, out, 1, 4, 64, 16, "fp16")
    assert same_bits(out, oracle.dequantize_k(p, s, z, 1, 4, 64, 16, True))


# ---------------------------------------------------------------- fused attention
def _run_fused_gpu(C, args, want_mw=True):
    (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16) = args
    out = torch.full((Hq, D), float("nan"), dtype=torch.float32, device="cuda")
    mw = torch.full((nd + nb * kgs,), float("nan"), dtype=torch.float32, device="cuda") if want_mw else None
    t = lambda a: dev(a) if a is not None and (not hasattr(a, "size") or a.size > 0) else None  # noqa: E731
    C.fused_attention_decode(dev(Q), t(dK) if nd else None, t(dV) if nd else None, nd,
                             t(KP) if nb else None, t(KS) if nb else None, t(KZ) if nb else None,
                             t(VP) if nb else None, t(VS) if nb else None, t(VZ) if nb else None,
                             t(ids) if nb else None, nb, Hq, Hkv, D, out, mw, kgs, "fp16" if fp16 else "fp32")
    torch.cuda.synchronize()
    return host(out), (host(mw) if want_mw else None)


def test_fused_attention_golden(C, golden):
    K = golden["kernels"]
    for i, c in enumerate(golden["kernels_index"]["fa"]):
        args = (K[f"fa{i}_Q"], K[f"fa{i}_dK"], K[f"fa{i}_dV"], c["nd"], K[f"fa{i}_KP"], K[f"fa{i}_KS"],
                K[f"fa{i}_KZ"], K[f"fa{i}_VP"], K[f"fa{i}_VS"], K[f"fa{i}_VZ"], K[f"fa{i}_ids"], c["nb"], c["Hq"],
                c["Hkv"], c["D"], c["kgs"], c["fp16"])
        out, mw = _run_fused_gpu(C, args)
        assert rel_err(out, K[f"fa{i}_out"]) <= ATTN_TOL, i
        assert rel_err(mw, K[f"fa{i}_mw"]) <= ATTN_TOL, i


SWEEP = [
    # Hq, Hkv, D, nd, nb, kgs, fp16, mask
    (1, 1, 16, 1, 1, 16, False, "none"),
    (4, 4, 16, 3, 2, 32, True, "tail"),
    (8, 2, 32, 17, 5, 16, False, "holes"),
    (6, 2, 32, 33, 5, 16, True, "block"),
    (32, 8, 128, 260, 20, 16, False, "none"),
    (32, 8, 128, 0, 40, 16, True, "tail"),
    (32, 8, 128, 300, 0, 16, False, "none"),
    (28, 4, 128, 70, 33, 16, False, "holes"),
    (12, 1, 64, 5, 9, 32, False, "tail"),
    (16, 1, 64, 40, 12, 16, True, "none"),
    (24, 2, 128, 9, 7, 16, False, "block"),
    (4, 2, 256, 18, 4, 16, True, "holes"),
    (8, 8, 256, 3, 3, 32, False, "none"),
    (3, 3, 64, 64, 8, 16, False, "all"),
    # head_dim 128 runs the matrix-core path over the packed store
    (32, 8, 128, 50, 9, 32, False, "holes"),
    (16, 2, 128, 20, 5, 32, True, "tail"),
    (16, 1, 128, 10, 6, 16, False, "none"),
    (8, 8, 128, 0, 1, 16, False, "none"),
    (7, 1, 128, 0, 3, 16, True, "block"),
    # two-head groups with 32-token blocks; three KV heads (the plan's uneven branch)
    (4, 2, 128, 12, 7, 32, True, "holes"),
    (12, 3, 128, 45, 11, 16, False, "tail"),
    # groups padded inside the matrix-core workgroup: 3 of 4 heads, 5 and 6 of 8
    (6, 2, 128, 21, 13, 16, False, "holes"),
    (10, 2, 128, 8, 10, 16, True, "tail"),
    (12, 2, 128, 33, 9, 32, False, "none"),
    # more than 64 query heads: the mean-weight rows of a 64-token block span 8 head groups
    (72, 8, 64, 30, 6, 16, False, "tail"),
    (66, 6, 128, 7, 5, 16, True, "holes"),
]


@pytest.mark.parametrize("case", SWEEP, ids=[str(c) for c in SWEEP])
def test_fused_attention_vs_oracle(C, oracle, case):
    Hq, Hkv, D, nd, nb, kgs, fp16, mask = case
    args = make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, mask, seed=500 + SWEEP.index(case))
    out, mw = _run_fused_gpu(C, args)
    ro, rmw = oracle.fused_attention_decode(*args)
    if mask == "all" and nd == 0:
        assert np.all(out == 0) and np.all(mw == 0)
        return
    assert rel_err(out, ro) <= ATTN_TOL, case
    assert rel_err(mw, rmw) <= ATTN_TOL, case
    ids = args[10]
    if nb:
        assert np.all(mw[nd:][ids[: nb * kgs] == -1] == 0)


def _random_shapes(n: int, seed: int):
    """n attention shapes drawn from a fixed seed: KV heads, group size, head_dim,
    block length, metadata width, tier lengths and the mask of the padding ids."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        Hkv = int(rng.choice([1, 2, 3, 4, 8]))
        G = int(rng.integers(1, 10))
        D = int(rng.choice([16, 32, 64, 128, 128, 128, 256]))
        kgs = int(rng.choice([16, 32]))
        nd = int(rng.choice([0, int(rng.integers(1, 40)), int(rng.integers(40, 400))]))
        nb = int(rng.choice([0, int(rng.integers(1, 8)), int(rng.integers(8, 90))]))
        if nd == 0 and nb == 0:
            continue
        mask = str(rng.choice(["none", "tail", "holes", "block"])) if nb else "none"
        out.append((Hkv * G, Hkv, D, nd, nb, kgs, bool(rng.integers(0, 2)), mask))
    return out


RANDOM_SHAPES = _random_shapes(48, 20261202)


@pytest.mark.parametrize("case", RANDOM_SHAPES, ids=[str(c) for c in RANDOM_SHAPES])
def test_fused_attention_random_shapes_vs_oracle(C, oracle, case):
    """48 seeded random shapes (GQA group 1-9, head_dim 16-256, ragged tiers,
    masked ids): output and mean weights against the oracle, elementwise. About a
    quarter of them plan an odd number of splits (3-9), whose per-head rows of
    split statistics start at odd pairs in the finalize's one-pass load."""
    Hq, Hkv, D, nd, nb, kgs, fp16, mask = case
    args = make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, mask, seed=900 + RANDOM_SHAPES.index(case))
    out, mw = _run_fused_gpu(C, args)
    ro, rmw = oracle.fused_attention_decode(*args)
    err = attention_errors(out, ro, mw, rmw)
    assert attention_ok(err), (case, err)


ODD_HEAD_DIMS = [(4, 2, 48, 37, 9, 16, False, "tail"), (6, 2, 80, 120, 30, 16, True, "holes"),
                 (12, 4, 96, 300, 41, 32, False, "block"), (7, 1, 112, 0, 25, 16, True, "none"),
                 (8, 8, 144, 19, 3, 32, True, "tail"), (10, 2, 160, 260, 17, 16, False, "holes"),
                 (3, 3, 176, 5, 60, 16, False, "tail"), (9, 3, 192, 77, 0, 16, True, "none"),
                 (2, 1, 208, 16, 12, 32, False, "holes"), (16, 2, 224, 40, 8, 16, True, "block"),
                 (4, 4, 240, 33, 14, 16, False, "tail")]


@pytest.mark.parametrize("case", ODD_HEAD_DIMS, ids=[str(c) for c in ODD_HEAD_DIMS])
def test_fused_attention_head_dims_not_powers_of_two_vs_oracle(C, oracle, case):
    """head_dim any multiple of 16 up to 256, as the reference accepts (48 to 240,
    GQA 1-8, both block sizes and metadata widths): each lane's channel range of
    the VALU kernel then starts inside a V word and can run into the next one."""
    Hq, Hkv, D, nd, nb, kgs, fp16, mask = case
    args = make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, mask, seed=1300 + D)
    out, mw = _run_fused_gpu(C, args)
    ro, rmw = oracle.fused_attention_decode(*args)
    err = attention_errors(out, ro, mw, rmw)
    assert attention_ok(err), (case, err)


@pytest.mark.parametrize("qs,ks,vs,voff", [(16.0, 50.0, 1000.0, 3000.0), (0.05, 0.01, 1e-3, 0.0), (1.0, 1.0, 1e-7, 1.0)])
def test_fused_attention_extreme_scales(C, oracle, qs, ks, vs, voff):
    """Q, K, V far from unit scale: the f16 operands of the matrix-core path are
    normalised per head (Q) and per tile (p * v_scale)."""
    Hq, Hkv, D, nd, nb, kgs = 16, 4, 128, 40, 24, 16
    args = list(make_case(oracle, Hq, Hkv, D, nd, nb, kgs, False, "tail", seed=77))
    rng = np.random.default_rng(77)
    Kp = rng.standard_normal((nb * kgs, Hkv, D)).astype(np.float32) * np.float32(ks)
    Vp = (rng.standard_normal((nb * kgs, Hkv, D)).astype(np.float32) * np.float32(vs) + np.float32(voff))
    packs = [(oracle.quantize_k(Kp[b * kgs:(b + 1) * kgs], kgs, False),
              oracle.quantize_v(Vp[b * kgs:(b + 1) * kgs], False)) for b in range(nb)]
    args[0] = (args[0] * np.float32(qs)).astype(np.float32)
    args[1] = (args[1] * np.float32(ks)).astype(np.float32)
    args[2] = (args[2] * np.float32(vs) + np.float32(voff)).astype(np.float32)
    args[4] = np.stack([k[0] for k, _ in packs])
    args[5] = np.stack([k[1] for k, _ in packs])
    args[6] = np.stack([k[2] for k, _ in packs])
    args[7] = np.concatenate([v[0] for _, v in packs])
    args[8] = np.concatenate([v[1] for _, v in packs])
    args[9] = np.concatenate([v[2] for _, v in packs])
    args = tuple(args)
    out, mw = _run_fused_gpu(C, args)
    ro, rmw = oracle.fused_attention_decode(*args)
    assert np.all(np.isfinite(out)) and np.all(np.isfinite(mw))
    assert rel_err(out, ro) <= ATTN_TOL, (qs, ks, vs, voff)
    assert rel_err(mw, rmw) <= ATTN_TOL, (qs, ks, vs, voff)


def test_fused_attention_without_mean_weights(C, oracle):
    args = make_case(oracle, 32, 8, 128, 100, 30, 16, False, "tail", seed=5)
    out, _ = _run_fused_gpu(C, args, want_mw=False)
    ro, _ = oracle.fused_attention_decode(*args)
    assert rel_err(out, ro) <= ATTN_TOL


def test_fused_attention_empty(C, oracle):
    """dense_count = 0 and num_blocks = 0: output is all zeros (sum_exp guard)."""
    args = make_case(oracle, 4, 2, 64, 0, 0, 16, False, "none", seed=6)
    out, mw = _run_fused_gpu(C, args)
    assert np.all(out == 0)


def test_fused_attention_host_pointers_like_reference_benchmark(C, oracle):
    """CPU tensors passed as data_ptr() integers, as benchmark_latency.py:214-233 does."""
    args = make_case(oracle, 32, 8, 128, 260, 20, 16, False, "none", seed=7)
    (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16) = args
    ts = [torch.from_numpy(np.ascontiguousarray(a)) for a in (Q, dK, dV, KP, KS, KZ, VP, VS, VZ, ids)]
    out = torch.empty((Hq, D), dtype=torch.float32)
    mw = torch.empty((nd + nb * kgs,), dtype=torch.float32)
    C.fused_attention_decode(ts[0].data_ptr(), ts[1].data_ptr(), ts[2].data_ptr(), nd, ts[3].data_ptr(),
                             ts[4].data_ptr(), ts[5].data_ptr(), ts[6].data_ptr(), ts[7].data_ptr(), ts[8].data_ptr(),
                             ts[9].data_ptr(), nb, Hq, Hkv, D, out.data_ptr(), mw.data_ptr())
    ro, rmw = oracle.fused_attention_decode(*args)
    assert rel_err(out.numpy(), ro) <= ATTN_TOL and rel_err(mw.numpy(), rmw) <= ATTN_TOL


def test_fused_attention_errors(C):
    z = torch.zeros(16, device="cuda")
    with pytest.raises(ValueError):
        C.fused_attention_decode(z, None, None, -1, None, None, None, None, None, None, None, 0, 1, 1, 16, z)
    with pytest.raises(ValueError):
        C.fused_attention_decode(z, None, None, 0, None, None, None, None, None, None, None, -2, 1, 1, 16, z)
    with pytest.raises(ValueError):
        C.fused_attention_decode(z, None, None, 0, None, None, None, None, None, None, None, 0, 0, 1, 16, z)
    with pytest.raises(ValueError):  # GQA ratio must be integral
        C.fused_attention_decode(z, None, None, 0, None, None, None, None, None, None, None, 0, 3, 2, 16, z)
    with pytest.raises(ValueError):  # unsupported head_dim
        C.fused_attention_decode(z, None, None, 0, None, None, None, None, None, None, None, 0, 1, 1, 24, z)
    with pytest.raises(ValueError):  # dense tier missing while dense_count > 0
        C.fused_attention_decode(z, None, None, 3, None, None, None, None, None, None, None, 0, 1, 1, 16, z)
    with pytest.raises(ValueError):
        C.fused_attention_decode(torch.zeros(4, 4, device="cuda").t(), None, None, 0, None, None, None, None, None,
                                 None, None, 0, 1, 1, 16, z)


# ------------------------------------------------------- full-size single layers
def _tiered_layer(C, Hq, Hkv, D, ctx, fp16, seed, k_outliers=None):
    """One layer at full context: 4 sinks + 256 recent + ceil(5%) heavy hitters in FP32,
    the rest packed on the GPU in 16-token blocks; the last block padded with a copy
    of the last valid token and -1 ids. K outlier channels (4 per KV head): "x8" scales
    them by 8, "t3" draws them from Student-t with 3 degrees of freedom."""
    S, R = 4, 256
    hh = int(np.ceil(np.float32(ctx) * np.float32(0.05)))
    nd = S + hh + R
    npk = ctx - nd
    nb = (npk + 15) // 16
    g = torch.Generator(device="cuda").manual_seed(seed)
    K = torch.randn((ctx, Hkv, D), generator=g, device="cuda")
    V = torch.randn((ctx, Hkv, D), generator=g, device="cuda")
    for h in range(Hkv if k_outliers else 0):
        ch = torch.randperm(D, generator=g, device="cuda")[:4]
        if k_outliers == "x8":
            K[:, h, ch] *= 8.0
        else:
            z = torch.randn((ctx, 4), generator=g, device="cuda")
            chi = (torch.randn((ctx, 4, 3), generator=g, device="cuda") ** 2).sum(-1)
            K[:, h, ch] = z / torch.sqrt(chi / 3.0)
    Q = torch.randn((Hq, D), generator=g, device="cuda")
    dK, dV = K[:nd].contiguous(), V[:nd].contiguous()
    pk, pv = K[nd:], V[nd:]
    pad = nb * 16 - npk
    if pad:
        pk = torch.cat([pk, pk[-1:].expand(pad, Hkv, D)])
        pv = torch.cat([pv, pv[-1:].expand(pad, Hkv, D)])
    blocks = quantize_blocks_gpu(C, pk.contiguous(), pv.contiguous(), 16, fp16)
    ids = torch.arange(nb * 16, dtype=torch.int64, device="cuda") + nd
    if pad:
        ids[-pad:] = -1
    return Q, dK, dV, nd, blocks, ids, nb


@pytest.mark.parametrize("name,Hq,Hkv,ctx,fp16,outliers", [
    ("mha-8k", 32, 32, 8192, False, None),
    ("llama3-8b-32k", 32, 8, 32768, False, "x8"),
    ("llama3-8b-32k-fp16", 32, 8, 32768, True, "x8"),
    # 7:1 GQA (8-head groups), 128-token mean-weight blocks (over 64k tokens) and
    # heavy-tailed K channels, as the 128k Qwen2-7B workload specifies
    ("qwen2-7b-128k", 28, 4, 131072, False, "t3"),
    ("qwen2-7b-128k-fp16", 28, 4, 131072, True, "t3"),
    # long enough that every wave of the four-head and one-head groups takes
    # more pairs than its logits buffer holds (flushes inside the loop)
    ("llama3-8b-96k", 32, 8, 98304, False, "x8"),
    ("mha-32k", 32, 32, 32768, True, None),
    # KV head counts that do not divide the CUs into whole rounds: slot groups
    # rounded up (40/40 at 8k) or down to what every XCD holds (40/10 at 16k)
    ("phi3-medium-16k", 40, 10, 16384, False, "x8"),
    ("mha40-8k", 40, 40, 8192, True, None),
    # head_dim 64: KV heads taken in pairs as heads of 128 channels on the matrix
    # cores (GQA 4:1 -> groups of 8, 1:1 -> groups of 2, 7:1 -> 14 in chunks of 8),
    # and an odd KV head count on the VALU kernel
    ("hd64-llama-32k", 32, 8, 32768, False, "x8"),
    ("hd64-llama-32k-fp16", 32, 8, 32768, True, "x8"),
    ("hd64-mha-8k", 16, 16, 8192, False, None),
    ("hd64-qwen2-0.5b-32k", 14, 2, 32768, True, "t3"),
    ("hd64-smollm-8k", 9, 3, 8192, True, None),
])
def test_full_size_layer_vs_oracle(C, oracle, name, Hq, Hkv, ctx, fp16, outliers):
    """A full-context layer against the oracle (the reference's float32 algorithm) and
    against float64 attention over the same exact tier values, elementwise:
    |gpu_i - exact_i| <= 1e-4 |exact_i| + 1e-6 max|exact| for the outputs, relative
    error <= 1e-4 for every mean weight >= 1e-8. Against the float32 oracle the
    bound is max-normwise 1e-4 plus the oracle's own normwise distance from the
    exact result, and elementwise with 1e-5 max|ref| of absolute slack (the
    oracle's sequential float32 softmax sums sit ~1e-6 max|ref| from exact, and
    up to ~1e-4 at head_dim 64 with 8x key outliers, where a few keys take most
    of a head's weight and later terms round away in the running sum)."""
    D = 64 if name.startswith("hd64") else 128
    Q, dK, dV, nd, blocks, ids, nb = _tiered_layer(C, Hq, Hkv, D, ctx, fp16, seed=ctx + Hkv, k_outliers=outliers)
    out = torch.empty((Hq, D), dtype=torch.float32, device="cuda")
    mw = torch.empty((nd + nb * 16,), dtype=torch.float32, device="cuda")
    dt = "fp16" if fp16 else "fp32"
    C.fused_attention_decode(Q, dK, dV, nd, *blocks, ids, nb, Hq, Hkv, D, out, mw, 16, dt)
    torch.cuda.synchronize()
    hb = [host(b) for b in blocks]
    args = (host(Q), host(dK), host(dV), nd, *hb, host(ids), nb, Hq, Hkv, D, 16, fp16)
    ro, rmw = oracle.fused_attention_decode(*args)
    xo, xmw = exact_attention(oracle, *args)
    go, gmw = host(out), host(mw)
    r = dict(norm_vs_oracle=rel_err(go, ro), elem_vs_oracle=elementwise_ratio(go, ro, atol_frac=1e-5),
             elem_vs_exact=elementwise_ratio(go, xo), mw_norm_vs_oracle=rel_err(gmw, rmw),
             mw_rel_vs_oracle=weights_rel_err(gmw, rmw), mw_rel_vs_exact=weights_rel_err(gmw, xmw),
             oracle_elem_vs_exact=elementwise_ratio(ro, xo), oracle_norm_vs_exact=rel_err(ro, xo),
             oracle_mw_norm_vs_exact=rel_err(rmw, xmw), oracle_mw_rel_vs_exact=weights_rel_err(rmw, xmw))
    print(name, {k: f"{v:.3g}" for k, v in r.items()}, flush=True)
    assert r["norm_vs_oracle"] <= ATTN_TOL + r["oracle_norm_vs_exact"] and r["elem_vs_oracle"] <= 1.0, (name, r)
    assert r["elem_vs_exact"] <= 1.0, (name, r)
    assert r["mw_norm_vs_oracle"] <= ATTN_TOL + r["oracle_mw_norm_vs_exact"], (name, r)
    assert r["mw_rel_vs_oracle"] <= 1e-4 + r["oracle_mw_rel_vs_exact"] and r["mw_rel_vs_exact"] <= 1e-4, (name, r)
    assert abs(float(gmw.astype(np.float64).sum()) - 1.0) < 1e-3


def test_library_workspace_grows_between_calls(C):
    """tt_fused_attention_decode keeps one library-owned workspace per device and
    grows it on demand (device synchronise, free, allocate). A small layer, then
    one whose workspace exceeds every earlier call's (64 query heads over a
    393,216-token layer: 96 MiB of logits), then the small layer again: every
    output and mean-weight vector equals, bit for bit, the same call with a
    caller-provided workspace (tt_fused_attention_decode_ws)."""
    import ctypes

    from tritiercache_amd import _lib

    L = _lib.load()
    D = 128
    layers = [_tiered_layer(C, 8, 2, D, 2048, False, seed=61),
              _tiered_layer(C, 64, 2, D, 393216, False, seed=62, k_outliers="x8")]
    hq = [8, 64]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i in (0, 1, 0):
        Q, dK, dV, nd, blocks, ids, nb = layers[i]
        Hq = hq[i]
        n = nd + nb * 16
        ptrs = [Q.data_ptr(), dK.data_ptr(), dV.data_ptr(), nd, *(b.data_ptr() for b in blocks), ids.data_ptr(), nb,
                Hq, 2, D]
        out_lib = torch.full((Hq, D), float("nan"), device="cuda")
        mw_lib = torch.full((n,), float("nan"), device="cuda")
        _lib.check(L.tt_fused_attention_decode(*ptrs, out_lib.data_ptr(), mw_lib.data_ptr(), 16, 0, stream),
                   "fused_attention_decode")
        ws_bytes = int(L.tt_fused_attention_workspace_bytes(nd, nb, Hq, 2, D, 16, 1))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        out_ws = torch.full_like(out_lib, float("nan"))
        mw_ws = torch.full_like(mw_lib, float("nan"))
        _lib.check(L.tt_fused_attention_decode_ws(*ptrs, out_ws.data_ptr(), mw_ws.data_ptr(), 16, 0, ws.data_ptr(),
                                                  ws_bytes, stream), "fused_attention_decode_ws")
        torch.cuda.synchronize()
        assert torch.isfinite(out_lib).all() and torch.isfinite(mw_lib).all(), i
        assert torch.equal(out_lib, out_ws) and torch.equal(mw_lib, mw_ws), (i, Hq, n)
        if i == 1:
            assert Hq * n * 4 >= 96 << 20
