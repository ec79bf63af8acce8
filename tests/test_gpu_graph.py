"""HIP-graph capture and replay of the stateless entry points (through the C ABI).

Each captured call is replayed several times with new inputs written into the
captured buffers between replays (eager kernels of the program itself run in
between), and every replay must match an eager call on the same inputs bit for
bit: the kernels are deterministic (no atomics, fixed merge order), and any
memset node or stale argument recorded in the graph would show up here.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import synth
from gpu_helpers import attention_errors, attention_ok, dev, host, rel_err, same_bits
from oracle.exact import weights_rel_err
import test_gpu_kernels as K

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    assert torch.cuda.is_available(), "GPU test on a machine without a GPU"
    from tritiercache_amd import _lib

    return _lib


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("Hq,Hkv,D,nd,nb,kgs,fp16,mask", [
    (32, 8, 128, 70, 40, 16, False, "holes"),
    (28, 4, 128, 33, 21, 16, True, "tail"),
    (8, 2, 64, 17, 9, 32, False, "none"),
])
def test_fused_attention_graph_replays(lib, oracle, Hq, Hkv, D, nd, nb, kgs, fp16, mask):
    L = lib.load()
    args = K.make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, mask, seed=900 + Hq)
    (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16) = args
    t = {k: dev(v) for k, v in dict(Q=Q, dK=dK, dV=dV, KP=KP, KS=KS, KZ=KZ, VP=VP, VS=VS, VZ=VZ, ids=ids).items()}
    n = nd + nb * kgs
    ws_bytes = int(L.tt_fused_attention_workspace_bytes(nd, nb, Hq, Hkv, D, kgs, 1))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")

    def call(out, mw, work):
        rc = L.tt_fused_attention_decode_ws(
            t["Q"].data_ptr(), t["dK"].data_ptr(), t["dV"].data_ptr(), nd, t["KP"].data_ptr(), t["KS"].data_ptr(),
            t["KZ"].data_ptr(), t["VP"].data_ptr(), t["VS"].data_ptr(), t["VZ"].data_ptr(), t["ids"].data_ptr(), nb,
            Hq, Hkv, D, out.data_ptr(), mw.data_ptr(), kgs, int(fp16), work.data_ptr(), ws_bytes, _stream())
        lib.check(rc, "fused_attention_decode_ws")

    g_out = torch.zeros((Hq, D), device="cuda")
    g_mw = torch.zeros((n,), device="cuda")
    call(g_out, g_mw, ws)  # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(g_out, g_mw, ws)

    e_out = torch.zeros_like(g_out)
    e_mw = torch.zeros_like(g_mw)
    e_ws = torch.empty_like(ws)
    for rep in range(4):
        # new query (and new dense keys on odd replays) in the captured buffers
        t["Q"].copy_(dev(synth.normal(7000 + rep, 0, (Hq, D))))
        if rep % 2:
            t["dK"].mul_(-0.5)
        g_out.fill_(float("nan"))
        g_mw.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        call(e_out, e_mw, e_ws)
        torch.cuda.synchronize()
        assert torch.equal(g_out, e_out), rep
        assert torch.equal(g_mw, e_mw), rep
        # and the replay is right, not only repeatable
        hargs = (host(t["Q"]), host(t["dK"]), dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16)
        ro, rmw = oracle.fused_attention_decode(*hargs)
        assert rel_err(host(g_out), ro) <= K.ATTN_TOL, rep
        assert rel_err(host(g_mw), rmw) <= K.ATTN_TOL, rep


def test_quantizers_graph_replays(lib, oracle):
    L = lib.load()
    kgs, H, D, nblk = 16, 8, 128, 6
    Kt = torch.zeros((nblk * kgs, H, D), device="cuda")
    Vt = torch.zeros((nblk * kgs, H, D), device="cuda")
    kp = torch.zeros((nblk, H, D), dtype=torch.int32, device="cuda")
    ks = torch.zeros((nblk, H, D), device="cuda")
    kz = torch.zeros((nblk, H, D), device="cuda")
    vp = torch.zeros((nblk * kgs, H, D // 16), dtype=torch.int32, device="cuda")
    vs = torch.zeros((nblk * kgs, H), device="cuda")
    vz = torch.zeros((nblk * kgs, H), device="cuda")

    def call():
        lib.check(L.tt_quantize_k_block(Kt.data_ptr(), kp.data_ptr(), ks.data_ptr(), kz.data_ptr(), nblk, H, D, kgs,
                                        0, _stream()), "quantize_k")
        lib.check(L.tt_quantize_v_block(Vt.data_ptr(), vp.data_ptr(), vs.data_ptr(), vz.data_ptr(), nblk * kgs, H, D,
                                        0, _stream()), "quantize_v")

    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for rep in range(3):
        Kh = synth.normal(8100 + rep, 0, (nblk * kgs, H, D)) * np.float32(1 + rep)
        Vh = synth.normal(8100 + rep, 1, (nblk * kgs, H, D))
        Kt.copy_(dev(Kh))
        Vt.copy_(dev(Vh))
        kp.fill_(-1)
        vp.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        for b in range(nblk):
            p, s, z = oracle.quantize_k(Kh[b * kgs:(b + 1) * kgs], kgs, False)
            assert same_bits(host(kp[b:b + 1]), p) and same_bits(host(ks[b]), s) and same_bits(host(kz[b]), z), rep
        p, s, z = oracle.quantize_v(Vh, False)
        assert same_bits(host(vp), p) and same_bits(host(vs), s) and same_bits(host(vz), z), rep


def test_batched_decode_graph_replays(lib, oracle):
    """tt_fused_attention_decode_batched captured once (its plan is fixed at capture) and replayed with new queries:
    every replay equals an eager call bit for bit and matches the oracle per sequence."""
    L = lib.load()
    Hq, Hkv, D, kgs = 32, 8, 128, 16
    sizes = [(260, 40), (0, 25), (300, 0), (17, 3), (120, 90)]
    cases = [K.make_case(oracle, Hq, Hkv, D, nd, nb, kgs, False, "tail", seed=1500 + i) for i, (nd, nb) in enumerate(sizes)]
    keep = []

    def tensors(args):
        (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, *_rest) = args
        return {k: dev(v) for k, v in dict(Q=Q, dK=dK, dV=dV, KP=KP, KS=KS, KZ=KZ, VP=VP, VS=VS, VZ=VZ, ids=ids).items()}

    ts = [tensors(a) for a in cases]

    def descs(outs, mws):
        arr = (lib.DecodeSeq * len(cases))()
        for i, (a, t) in enumerate(zip(cases, ts)):
            nd, nb = a[3], a[11]
            s = arr[i]
            s.Q = t["Q"].data_ptr()
            if nd:
                s.dense_K, s.dense_V = t["dK"].data_ptr(), t["dV"].data_ptr()
            if nb:
                s.PBS_K_Packed, s.PBS_K_Scales, s.PBS_K_Zeroes = (t["KP"].data_ptr(), t["KS"].data_ptr(),
                                                                  t["KZ"].data_ptr())
                s.PBS_V_Packed, s.PBS_V_Scales, s.PBS_V_Zeroes = (t["VP"].data_ptr(), t["VS"].data_ptr(),
                                                                  t["VZ"].data_ptr())
                s.PBS_token_ids = t["ids"].data_ptr()
            s.attn_output, s.mean_attn_weights = outs[i].data_ptr(), mws[i].data_ptr()
            s.dense_count, s.num_blocks = nd, nb
        d = torch.from_numpy(np.frombuffer(bytes(arr), dtype=np.uint8).copy()).cuda()
        keep.append(d)
        return arr, d

    g_out = [torch.zeros((Hq, D), device="cuda") for _ in cases]
    g_mw = [torch.zeros((a[3] + a[11] * kgs,), device="cuda") for a in cases]
    e_out = [torch.zeros_like(x) for x in g_out]
    e_mw = [torch.zeros_like(x) for x in g_mw]
    g_arr, g_dev = descs(g_out, g_mw)
    e_arr, e_dev = descs(e_out, e_mw)
    n = len(cases)
    ws_bytes = int(L.tt_batched_decode_workspace_bytes(g_arr, n, Hq, Hkv, D, kgs))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    e_ws = torch.empty_like(ws)

    def call(arr, d, work):
        lib.check(L.tt_fused_attention_decode_batched(arr, d.data_ptr(), n, Hq, Hkv, D, kgs, 0, work.data_ptr(),
                                                      ws_bytes, _stream()), "batched")

    call(g_arr, g_dev, ws)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(g_arr, g_dev, ws)
    for rep in range(3):
        for i, t in enumerate(ts):
            t["Q"].copy_(dev(synth.normal(7100 + 10 * rep + i, 0, (Hq, D))))
        for x in g_out + g_mw:
            x.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        call(e_arr, e_dev, e_ws)
        torch.cuda.synchronize()
        for i, a in enumerate(cases):
            assert torch.equal(g_out[i], e_out[i]), (rep, i)
            assert torch.equal(g_mw[i], e_mw[i]), (rep, i)
            hargs = (host(ts[i]["Q"]),) + tuple(a[1:])
            ro, rmw = oracle.fused_attention_decode(*hargs)
            assert rel_err(host(g_out[i]), ro) <= K.ATTN_TOL, (rep, i)
            assert rel_err(host(g_mw[i]), rmw) <= K.ATTN_TOL, (rep, i)


@pytest.mark.parametrize("Hq,Hkv,D,nd,nb,kgs,fp16", [(32, 8, 128, 300, 120, 16, False), (8, 2, 64, 40, 30, 32, True)])
def test_split_finalize_on_two_streams(lib, oracle, Hq, Hkv, D, nd, nb, kgs, fp16):
    """tt_attention_partials, a merge-only tt_attention_finalize on the main stream and
    a mean-weights-only one on a second stream after an event (eagerly, and as one
    captured graph replayed with new inputs) match tt_fused_attention_decode_ws: the
    output bit for bit (same merge), the mean weights within 1e-6 (their softmax
    statistics come from the merge instead of being rebuilt)."""
    L = lib.load()
    args = K.make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, "tail", seed=950 + Hq)
    (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16) = args
    t = {k: dev(v) for k, v in dict(Q=Q, dK=dK, dV=dV, KP=KP, KS=KS, KZ=KZ, VP=VP, VS=VS, VZ=VZ, ids=ids).items()}
    n = nd + nb * kgs
    ws_bytes = int(L.tt_fused_attention_workspace_bytes(nd, nb, Hq, Hkv, D, kgs, 1))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    tier = lambda: (t["Q"].data_ptr(), t["dK"].data_ptr(), t["dV"].data_ptr(), nd, t["KP"].data_ptr(),  # noqa: E731
                    t["KS"].data_ptr(), t["KZ"].data_ptr(), t["VP"].data_ptr(), t["VS"].data_ptr(),
                    t["VZ"].data_ptr(), t["ids"].data_ptr(), nb, Hq, Hkv, D)

    def fused(out, mw):
        lib.check(L.tt_fused_attention_decode_ws(*tier(), out.data_ptr(), mw.data_ptr(), kgs, int(fp16),
                                                 ws.data_ptr(), ws_bytes, _stream()), "fused")

    def split(out, mw):
        main_s = torch.cuda.current_stream()
        lib.check(L.tt_attention_partials(*tier(), kgs, int(fp16), 1, ws.data_ptr(), ws_bytes, _stream()), "partials")
        lib.check(L.tt_attention_finalize(t["Q"].data_ptr(), nd, nb, Hq, Hkv, D, out.data_ptr(), None, kgs, int(fp16),
                                          1, ws.data_ptr(), ws_bytes, _stream()), "merge")
        ev = torch.cuda.Event()
        ev.record(main_s)
        side.wait_event(ev)
        lib.check(L.tt_attention_finalize(t["Q"].data_ptr(), nd, nb, Hq, Hkv, D, None, mw.data_ptr(), kgs, int(fp16),
                                          1, ws.data_ptr(), ws_bytes, C.c_void_p(side.cuda_stream)), "mean")
        main_s.wait_stream(side)

    def check(out, mw):
        r_out = torch.empty((Hq, D), device="cuda")
        r_mw = torch.empty((n,), device="cuda")
        fused(r_out, r_mw)
        torch.cuda.synchronize()
        assert same_bits(host(out), host(r_out))
        assert np.abs(host(mw) - host(r_mw)).max() <= 1e-6 * np.abs(host(r_mw)).max()
        # elementwise, like every other mean-weight check: against the fused call and the oracle
        assert weights_rel_err(host(mw), host(r_mw)) <= 1e-5
        ro, rmw = oracle.fused_attention_decode(host(t["Q"]), *args[1:])
        err = attention_errors(host(out), ro, host(mw), rmw)
        assert attention_ok(err), err

    out = torch.full((Hq, D), float("nan"), device="cuda")
    mw = torch.full((n,), float("nan"), device="cuda")
    split(out, mw)
    torch.cuda.synchronize()
    check(out, mw)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        split(out, mw)
    for r in range(3):
        t["Q"].copy_(dev(synth.normal(960 + r, 0, (Hq, D))))
        out.fill_(float("nan"))
        mw.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        check(out, mw)
    # neither output: rejected
    assert L.tt_attention_finalize(t["Q"].data_ptr(), nd, nb, Hq, Hkv, D, None, None, kgs, int(fp16), 1,
                                   ws.data_ptr(), ws_bytes, _stream()) == 1


@pytest.mark.parametrize("Hq,Hkv,D,kgs,fp16,sizes", [
    (32, 8, 128, 16, False, [(300, 120), (250, 140), (330, 90)]),
    (28, 4, 128, 16, True, [(40, 600), (70, 560), (33, 610)]),
    (8, 2, 64, 32, False, [(40, 30), (12, 44), (64, 9)]),
])
def test_deferred_mean_weights_across_layers(lib, oracle, Hq, Hkv, D, kgs, fp16, sizes):
    """Layers run back to back, each layer's mean weights computed in the next layer's finalize launch
    (tt_attention_finalize_deferred over two alternating workspaces; the first layer merged alone, the last
    layer's mean weights by a mean-only tt_attention_finalize) match one tt_fused_attention_decode_ws call
    per layer: outputs bit for bit (same merge), mean weights within 1e-6 of the largest (their softmax
    statistics come from the merge instead of being rebuilt); eagerly and as a captured graph replayed with
    new queries. Overlapping workspaces are rejected."""
    L = lib.load()
    layers = []
    for i, (nd, nb) in enumerate(sizes):
        args = K.make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, "tail", seed=970 + 7 * i + Hq)
        (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb) = args[:12]
        t = {k: dev(v) for k, v in dict(Q=Q, dK=dK, dV=dV, KP=KP, KS=KS, KZ=KZ, VP=VP, VS=VS, VZ=VZ, ids=ids).items()}
        n = nd + nb * kgs
        t.update(nd=nd, nb=nb, args=args, out=torch.empty((Hq, D), device="cuda"), mw=torch.empty((n,), device="cuda"),
                 rout=torch.empty((Hq, D), device="cuda"), rmw=torch.empty((n,), device="cuda"))
        layers.append(t)
    ws_bytes = max(int(L.tt_fused_attention_workspace_bytes(t["nd"], t["nb"], Hq, Hkv, D, kgs, 1)) for t in layers)
    ws = [torch.empty(ws_bytes, dtype=torch.uint8, device="cuda") for _ in range(2)]

    def tier(t):
        return (t["Q"].data_ptr(), t["dK"].data_ptr(), t["dV"].data_ptr(), t["nd"], t["KP"].data_ptr(),
                t["KS"].data_ptr(), t["KZ"].data_ptr(), t["VP"].data_ptr(), t["VS"].data_ptr(), t["VZ"].data_ptr(),
                t["ids"].data_ptr(), t["nb"], Hq, Hkv, D)

    def reference():
        for t in layers:
            lib.check(L.tt_fused_attention_decode_ws(*tier(t), t["rout"].data_ptr(), t["rmw"].data_ptr(), kgs,
                                                     int(fp16), ws[0].data_ptr(), ws_bytes, _stream()), "fused")

    def deferred():
        last = len(layers) - 1
        for i, t in enumerate(layers):
            w = ws[i % 2]
            lib.check(L.tt_attention_partials(*tier(t), kgs, int(fp16), 1, w.data_ptr(), ws_bytes, _stream()),
                      "partials")
            if i == 0:
                lib.check(L.tt_attention_finalize(t["Q"].data_ptr(), t["nd"], t["nb"], Hq, Hkv, D,
                                                  t["out"].data_ptr(), None, kgs, int(fp16), 1, w.data_ptr(),
                                                  ws_bytes, _stream()), "merge")
            else:
                p = layers[i - 1]
                lib.check(L.tt_attention_finalize_deferred(
                    t["Q"].data_ptr(), t["nd"], t["nb"], Hq, Hkv, D, t["out"].data_ptr(), kgs, int(fp16),
                    w.data_ptr(), ws_bytes, p["nd"], p["nb"], p["mw"].data_ptr(), ws[(i - 1) % 2].data_ptr(),
                    ws_bytes, _stream()), "deferred")
        t = layers[last]
        lib.check(L.tt_attention_finalize(t["Q"].data_ptr(), t["nd"], t["nb"], Hq, Hkv, D, None, t["mw"].data_ptr(),
                                          kgs, int(fp16), 1, ws[last % 2].data_ptr(), ws_bytes, _stream()), "mean")

    def check(tag):
        reference()
        torch.cuda.synchronize()
        for i, t in enumerate(layers):
            assert same_bits(host(t["out"]), host(t["rout"])), (tag, i)
            r = host(t["rmw"])
            assert np.abs(host(t["mw"]) - r).max() <= 1e-6 * np.abs(r).max(), (tag, i)
            # elementwise, like every other mean-weight check: against the fused call and the oracle
            assert weights_rel_err(host(t["mw"]), r) <= 1e-5, (tag, i)
            ro, rmw = oracle.fused_attention_decode(host(t["Q"]), *t["args"][1:])
            err = attention_errors(host(t["out"]), ro, host(t["mw"]), rmw)
            assert attention_ok(err), (tag, i, err)

    for t in layers:
        t["out"].fill_(float("nan"))
        t["mw"].fill_(float("nan"))
    deferred()
    torch.cuda.synchronize()
    check("eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        deferred()
    for r in range(3):
        for i, t in enumerate(layers):
            t["Q"].copy_(dev(synth.normal(990 + 10 * r + i, 0, (Hq, D))))
            t["out"].fill_(float("nan"))
            t["mw"].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        check(f"replay {r}")
    # one workspace for both calls: rejected before any launch
    t, p = layers[1], layers[0]
    assert L.tt_attention_finalize_deferred(t["Q"].data_ptr(), t["nd"], t["nb"], Hq, Hkv, D, t["out"].data_ptr(), kgs,
                                            int(fp16), ws[0].data_ptr(), ws_bytes, p["nd"], p["nb"],
                                            p["mw"].data_ptr(), ws[0].data_ptr(), ws_bytes, _stream()) == 1
