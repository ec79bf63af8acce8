"""tt_fused_attention_decode_noalloc (scratch in a static device array) against
tt_fused_attention_decode (allocated workspace), called through the C ABI.

Two calls in a row on one GPU, the second with a smaller input, so the second
runs on scratch that still holds the first call's contents; both must match
the allocating entry point bit for bit (same kernels, same plan). A call whose
workspace exceeds the static scratch is rejected on the host.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import dev, host, make_case, same_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("needs the GPU")
    from tritiercache_amd import _lib

    return _lib.load()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _args(case):
    Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16 = case
    return dict(Q=dev(Q), dK=dev(dK), dV=dev(dV), nd=nd, KP=dev(KP), KS=dev(KS), KZ=dev(KZ), VP=dev(VP),
                VS=dev(VS), VZ=dev(VZ), ids=dev(ids), nb=nb, Hq=Hq, Hkv=Hkv, D=D, kgs=kgs, fp16=int(fp16))


def _call(fn, a, out, mw):
    return fn(_ptr(a["Q"]), _ptr(a["dK"]), _ptr(a["dV"]), a["nd"], _ptr(a["KP"]), _ptr(a["KS"]), _ptr(a["KZ"]),
              _ptr(a["VP"]), _ptr(a["VS"]), _ptr(a["VZ"]), _ptr(a["ids"]), a["nb"], a["Hq"], a["Hkv"], a["D"],
              _ptr(out), _ptr(mw), a["kgs"], a["fp16"], None)


def _both(lib, a):
    n_tok = a["nd"] + a["nb"] * a["kgs"]
    res = []
    for fn in (lib.tt_fused_attention_decode, lib.tt_fused_attention_decode_noalloc):
        out = torch.full((a["Hq"], a["D"]), float("nan"), dtype=torch.float32, device="cuda")
        mw = torch.full((n_tok,), float("nan"), dtype=torch.float32, device="cuda")
        rc = _call(fn, a, out, mw)
        assert rc == 0, lib.tt_last_error()
        torch.cuda.synchronize()
        res.append((host(out), host(mw)))
    return res


def test_noalloc_matches_allocating_entry_point_twice(lib, oracle):
    # First call: the 32k Llama-3-8B layer shape with FP32 metadata (about
    # 6 MB of scratch); second: a small GQA case with FP16 metadata, masked
    # slots and head_dim 64 (the VALU kernel), on the same scratch.
    cases = [
        make_case(oracle, 32, 8, 128, 1899, 1930, 16, False, "tail", 701, k_outliers=True),
        make_case(oracle, 8, 2, 64, 40, 6, 16, True, "holes", 702),
    ]
    for i, case in enumerate(cases):
        print(f"noalloc call {i}: Hq={case[12]} Hkv={case[13]} D={case[14]} nd={case[3]} nb={case[11]}", flush=True)
        (o_ref, mw_ref), (o_na, mw_na) = _both(lib, _args(case))
        assert np.isfinite(o_ref).all()
        assert same_bits(o_na, o_ref), i
        assert same_bits(mw_na, mw_ref), i


def test_noalloc_rejects_oversized_call_on_host(lib):
    # 300k tokens x 32 heads of logits exceed the 32 MiB scratch: the call must
    # fail before enqueuing anything (the tier pointers are never read).
    t = torch.zeros(16, dtype=torch.float32, device="cuda")
    a = dict(Q=t, dK=t, dV=t, nd=0, KP=t, KS=t, KZ=t, VP=t, VS=t, VZ=t, ids=t, nb=300000 // 16, Hq=32, Hkv=8,
             D=128, kgs=16, fp16=0)
    rc = _call(lib.tt_fused_attention_decode_noalloc, a, t, t)
    assert rc == 1
    assert b"scratch" in lib.tt_last_error()
    # the workspace query agrees that this call is above the limit
    assert lib.tt_fused_attention_workspace_bytes(0, 300000 // 16, 32, 8, 128, 16, 1) > (32 << 20)
    torch.cuda.synchronize()


def test_noalloc_graph_replay_without_mean_weights_and_no_memory_growth(lib, oracle):
    """After a warm-up call, (1) calls with and without mean weights (NULL) leave the
    device's free memory unchanged, and (2) the call captured in a graph and replayed
    with new queries matches the allocating entry point bit for bit on every replay,
    with eager calls and synchronisations between the replays."""
    from oracle import synth

    case = make_case(oracle, 32, 8, 128, 300, 120, 16, False, "tail", 703)
    a = _args(case)
    n_tok = a["nd"] + a["nb"] * a["kgs"]
    out = torch.empty((a["Hq"], a["D"]), dtype=torch.float32, device="cuda")
    mw = torch.empty((n_tok,), dtype=torch.float32, device="cuda")
    assert _call(lib.tt_fused_attention_decode_noalloc, a, out, mw) == 0, lib.tt_last_error()
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    out2 = torch.empty_like(out)
    for m in (None, mw, None):
        assert _call(lib.tt_fused_attention_decode_noalloc, a, out2, m) == 0, lib.tt_last_error()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert same_bits(host(out2), host(out))  # the output does not depend on whether weights are asked for

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rc = lib.tt_fused_attention_decode_noalloc(
                _ptr(a["Q"]), _ptr(a["dK"]), _ptr(a["dV"]), a["nd"], _ptr(a["KP"]), _ptr(a["KS"]), _ptr(a["KZ"]),
                _ptr(a["VP"]), _ptr(a["VS"]), _ptr(a["VZ"]), _ptr(a["ids"]), a["nb"], a["Hq"], a["Hkv"], a["D"],
                _ptr(out), _ptr(mw), a["kgs"], a["fp16"], ctypes.c_void_p(s.cuda_stream))
    torch.cuda.current_stream().wait_stream(s)
    assert rc == 0, lib.tt_last_error()
    for r in range(3):
        a["Q"].copy_(dev(synth.normal(704 + r, 0, (a["Hq"], a["D"]))))
        out.fill_(float("nan"))
        mw.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got_out, got_mw = host(out), host(mw)
        (o_ref, mw_ref), (o_na, mw_na) = _both(lib, a)  # eager calls of both entry points between replays
        assert same_bits(got_out, o_ref) and same_bits(got_mw, mw_ref), r
        assert same_bits(o_na, o_ref) and same_bits(mw_na, mw_ref), r
    del g
    torch.cuda.synchronize()
