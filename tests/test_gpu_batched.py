"""GPU parity of the batched ragged decode (tt_fused_attention_decode_batched) against the oracle.

Every sequence of a batch has its own tier tables and lengths; its output and
mean weights must match the oracle's fused_attention_decode of that sequence
alone, to the single-sequence bar: max|gpu - ref| / max|ref| <= 1e-4.
"""
import ctypes as Ct

import numpy as np
import pytest
import torch

from gpu_helpers import dev, host, make_case, rel_err

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-4


@pytest.fixture(scope="module")
def C():
    assert torch.cuda.is_available(), "GPU test on a machine without a GPU"
    from tritiercache_amd import _C

    assert _C.device_count() > 0
    return _C


def _entry(args, want_mw=True):
    (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16) = args
    out = torch.full((Hq, D), float("nan"), dtype=torch.float32, device="cuda")
    mw = torch.full((nd + nb * kgs,), float("nan"), dtype=torch.float32, device="cuda") if want_mw else None
    e = {"Q": dev(Q), "dense_count": nd, "num_blocks": nb, "attn_output": out, "mean_attn_weights": mw}
    if nd:
        e["dense_K"], e["dense_V"] = dev(dK), dev(dV)
    if nb:
        e.update(PBS_K_Packed=dev(KP), PBS_K_Scales=dev(KS), PBS_K_Zeroes=dev(KZ), PBS_V_Packed=dev(VP),
                 PBS_V_Scales=dev(VS), PBS_V_Zeroes=dev(VZ), PBS_token_ids=dev(ids))
    return e


def _check(oracle, cases, entries, want):
    for i, (args, e) in enumerate(zip(cases, entries)):
        ro, rmw = oracle.fused_attention_decode(*args)
        out = host(e["attn_output"])
        assert rel_err(out, ro) <= ATTN_TOL, (i, args[3], args[11])
        if want[i]:
            assert rel_err(host(e["mean_attn_weights"]), rmw) <= ATTN_TOL, (i, args[3], args[11])


def _ragged(oracle, Hq, Hkv, D, kgs, fp16, sizes, seed, masks=("none", "tail", "holes", "block")):
    return [make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, masks[i % len(masks)], seed=seed + i, k_outliers=i % 2 == 0)
            for i, (nd, nb) in enumerate(sizes)]


# (nd, nb) per sequence: FP32-only, packed-only, one block, long and short mixed
RAGGED = [(260, 40), (0, 35), (300, 0), (17, 1), (120, 130), (5, 3), (64, 64), (270, 90)]


@pytest.mark.parametrize("Hq,Hkv,kgs,fp16", [(32, 8, 16, False), (32, 8, 16, True), (28, 4, 16, False),
                                            (16, 2, 32, False), (8, 8, 16, True), (12, 2, 16, True),
                                            (6, 2, 16, False), (28, 4, 32, True), (16, 8, 16, False)])
def test_batched_ragged_vs_oracle(C, oracle, Hq, Hkv, kgs, fp16):
    cases = _ragged(oracle, Hq, Hkv, 128, kgs, fp16, RAGGED, seed=1000 + Hq + kgs)
    entries = [_entry(a) for a in cases]
    C.fused_attention_decode_batched(entries, Hq, Hkv, 128, kgs, "fp16" if fp16 else "fp32")
    torch.cuda.synchronize()
    _check(oracle, cases, entries, [True] * len(cases))


def test_batched_mixed_mean_weights(C, oracle):
    """Sequences without mean weights next to sequences with them."""
    cases = _ragged(oracle, 32, 8, 128, 16, False, RAGGED[:5], seed=1100)
    want = [True, False, True, False, False]
    entries = [_entry(a, w) for a, w in zip(cases, want)]
    C.fused_attention_decode_batched(entries, 32, 8, 128)
    torch.cuda.synchronize()
    _check(oracle, cases, entries, want)


def test_batched_more_sequences_than_one_launch(C, oracle):
    """70 sequences: two launches of at most 64 sharing the workspace."""
    rng = np.random.default_rng(7)
    sizes = [(int(rng.integers(0, 40)), int(rng.integers(1, 6))) for _ in range(70)]
    cases = _ragged(oracle, 8, 2, 128, 16, False, sizes, seed=1200)
    entries = [_entry(a) for a in cases]
    C.fused_attention_decode_batched(entries, 8, 2, 128)
    torch.cuda.synchronize()
    _check(oracle, cases, entries, [True] * len(cases))


@pytest.mark.parametrize("D", [64, 256])
def test_batched_other_head_dims(C, oracle, D):
    """head_dim != 128 runs the sequences one after another through the single-sequence path."""
    cases = _ragged(oracle, 8, 2, D, 16, False, [(20, 6), (0, 9), (33, 0)], seed=1300 + D)
    entries = [_entry(a) for a in cases]
    C.fused_attention_decode_batched(entries, 8, 2, D)
    torch.cuda.synchronize()
    _check(oracle, cases, entries, [True] * len(cases))


def test_batched_equals_single_sequence_calls(C, oracle):
    """The batched result of a sequence equals its single-sequence result to the tolerance, at a longer context."""
    cases = _ragged(oracle, 32, 8, 128, 16, False, [(1899, 300), (700, 1000), (260, 125)], seed=1400)
    entries = [_entry(a) for a in cases]
    C.fused_attention_decode_batched(entries, 32, 8, 128)
    for args, e in zip(cases, entries):
        (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16) = args
        out = torch.empty((Hq, D), device="cuda")
        mw = torch.empty((nd + nb * kgs,), device="cuda")
        C.fused_attention_decode(dev(Q), dev(dK), dev(dV), nd, dev(KP), dev(KS), dev(KZ), dev(VP), dev(VS), dev(VZ),
                                 dev(ids), nb, Hq, Hkv, D, out, mw, kgs, "fp32")
        torch.cuda.synchronize()
        assert rel_err(host(e["attn_output"]), host(out)) <= ATTN_TOL
        assert rel_err(host(e["mean_attn_weights"]), host(mw)) <= ATTN_TOL


@pytest.mark.parametrize("fp16", [False, True])
def test_batched_device_filling_plan_with_one_tier_sequences(C, oracle, fp16):
    """Enough work to fill the device (packed slots of all sequences launched before all FP32-tier slots), with
    sequences that have no FP32 tokens or no packed blocks between the others: each sequence's slots are found
    through the packed and FP32 prefix tables, where a sequence without FP32 tokens repeats its predecessor's
    FP32 offset."""
    sizes = [(0, 800), (260, 400), (0, 300), (300, 0), (40, 520), (0, 1), (1000, 64)]
    cases = _ragged(oracle, 32, 8, 128, 16, fp16, sizes, seed=1500 + fp16)
    entries = [_entry(a) for a in cases]
    C.fused_attention_decode_batched(entries, 32, 8, 128, 16, "fp16" if fp16 else "fp32")
    torch.cuda.synchronize()
    _check(oracle, cases, entries, [True] * len(cases))


def test_batched_errors(C, oracle):
    from tritiercache_amd import _lib

    L = _lib.load()
    args = make_case(oracle, 8, 2, 128, 10, 2, 16, False, "none", seed=3)
    e = _entry(args)
    with pytest.raises(ValueError):
        C.fused_attention_decode_batched([dict(e, attn_output=None)], 8, 2, 128)
    with pytest.raises(ValueError):
        C.fused_attention_decode_batched([dict(e, dense_count=-1)], 8, 2, 128)
    with pytest.raises(ValueError):
        C.fused_attention_decode_batched([e], 7, 2, 128)  # GQA ratio not integral
    seqs = (_lib.DecodeSeq * 1)()
    s = seqs[0]
    s.Q, s.dense_K, s.dense_V = e["Q"].data_ptr(), e["dense_K"].data_ptr(), e["dense_V"].data_ptr()
    s.PBS_K_Packed, s.PBS_K_Scales, s.PBS_K_Zeroes = (e["PBS_K_Packed"].data_ptr(), e["PBS_K_Scales"].data_ptr(),
                                                      e["PBS_K_Zeroes"].data_ptr())
    s.PBS_V_Packed, s.PBS_V_Scales, s.PBS_V_Zeroes = (e["PBS_V_Packed"].data_ptr(), e["PBS_V_Scales"].data_ptr(),
                                                      e["PBS_V_Zeroes"].data_ptr())
    s.PBS_token_ids, s.attn_output = e["PBS_token_ids"].data_ptr(), e["attn_output"].data_ptr()
    s.dense_count, s.num_blocks = 10, 2
    need = int(L.tt_batched_decode_workspace_bytes(seqs, 1, 8, 2, 128, 16))
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    stream = Ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    # workspace too small, no device copy of the descriptors
    assert L.tt_fused_attention_decode_batched(seqs, None, 1, 8, 2, 128, 16, 0, ws.data_ptr(), need - 1, stream) == 1
    assert L.tt_fused_attention_decode_batched(seqs, None, 1, 8, 2, 128, 16, 0, ws.data_ptr(), need, stream) == 1
    # an empty batch is a no-op
    assert L.tt_fused_attention_decode_batched(seqs, None, 0, 8, 2, 128, 16, 0, ws.data_ptr(), need, stream) == 0
    torch.cuda.synchronize()
