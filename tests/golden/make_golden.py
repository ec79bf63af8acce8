"""Writes the golden fixtures in tests/golden/ from the reference itself.

Run in a checkout that has the reference at /root/reference and the compiled
reference library oracle/_ref/libttref.so (``make -C oracle``):

    python tests/golden/make_golden.py

Outputs (data only):
  quantize_v_kat.json   the reference's own known-answer vectors, parsed from
                        its tests/test_quantize_v.cpp (1024 inputs, 32 min/scale
                        values at 1e-4, 64 packed words exact)
  tie_kat.json          the round-half-even case of its tests/tie_test_v.cpp,
                        with the full output of the compiled reference
  kernels_small.npz     quantize_k / quantize_v / dequantize / fused attention
                        inputs and outputs of the compiled reference
  engine_digests.json   per-checkpoint SHA-256 state digests of the compiled
                        reference engine for every run in tests/engine_runs.py
"""
from __future__ import annotations

import json
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import synth  # noqa: E402
from oracle.binding import load_reference  # noqa: E402
import engine_runs  # noqa: E402

REF_TESTS = "/root/reference/tests"


def _floats(block: str):
    return [float(x.rstrip("f")) for x in re.findall(r"-?\d+\.\d+(?:e[-+]?\d+)?f", block)]


def quantize_v_kat():
    src = open(os.path.join(REF_TESTS, "test_quantize_v.cpp")).read()

    def vec(name):
        m = re.search(r"std::vector<[^>]+>\s+" + name + r"\s*=\s*\{(.*?)\};", src, re.S)
        return m.group(1)

    V = _floats(vec("V"))
    mins = _floats(vec("expected_min"))
    scales = _floats(vec("expected_scale"))
    packed = [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{8})u", vec("expected_packed"))]
    assert len(V) == 1024 and len(mins) == 32 and len(scales) == 32 and len(packed) == 64
    return {
        "source": "reference tests/test_quantize_v.cpp:10-13 (num_heads=2, head_dim=32, chunk 16)",
        "num_heads": 2, "head_dim": 32, "chunk_size": 16, "tolerance_min_scale": 1e-4,
        "V": V, "expected_min": mins, "expected_scale": scales, "expected_packed": packed,
    }


def tie_kat(R):
    # reference tests/tie_test_v.cpp:8-16: one head, head_dim 16, every value 3.0
    # except token 0 channels 0,1,2,3,10 = 0,6,1,3,5 -> scale 2, normalised
    # 0.5 -> 0, 1.5 -> 2, 2.5 -> 2 under round-half-even.
    V = np.full((16, 1, 16), 3.0, np.float32)
    V[0, 0, 0], V[0, 0, 1], V[0, 0, 2], V[0, 0, 3], V[0, 0, 10] = 0.0, 6.0, 1.0, 3.0, 5.0
    p, s, z = R.quantize_v(V, fp16=False)
    w = int(np.uint32(p.reshape(-1)[0]))
    q = [(w >> (2 * c)) & 3 for c in range(16)]
    assert s[0, 0] == 2.0 and q[2] == 0 and q[3] == 2 and q[10] == 2
    return {
        "source": "reference tests/tie_test_v.cpp:8-16",
        "V": V.reshape(-1).tolist(), "num_heads": 1, "head_dim": 16, "expected_scale0": 2.0,
        "expected_q": {"2": 0, "3": 2, "10": 2},
        "reference_packed": [int(x) for x in p.reshape(-1).view(np.uint32)],
        "reference_scale": s.reshape(-1).tolist(), "reference_zero": z.reshape(-1).tolist(),
    }


QK_CASES = [dict(H=2, D=32, kgs=16, fp16=False), dict(H=3, D=64, kgs=32, fp16=True),
            dict(H=2, D=8, kgs=16, fp16=False), dict(H=1, D=12, kgs=16, fp16=False),
            dict(H=4, D=128, kgs=16, fp16=True)]
QV_CASES = [dict(H=2, D=32, chunk=16, fp16=False), dict(H=4, D=64, chunk=16, fp16=True),
            dict(H=1, D=16, chunk=32, fp16=False), dict(H=2, D=128, chunk=16, fp16=True),
            # rows holding NaN, +-inf and signed zeros (the min/max fold order decides them)
            dict(H=2, D=64, chunk=16, fp16=False, special=True), dict(H=3, D=128, chunk=16, fp16=True, special=True)]
FA_CASES = [dict(Hq=4, Hkv=2, D=64, nd=20, nb=3, kgs=16, fp16=False, masked=3),
            dict(Hq=8, Hkv=8, D=128, nd=5, nb=7, kgs=16, fp16=True, masked=0),
            dict(Hq=4, Hkv=4, D=16, nd=3, nb=2, kgs=32, fp16=True, masked=5),
            dict(Hq=7, Hkv=1, D=128, nd=0, nb=4, kgs=16, fp16=False, masked=14),
            dict(Hq=4, Hkv=2, D=64, nd=10, nb=0, kgs=16, fp16=False, masked=0),
            dict(Hq=6, Hkv=2, D=32, nd=33, nb=5, kgs=16, fp16=True, masked=1)]


def _special_k(K):
    """Plant edge cases: a constant channel (scale floor), exact .5 ties, signed zeros."""
    K = K.copy()
    kgs, H, D = K.shape
    K[:, 0, 0] = 1.25
    if D > 3:
        K[:, 0, 1] = np.linspace(0.0, 3.0, kgs, dtype=np.float32)
        K[:, 0, 2] = 0.0
        K[::2, 0, 2] = -0.0
    return K


def _special_v(V):
    """Rows of head 0 with the values whose handling depends on the order of the
    quantiser's min/max fold and conversions: signed zeros, NaN, infinities."""
    V = V.copy()
    D = V.shape[2]
    V[1, 0, :] = 0.0
    V[1, 0, 5::16] = -0.0
    V[2, 0, :] = -0.0
    V[2, 0, D // 2] = 0.0
    V[3, 0, 37 % D] = np.nan
    V[4, 0, 9] = np.inf
    V[5, 0, 3] = -np.inf
    V[6, 0, ::9] = np.nan
    V[6, 0, 4] = 0.0
    V[7, 0, 0] = np.inf
    V[7, 0, D - 1] = -np.inf
    V[8, 0, :8] = np.nan      # a whole 8-channel chunk NaN
    V[9, 0, :] = np.nan       # every channel NaN
    V[10, 0, 8:16] = -0.0     # a chunk of -0 after a chunk of finite values
    return V


def build_quantized_blocks(R, K, V, kgs, fp16):
    """Pack token-major K/V [nb*kgs, H, D] with the reference quantisers."""
    nb = K.shape[0] // kgs
    KP, KS, KZ, VP, VS, VZ = [], [], [], [], [], []
    for b in range(nb):
        p, s, z = R.quantize_k(K[b * kgs:(b + 1) * kgs], kgs, fp16)
        KP.append(p); KS.append(s); KZ.append(z)
        p, s, z = R.quantize_v(V[b * kgs:(b + 1) * kgs], fp16)
        VP.append(p); VS.append(s); VZ.append(z)
    return (np.stack(KP), np.stack(KS), np.stack(KZ), np.concatenate(VP), np.concatenate(VS), np.concatenate(VZ))


def kernels_small(R):
    out = {}
    index = {"qk": QK_CASES, "qv": QV_CASES, "fa": FA_CASES}
    for i, c in enumerate(QK_CASES):
        K = _special_k(synth.normal(100 + i, 0, (c["kgs"], c["H"], c["D"]), std=1.5))
        p, s, z = R.quantize_k(K, c["kgs"], c["fp16"])
        dq = R.dequantize_k(p, s, z, 1, c["H"], c["D"], c["kgs"], c["fp16"])
        out.update({f"qk{i}_K": K, f"qk{i}_packed": p, f"qk{i}_scale": s, f"qk{i}_zero": z, f"qk{i}_deq": dq})
    for i, c in enumerate(QV_CASES):
        V = synth.normal(200 + i, 0, (c["chunk"], c["H"], c["D"]))
        V[0, 0, :] = 0.75  # constant row -> scale floor
        if c.get("special"):
            V = _special_v(V)
        p, s, z = R.quantize_v(V, c["fp16"])
        dq = R.dequantize_v(p, s, z, c["chunk"], c["H"], c["D"], c["fp16"])
        out.update({f"qv{i}_V": V, f"qv{i}_packed": p, f"qv{i}_scale": s, f"qv{i}_zero": z, f"qv{i}_deq": dq})
    for i, c in enumerate(FA_CASES):
        Hq, Hkv, D, nd, nb, kgs = c["Hq"], c["Hkv"], c["D"], c["nd"], c["nb"], c["kgs"]
        Q = synth.normal(300 + i, 0, (Hq, D))
        dK = synth.normal(300 + i, 1, (nd, Hkv, D))
        dV = synth.normal(300 + i, 2, (nd, Hkv, D))
        Kp = synth.normal(300 + i, 3, (max(nb, 1) * kgs, Hkv, D))
        Vp = synth.normal(300 + i, 4, (max(nb, 1) * kgs, Hkv, D))
        blocks = build_quantized_blocks(R, Kp, Vp, kgs, c["fp16"])
        ids = np.arange(max(nb, 1) * kgs, dtype=np.int64) + nd
        if c["masked"]:
            ids[-c["masked"]:] = -1
        o, mw = R.fused_attention_decode(Q, dK, dV, nd, *blocks, ids, nb, Hq, Hkv, D, kgs, c["fp16"])
        out.update({f"fa{i}_Q": Q, f"fa{i}_dK": dK, f"fa{i}_dV": dV, f"fa{i}_KP": blocks[0], f"fa{i}_KS": blocks[1],
                    f"fa{i}_KZ": blocks[2], f"fa{i}_VP": blocks[3], f"fa{i}_VS": blocks[4], f"fa{i}_VZ": blocks[5],
                    f"fa{i}_ids": ids, f"fa{i}_out": o, f"fa{i}_mw": mw})
    return out, index


def run_engine(impl, cfg):
    """Drive `impl` (oracle or reference CpuImpl) through a run; return digests."""
    e = impl.engine(*engine_runs.engine_args(cfg))
    if cfg["prefill"]:
        Kp, Vp = engine_runs.prefill_inputs(cfg)
        e.prefill(Kp, Vp)
    digests = {}
    for s in range(cfg["steps"]):
        Q, K, V = engine_runs.step_inputs(cfg, s)
        if cfg["mode"] == "step":
            e.step(Q, K, V)
        else:
            e.ingest(K, V)
            e.feedback(engine_runs.inject_weights(cfg, s, e.visible()))
        if engine_runs.is_checkpoint(cfg, s):
            st = e.state()
            digests[str(s)] = synth.state_digest(st["counters"], st)
    return digests, e.counters()


def main():
    R = load_reference()
    if R is None:
        raise SystemExit("oracle/_ref/libttref.so is missing: run `make -C oracle` where the reference exists")
    with open(os.path.join(HERE, "quantize_v_kat.json"), "w") as f:
        json.dump(quantize_v_kat(), f)
    with open(os.path.join(HERE, "tie_kat.json"), "w") as f:
        json.dump(tie_kat(R), f)
    arrays, index = kernels_small(R)
    np.savez_compressed(os.path.join(HERE, "kernels_small.npz"), **arrays)
    with open(os.path.join(HERE, "kernels_small.json"), "w") as f:
        json.dump(index, f, indent=1)
    runs = {}
    for name, cfg in engine_runs.RUNS.items():
        d, counters = run_engine(R, cfg)
        runs[name] = {"config": cfg, "digests": d, "final_counters": counters}
        print(name, counters["hh_count"], counters["pbs_blocks_used"], counters["wr_count"], flush=True)
    with open(os.path.join(HERE, "engine_digests.json"), "w") as f:
        json.dump(runs, f, indent=1)


if __name__ == "__main__":
    main()
