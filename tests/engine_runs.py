"""Engine workloads shared by the golden-fixture generator and the parity tests.

Each run drives an engine for a number of steps with inputs from
oracle.synth. Mode "step" runs the full decode step (attention included);
mode "inject" runs only the tier maintenance (ingest) and feeds the decayed
score update with synthetic per-token weights, softmax of N(0, 2^2) logits
over the visible set -- the tier-maintenance workload at 32 KV heads x 128,
a 256-token ring and 4 sinks over 2048 appends.
"""
from __future__ import annotations

from oracle import synth

RUNS = {
    "step_small_fp16": dict(mode="step", Hq=4, Hkv=2, D=64, msl=512, S=4, R=16, hr=0.1, decay=0.999, iv=32,
                            kgs=16, fp16=True, steps=300, prefill=0, seed=11, every=25),
    "step_prefill_kgs32_fp32": dict(mode="step", Hq=4, Hkv=2, D=64, msl=1024, S=4, R=16, hr=0.1, decay=0.999,
                                    iv=16, kgs=32, fp16=False, steps=200, prefill=96, seed=12, every=25),
    "step_gqa_d128_fp32": dict(mode="step", Hq=8, Hkv=2, D=128, msl=1024, S=4, R=32, hr=0.05, decay=0.999, iv=32,
                               kgs=16, fp16=False, steps=400, prefill=50, seed=13, every=50),
    # f16 metadata (the reference engine's default) on the matrix-core path: four-head
    # groups with 16-token blocks, seven-head groups (padded to eight) with 32-token blocks
    "step_gqa_d128_fp16": dict(mode="step", Hq=8, Hkv=2, D=128, msl=1024, S=4, R=32, hr=0.05, decay=0.999, iv=32,
                               kgs=16, fp16=True, steps=300, prefill=64, seed=15, every=50),
    "step_gqa7_d128_kgs32_fp16": dict(mode="step", Hq=14, Hkv=2, D=128, msl=1024, S=4, R=32, hr=0.05, decay=0.999,
                                      iv=16, kgs=32, fp16=True, steps=200, prefill=40, seed=16, every=50),
    # long prefill: thresholds over ~36k candidates (the many-workgroup selection on the GPU)
    "step_long_prefill_fp32": dict(mode="step", Hq=4, Hkv=1, D=64, msl=36200, S=4, R=32, hr=0.05, decay=0.999,
                                   iv=32, kgs=16, fp16=False, steps=70, prefill=36000, seed=14, every=32),
    "inject_maint_fp16": dict(mode="inject", Hq=32, Hkv=32, D=128, msl=2048, S=4, R=256, hr=0.05, decay=0.999,
                              iv=32, kgs=16, fp16=True, steps=2048, prefill=0, seed=2, every=128),
    "inject_maint_fp32": dict(mode="inject", Hq=32, Hkv=32, D=128, msl=2048, S=4, R=256, hr=0.05, decay=0.999,
                              iv=32, kgs=16, fp16=False, steps=2048, prefill=0, seed=3, every=128),
}


def step_inputs(cfg: dict, s: int):
    seed = cfg["seed"]
    kvs = cfg["Hkv"] * cfg["D"]
    K = synth.normal(seed, 1_000_000 + 2 * s, (kvs,))
    V = synth.normal(seed, 1_000_001 + 2 * s, (kvs,))
    Q = synth.normal(seed, 3_000_000 + s, (cfg["Hq"] * cfg["D"],))
    return Q, K, V


def prefill_inputs(cfg: dict):
    shape = (cfg["prefill"], cfg["Hkv"], cfg["D"])
    return synth.normal(cfg["seed"], 1, shape), synth.normal(cfg["seed"], 2, shape)


def inject_weights(cfg: dict, s: int, visible: int):
    return synth.softmax_weights(cfg["seed"], 5_000_000 + s, visible, sigma=2.0)


def is_checkpoint(cfg: dict, s: int) -> bool:
    return (s + 1) % cfg["every"] == 0 or s + 1 == cfg["steps"]


def engine_args(cfg: dict):
    return (cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["msl"], cfg["S"], cfg["R"], cfg["hr"], cfg["decay"], cfg["iv"],
            cfg["kgs"], cfg["fp16"])
