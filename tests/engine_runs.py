"""Engine workloads shared by the golden-fixture generator and the parity tests.

Each run drives an engine for a number of steps with inputs from
oracle.synth. Mode "step" runs the full decode step (attention included);
mode "inject" runs only the tier maintenance (ingest) and feeds the decayed
score update with synthetic per-token weights, softmax of N(0, 2^2) logits
over the visible set -- the tier-maintenance workload at 32 KV heads x 128,
a 256-token ring and 4 sinks over 2048 appends.
"""
from __future__ import annotations

import numpy as np

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
    # head_dims that are multiples of 16 but not powers of two (the VALU kernel with
    # lane channel ranges straddling V words; the flush's V rows on padded lane groups)
    "step_d80_fp16": dict(mode="step", Hq=6, Hkv=2, D=80, msl=1024, S=4, R=16, hr=0.1, decay=0.999, iv=16,
                          kgs=16, fp16=True, steps=200, prefill=64, seed=17, every=40),
    "step_d96_kgs32_fp32": dict(mode="step", Hq=12, Hkv=4, D=96, msl=1024, S=4, R=16, hr=0.1, decay=0.999,
                                iv=32, kgs=32, fp16=False, steps=200, prefill=40, seed=18, every=40),
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


# Heavy-hitter argmin with tied scores (cache_engine.cpp:224-232: first slot of
# the minimum under '<'). Tier maintenance with injected weights and no score
# decay, so scores are sums of equal increments added in the same order and
# many slots share the minimum.
#  * "small": weight 1e-3 on every second dense position (sinks, heavy hitters,
#    recent window), none on the packed store; the tier (60 slots) fills and
#    its first minimal slot is replaced now and then;
#  * "large": no weights for 40 steps (the first threshold is then 0, and with
#    an update interval past the run it stays 0, so every eviction is promoted),
#    then 1e-3 x ((s + j) % 3) on recent-window position j; the tier fills all
#    8750 slots, beyond the 8192 scores one pass of the GPU scan covers, and
#    positive-score evictions replace its zero-score slots in order.
TIE_RUNS = {
    "small": dict(args=(2, 1, 16, 1200, 4, 16, 0.05, 1.0, 16, 16), steps=1100, checkpoints=tuple(range(99, 1100, 100))),
    "large": dict(args=(2, 1, 16, 17500, 4, 16, 0.5, 1.0, 1 << 30, 16), steps=9100, checkpoints=(8768, 8900, 9099)),
}


def tie_kv(s: int):
    return synth.normal(71, 2 * s, (16,)), synth.normal(71, 2 * s + 1, (16,))


def tie_weights(run: str, counters: dict, n: int, s: int):
    w = np.zeros(n, np.float32)
    ring0 = counters["s_count"] + counters["hh_count"]
    nd = ring0 + counters["rw_count"]
    if run == "small":
        w[:nd:2] = 1e-3
    elif s >= 40:
        w[ring0:nd] = 1e-3 * ((s + np.arange(nd - ring0)) % 3)
    return w
