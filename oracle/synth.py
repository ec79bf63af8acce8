"""Deterministic synthetic inputs and state digests for the oracle (test infrastructure only).

Inputs come from a counter-based generator of our own (splitmix64 over
(seed, stream, index)) so fixtures do not depend on numpy's or torch's RNG
streams: uniform(0,1) from the top 53 bits, normal via Box-Muller in float64
then rounded to float32, Student-t(3) as Z / sqrt(chi2_3 / 3).
"""
from __future__ import annotations

import hashlib

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_C1 = np.uint64(0xBF58476D1CE4E5B9)
_C2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _C1
    z = (z ^ (z >> np.uint64(27))) * _C2
    return z ^ (z >> np.uint64(31))


def _key(seed: int, stream: int) -> np.uint64:
    k = _mix(np.array([(seed * 0x100000001B3 + stream * 0xC2B2AE3D27D4EB4F + 1) & 0xFFFFFFFFFFFFFFFF],
                      dtype=np.uint64))
    return k[0]


def uniform(seed: int, stream: int, n: int) -> np.ndarray:
    """n float64 values in (0, 1)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = _mix(_key(seed, stream) + i * _GOLDEN)
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed: int, stream: int, shape, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = uniform(seed, stream, 2 * m)
    r = np.sqrt(-2.0 * np.log(u[:m]))
    t = 2.0 * np.pi * u[m:]
    z = np.concatenate([r * np.cos(t), r * np.sin(t)])[:n]
    return (z * std).astype(np.float32).reshape(shape)


def student_t3(seed: int, stream: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    z = normal(seed, stream, (n,)).astype(np.float64)
    c = normal(seed, stream + 1, (3, n)).astype(np.float64)
    chi2 = (c * c).sum(axis=0)
    return (z / np.sqrt(chi2 / 3.0)).astype(np.float32).reshape(shape)


def softmax_weights(seed: int, stream: int, n: int, sigma: float = 2.0) -> np.ndarray:
    """Per-token attention weights: softmax of N(0, sigma^2) logits (float32, sum 1)."""
    if n <= 0:
        return np.zeros(0, np.float32)
    lg = normal(seed, stream, (n,)).astype(np.float64) * sigma
    w = np.exp(lg - lg.max())
    return (w / w.sum()).astype(np.float32)


COUNTERS_FOR_DIGEST = (
    "s_count", "rw_count", "rw_head_index", "hh_count", "wr_count", "pbs_allocated_blocks", "pbs_blocks_used",
    "pbs_count", "total_processed_tokens", "last_calc_pos", "total_evictions",
)
BUFFERS_FOR_DIGEST = (
    "S_K", "S_V", "RW_K", "RW_V", "HH_K", "HH_V", "HH_token_ids", "HH_scores", "WR_K", "WR_V", "WR_token_ids",
    "PBS_K_Packed", "PBS_K_Scales", "PBS_K_Zeroes", "PBS_V_Packed", "PBS_V_Scales", "PBS_V_Zeroes",
    "PBS_token_ids", "global_attn_scores",
)


def state_digest(counters: dict, buffers: dict) -> str:
    """SHA-256 over the data-dependent counters and the raw bytes of every tier
    buffer (logical sizes), in a fixed order."""
    h = hashlib.sha256()
    h.update(np.array([counters[k] for k in COUNTERS_FOR_DIGEST], dtype=np.int64).tobytes())
    for name in BUFFERS_FOR_DIGEST:
        a = np.ascontiguousarray(buffers[name])
        h.update(name.encode())
        h.update(np.int64(a.nbytes).tobytes())
        h.update(a.view(np.uint8).tobytes())
    return h.hexdigest()
