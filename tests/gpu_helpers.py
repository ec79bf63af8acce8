"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch

from oracle import synth


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.uint16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def rel_err(got, want) -> float:
    """max |got - want| / max |want| -- the tolerance metric for FP32 outputs."""
    want = np.asarray(want, np.float64)
    denom = max(float(np.abs(want).max()), 1e-30)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / denom)


def same_bits(a, b) -> bool:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    if a.nbytes == 0 and b.nbytes == 0:
        return True
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


_GETTERS = {
    "S_K": "get_S_K", "S_V": "get_S_V", "RW_K": "get_RW_K", "RW_V": "get_RW_V", "HH_K": "get_HH_K",
    "HH_V": "get_HH_V", "HH_token_ids": "get_HH_token_ids", "HH_scores": "get_HH_scores", "WR_K": "get_WR_K",
    "WR_V": "get_WR_V", "WR_token_ids": "get_WR_token_ids", "PBS_K_Packed": "get_PBS_K_Packed",
    "PBS_K_Scales": "get_PBS_K_Scales", "PBS_K_Zeroes": "get_PBS_K_Zeroes", "PBS_V_Packed": "get_PBS_V_Packed",
    "PBS_V_Scales": "get_PBS_V_Scales", "PBS_V_Zeroes": "get_PBS_V_Zeroes", "PBS_token_ids": "get_PBS_token_ids",
    "global_attn_scores": "get_global_attn_scores",
}


def gpu_engine_state(eng) -> dict:
    """Counters plus flat host copies of every tier buffer, in the layout of
    oracle.binding.CpuEngine.state()."""
    st = {"counters": eng.counters()}
    for name, getter in _GETTERS.items():
        st[name] = host(getattr(eng, getter)()).reshape(-1)
    return st


def gpu_state_digest(eng) -> str:
    st = gpu_engine_state(eng)
    return synth.state_digest(st["counters"], st)


def quantize_blocks_gpu(C, K: torch.Tensor, V: torch.Tensor, kgs: int, fp16: bool):
    """Pack token-major device K/V [nb*kgs, H, D] into the reference PBS layout."""
    n, H, D = K.shape
    nb = n // kgs
    mdt = torch.uint16 if fp16 else torch.float32
    dt = "fp16" if fp16 else "fp32"
    KP = torch.empty((nb, kgs // 16, H, D), dtype=torch.int32, device="cuda")
    KS = torch.empty((nb, H, D), dtype=mdt, device="cuda")
    KZ = torch.empty((nb, H, D), dtype=mdt, device="cuda")
    VP = torch.empty((nb * kgs, H, D // 16), dtype=torch.int32, device="cuda")
    VS = torch.empty((nb * kgs, H, 1), dtype=mdt, device="cuda")
    VZ = torch.empty((nb * kgs, H, 1), dtype=mdt, device="cuda")
    C.quantize_k_blocks(K, KP, KS, KZ, nb, H, D, kgs, dt)
    C.quantize_v_block(V, VP, VS, VZ, H, D, nb * kgs, dt)
    return KP, KS, KZ, VP, VS, VZ


def make_case(oracle, Hq, Hkv, D, nd, nb, kgs, fp16, mask, seed, k_outliers=False):
    Q = synth.normal(seed, 0, (Hq, D))
    dK, dV = synth.normal(seed, 1, (nd, Hkv, D)), synth.normal(seed, 2, (nd, Hkv, D))
    nbk = max(nb, 1)
    Kp, Vp = synth.normal(seed, 3, (nbk * kgs, Hkv, D)), synth.normal(seed, 4, (nbk * kgs, Hkv, D))
    if k_outliers:
        Kp[:, :, :4] *= 8.0
        dK[:, :, :4] *= 8.0
    packs = [(oracle.quantize_k(Kp[b * kgs:(b + 1) * kgs], kgs, fp16), oracle.quantize_v(Vp[b * kgs:(b + 1) * kgs], fp16))
             for b in range(nbk)]
    KP = np.stack([k[0] for k, _ in packs])
    KS = np.stack([k[1] for k, _ in packs])
    KZ = np.stack([k[2] for k, _ in packs])
    VP = np.concatenate([v[0] for _, v in packs])
    VS = np.concatenate([v[1] for _, v in packs])
    VZ = np.concatenate([v[2] for _, v in packs])
    ids = np.arange(nbk * kgs, dtype=np.int64) + nd
    rng = np.random.default_rng(seed)
    if mask == "tail":
        ids[-(kgs // 2 + 3):] = -1
    elif mask == "holes":
        ids[rng.random(ids.size) < 0.2] = -1
    elif mask == "block":
        ids[:kgs] = -1
    elif mask == "all":
        ids[:] = -1
    return (Q, dK, dV, nd, KP, KS, KZ, VP, VS, VZ, ids, nb, Hq, Hkv, D, kgs, fp16)


def compare_state(g: dict, o: dict, tag) -> None:
    """Counters and every tier buffer of a GPU engine (gpu_engine_state) equal the
    oracle engine's (CpuEngine.state()), bit for bit."""
    assert g["counters"] == o["counters"], (tag, g["counters"], o["counters"])
    for name in o:
        if name != "counters":
            assert same_bits(g[name], o[name].reshape(-1)), (tag, name)


def attention_errors(out, ro, mw=None, rmw=None) -> dict:
    """Errors of a GPU step's output (and mean weights) against the oracle's: the
    max-normwise error, and the elementwise ratio with 1e-5 max|ref| of absolute
    slack (the float32 oracle's own sequential sums sit about 1e-6 max|ref| from
    exact attention, see oracle.exact)."""
    from oracle.exact import elementwise_ratio, weights_rel_err

    r = {"norm": rel_err(out, ro), "elem": elementwise_ratio(out, ro, atol_frac=1e-5)}
    if mw is not None:
        r["mw_norm"] = rel_err(mw, rmw)
        r["mw_rel"] = weights_rel_err(mw, rmw)
    return r


def attention_ok(r: dict, tol: float = 1e-4) -> bool:
    return (r["norm"] <= tol and r["elem"] <= 1.0 and r.get("mw_norm", 0.0) <= tol
            and r.get("mw_rel", 0.0) <= tol)


class Lockstep:
    """An oracle engine driven beside a GPU engine: the same prefill and step
    inputs, and after every GPU step the GPU's mean attention weights as the
    oracle's score feedback (score-injected lockstep). Tier membership, packed
    words, scales/zeros and scores must then stay bit-identical, while the
    attention outputs are compared to the tolerance."""

    def __init__(self, oracle, Hq, Hkv, D, msl, S, R, hr, decay, iv, kgs, fp16):
        self.oe = oracle.engine(Hq, Hkv, D, msl, S, R, hr, decay, iv, kgs, fp16)

    def prefill(self, K, V) -> None:
        self.oe.prefill(np.ascontiguousarray(K, np.float32), np.ascontiguousarray(V, np.float32))

    def step(self, Q, K, V, out, mw, attend=True):
        """The oracle's side of one GPU step (host arrays); returns attention_errors
        of `out` / `mw` when `attend`."""
        self.oe.ingest(K, V)
        r = None
        if attend:
            ro, rmw = self.oe.attend(Q)
            r = attention_errors(out, ro, mw, rmw)
        self.oe.feedback(mw)
        return r

    def check_state(self, eng, tag) -> None:
        compare_state(gpu_engine_state(eng), self.oe.state(), tag)
