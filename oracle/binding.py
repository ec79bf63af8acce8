"""ctypes bindings for the oracle libraries (test infrastructure only).

Two implementations share one Python surface:

* ``load_oracle()``    -> oracle/libtt_oracle.so, the C restatement (tt_oracle.c)
* ``load_reference()`` -> oracle/_ref/libttref.so, the reference's own C++
                          sources compiled by oracle/Makefile (absent where the
                          reference checkout was not available at build time)

All arrays are host numpy arrays. Nothing here touches a GPU.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_HERE, "libtt_oracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libttref.so")

N_COUNTERS = 23
COUNTER_NAMES = (
    "num_q_heads", "num_kv_heads", "head_dim", "max_seq_len", "sink_size", "rw_size",
    "update_interval", "k_group_size", "chunk_size", "quant_head_dim", "max_hh",
    "use_fp16_meta", "s_count", "rw_count", "rw_head_index", "hh_count", "wr_count",
    "pbs_allocated_blocks", "pbs_blocks_used", "pbs_count", "total_processed_tokens",
    "last_calc_pos", "total_evictions",
)
BUFFER_NAMES = (
    "S_K", "S_V", "RW_K", "RW_V", "HH_K", "HH_V", "HH_token_ids", "HH_scores", "WR_K", "WR_V",
    "WR_token_ids", "PBS_K_Packed", "PBS_K_Scales", "PBS_K_Zeroes", "PBS_V_Packed",
    "PBS_V_Scales", "PBS_V_Zeroes", "PBS_token_ids", "global_attn_scores",
)

_vp = C.c_void_p
_i = C.c_int
_f = C.c_float


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class CpuImpl:
    """One of the two CPU implementations, selected by symbol prefix."""

    def __init__(self, path: str, prefix: str, kind: str):
        self.path = path
        self.kind = kind
        self.lib = C.CDLL(path)
        p = prefix
        L = self.lib

        def fn(name, args, res=None):
            f = getattr(L, p + name)
            f.argtypes = args
            f.restype = res
            return f

        self._qk = fn("quantize_k_block", [_vp, _vp, _vp, _vp, _i, _i, _i, _i])
        self._qv = fn("quantize_v_block", [_vp, _vp, _vp, _vp, _i, _i, _i, _i])
        self._dk = fn("dequantize_k", [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i])
        self._dv = fn("dequantize_v", [_vp, _vp, _vp, _vp, _i, _i, _i, _i])
        self._fa = fn("fused_attention_decode",
                      [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _i, _i])
        self._ecreate = fn("engine_create", [_i, _i, _i, _i, _i, _i, _f, _f, _i, _i, _i], _vp)
        self._edestroy = fn("engine_destroy", [_vp])
        self._estep = fn("engine_step", [_vp, _vp, _vp, _vp, _vp])
        self._eprefill = fn("engine_prefill", [_vp, _vp, _vp, _i])
        self._eingest = fn("engine_ingest", [_vp, _vp, _vp])
        self._efeedback = fn("engine_feedback", [_vp, _vp])
        self._evisible = fn("engine_visible", [_vp], _i)
        self._ebytes = fn("engine_buffer_bytes", [_vp], C.c_size_t)
        self._ecounters = fn("engine_counters", [_vp, _vp])
        self._ethr = fn("engine_cached_threshold", [_vp], _f)
        self._ebuf = fn("engine_buffer", [_vp, _i, C.POINTER(C.c_int64), C.POINTER(C.c_int)], _vp)
        self._eattend = fn("engine_attend", [_vp, _vp, _vp, _vp]) if hasattr(L, p + "engine_attend") else None

    # ---- stateless kernels ----
    def quantize_k(self, K, k_group_size=16, fp16=False):
        K = _c(K, np.float32)
        kgs, H, D = K.shape
        assert kgs == k_group_size
        mt = np.uint16 if fp16 else np.float32
        packed = np.zeros((kgs // 16, H, D), np.int32)
        scale = np.zeros((H, D), mt)
        zero = np.zeros((H, D), mt)
        self._qk(_ptr(K), _ptr(packed), _ptr(scale), _ptr(zero), H, D, kgs, int(fp16))
        return packed, scale, zero

    def quantize_v(self, V, fp16=False):
        V = _c(V, np.float32)
        ch, H, D = V.shape
        mt = np.uint16 if fp16 else np.float32
        packed = np.zeros((ch, H, (D + 15) // 16), np.int32)
        scale = np.zeros((ch, H), mt)
        zero = np.zeros((ch, H), mt)
        self._qv(_ptr(V), _ptr(packed), _ptr(scale), _ptr(zero), H, D, ch, int(fp16))
        return packed, scale, zero

    def dequantize_k(self, packed, scale, zero, num_blocks, H, D, k_group_size=16, fp16=False):
        mt = np.uint16 if fp16 else np.float32
        packed, scale, zero = _c(packed, np.int32), _c(scale, mt), _c(zero, mt)
        out = np.zeros((num_blocks * k_group_size, H, D), np.float32)
        self._dk(_ptr(packed), _ptr(scale), _ptr(zero), _ptr(out), num_blocks, H, D, k_group_size, int(fp16))
        return out

    def dequantize_v(self, packed, scale, zero, total_tokens, H, D, fp16=False):
        mt = np.uint16 if fp16 else np.float32
        packed, scale, zero = _c(packed, np.int32), _c(scale, mt), _c(zero, mt)
        out = np.zeros((total_tokens, H, D), np.float32)
        self._dv(_ptr(packed), _ptr(scale), _ptr(zero), _ptr(out), total_tokens, H, D, int(fp16))
        return out

    def fused_attention_decode(self, Q, dense_K, dense_V, dense_count, KP, KS, KZ, VP, VS, VZ, ids,
                               num_blocks, Hq, Hkv, D, k_group_size=16, fp16=False, want_mean=True):
        mt = np.uint16 if fp16 else np.float32
        Q = _c(Q, np.float32)
        dK = _c(dense_K, np.float32) if dense_count > 0 else None
        dV = _c(dense_V, np.float32) if dense_count > 0 else None
        arrs = [None] * 7
        if num_blocks > 0:
            arrs = [_c(KP, np.int32), _c(KS, mt), _c(KZ, mt), _c(VP, np.int32), _c(VS, mt), _c(VZ, mt),
                    _c(ids, np.int64)]
        out = np.zeros((Hq, D), np.float32)
        total = dense_count + num_blocks * k_group_size
        mw = np.zeros(max(total, 1), np.float32) if want_mean else None
        self._fa(_ptr(Q), _ptr(dK), _ptr(dV), dense_count, *[_ptr(a) for a in arrs], num_blocks, Hq, Hkv, D,
                 _ptr(out), _ptr(mw), k_group_size, int(fp16))
        return out, (mw[:total] if want_mean else None)

    # ---- engine ----
    def engine(self, num_q_heads, num_kv_heads, head_dim, max_seq_len, sink_size=4, rw_size=64,
               h_ratio=0.1, score_decay=0.999, update_interval=16, k_group_size=16, fp16=True):
        return CpuEngine(self, num_q_heads, num_kv_heads, head_dim, max_seq_len, sink_size, rw_size,
                         h_ratio, score_decay, update_interval, k_group_size, fp16)


class CpuEngine:
    def __init__(self, impl: CpuImpl, Hq, Hkv, D, msl, sink, rw, h_ratio, decay, interval, kgs, fp16):
        self.impl = impl
        self.Hq, self.Hkv, self.D = Hq, Hkv, D
        self.h = impl._ecreate(Hq, Hkv, D, msl, sink, rw, float(h_ratio), float(decay), interval, kgs, int(fp16))
        self.fp16 = bool(fp16)

    def __del__(self):
        h = getattr(self, "h", None)
        if h:
            self.impl._edestroy(h)
            self.h = None

    def step(self, Q, K, V):
        Q, K, V = _c(Q, np.float32), _c(K, np.float32), _c(V, np.float32)
        out = np.zeros(self.Hq * self.D, np.float32)
        self.impl._estep(self.h, _ptr(Q), _ptr(K), _ptr(V), _ptr(out))
        return out

    def prefill(self, K_all, V_all, q_len=None):
        K_all, V_all = _c(K_all, np.float32), _c(V_all, np.float32)
        q_len = K_all.shape[0] if q_len is None else q_len
        self.impl._eprefill(self.h, _ptr(K_all), _ptr(V_all), int(q_len))

    def ingest(self, K, V):
        K, V = _c(K, np.float32), _c(V, np.float32)
        self.impl._eingest(self.h, _ptr(K), _ptr(V))

    def feedback(self, mw):
        mw = _c(mw, np.float32)
        assert mw.size >= self.visible()
        self.impl._efeedback(self.h, _ptr(mw))

    def attend(self, Q):
        if self.impl._eattend is None:
            raise NotImplementedError("attend() is only provided by the C restatement")
        Q = _c(Q, np.float32)
        out = np.zeros(self.Hq * self.D, np.float32)
        mw = np.zeros(max(self.visible(), 1), np.float32)
        self.impl._eattend(self.h, _ptr(Q), _ptr(out), _ptr(mw))
        return out, mw[: self.visible()]

    def visible(self) -> int:
        return int(self.impl._evisible(self.h))

    def buffer_bytes(self) -> int:
        return int(self.impl._ebytes(self.h))

    def cached_threshold(self) -> float:
        return float(self.impl._ethr(self.h))

    def counters(self) -> dict:
        a = np.zeros(N_COUNTERS, np.int64)
        self.impl._ecounters(self.h, _ptr(a))
        return dict(zip(COUNTER_NAMES, (int(x) for x in a)))

    def buffer(self, name: str) -> np.ndarray:
        which = BUFFER_NAMES.index(name)
        n = C.c_int64(0)
        es = C.c_int(0)
        p = self.impl._ebuf(self.h, which, C.byref(n), C.byref(es))
        if not p or n.value == 0:
            return np.zeros(0, np.uint8)
        dt = {8: np.int64, 2: np.uint16, 4: np.int32 if name.endswith(("Packed",)) else np.float32}[es.value]
        buf = (C.c_uint8 * (n.value * es.value)).from_address(p)
        return np.frombuffer(buf, dtype=dt).copy()

    def state(self) -> dict:
        """Counters plus a copy of every tier buffer (for bit-exact comparison)."""
        s = {"counters": self.counters()}
        for name in BUFFER_NAMES:
            s[name] = self.buffer(name)
        return s


_ORACLE = None
_REF = None


def load_oracle() -> CpuImpl:
    global _ORACLE
    if _ORACLE is None:
        if not os.path.exists(ORACLE_SO):
            raise FileNotFoundError(f"{ORACLE_SO} not built (run `make -C oracle`)")
        _ORACLE = CpuImpl(ORACLE_SO, "orc_", "port")
    return _ORACLE


def load_reference():
    """The compiled reference, or None where it was never built."""
    global _REF
    if _REF is None and os.path.exists(REF_SO):
        _REF = CpuImpl(REF_SO, "ttref_", "reference")
    return _REF
