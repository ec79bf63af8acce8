"""Loader for libtritiercache_amd.so (the gfx950 C ABI in include/tritiercache_amd.h).

The library is built in-tree by ``tritiercache_amd/csrc/Makefile`` (or
``__graft_entry__.build()``). There is no fallback: if it is missing or does not
load, importing the extension raises ImportError naming the file.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtritiercache_amd.so")

TT_OK = 0
TT_ERR_INVALID_ARGUMENT = 1
TT_ERR_OUT_OF_RANGE = 2
TT_ERR_NO_MEMORY = 3
TT_ERR_RUNTIME = 4
TT_ERR_HIP = 5

_vp = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t



class DecodeSeq(C.Structure):
    """tt_decode_seq: one sequence of a batched decode step (device pointers)."""
    _fields_ = [
        ("Q", _vp), ("dense_K", _vp), ("dense_V", _vp),
        ("PBS_K_Packed", _vp), ("PBS_K_Scales", _vp), ("PBS_K_Zeroes", _vp),
        ("PBS_V_Packed", _vp), ("PBS_V_Scales", _vp), ("PBS_V_Zeroes", _vp),
        ("PBS_token_ids", _vp), ("attn_output", _vp), ("mean_attn_weights", _vp),
        ("dense_count", C.c_int32), ("num_blocks", C.c_int32),
    ]


# name -> (restype, argtypes); mirrors include/tritiercache_amd.h
_SIGNATURES = {
    "tt_last_error": (C.c_char_p, []),
    "tt_version": (C.c_char_p, []),
    "tt_device_count": (_i, []),
    "tt_pointer_kind": (_i, [_vp]),
    "tt_quantize_k_block": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "tt_quantize_v_block": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "tt_dequantize_k": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "tt_dequantize_v": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "tt_fused_attention_decode": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                       _vp, _vp, _i, _i, _vp]),
    "tt_fused_attention_decode_noalloc": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i,
                                               _i, _vp, _vp, _i, _i, _vp]),
    "tt_fused_attention_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "tt_fused_attention_decode_ws": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                          _vp, _vp, _i, _i, _vp, _sz, _vp]),
    "tt_attention_partials": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i,
                                   _i, _vp, _sz, _vp]),
    "tt_attention_finalize": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "tt_attention_finalize_deferred": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _i, _i, _vp, _sz, _i, _i, _vp, _vp, _sz,
                                            _vp]),
    "tt_batched_decode_workspace_bytes": (_sz, [C.POINTER(DecodeSeq), _i, _i, _i, _i, _i]),
    "tt_fused_attention_decode_batched": (_i, [C.POINTER(DecodeSeq), _vp, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "tt_engine_create": (_i, [C.POINTER(_vp), _i, _i, _i, _i, _i, _i, _f, _f, _i, _i, C.c_char_p, _vp]),
    "tt_engine_destroy": (_i, [_vp]),
    "tt_engine_step": (_i, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "tt_engine_step_deferred": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tt_engine_flush_feedback": (_i, [_vp, _vp]),
    "tt_engine_step_weights": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, C.POINTER(_i), _vp]),
    "tt_engine_prefill": (_i, [_vp, _vp, _vp, _i, _vp]),
    "tt_engine_ingest": (_i, [_vp, _vp, _vp, _vp]),
    "tt_engine_feedback": (_i, [_vp, _vp, _vp]),
    "tt_engine_counters": (_i, [_vp, _vp, _vp]),
    "tt_engine_counter_names": (C.c_char_p, []),
    "tt_engine_buffer_bytes": (_i, [_vp, C.POINTER(_sz), _vp]),
    "tt_engine_buffer": (_i, [_vp, _i, C.POINTER(_vp), C.POINTER(C.c_int64), C.POINTER(_i), _vp]),
    "tt_engine_visible": (_i, [_vp, C.POINTER(_i), _vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib = None


def load() -> C.CDLL:
    """Load the library once; raise ImportError with the path if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"tritiercache_amd: native library not found at {LIB_PATH}; build it with "
            "`make -C tritiercache_amd/csrc` (or __graft_entry__.build())")
    try:
        lib = C.CDLL(LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the ROCm runtime
        raise ImportError(f"tritiercache_amd: cannot load {LIB_PATH}: {e}") from e
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().tt_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str = "") -> None:
    """Raise the exception the reference's translator raises for this status
    (csrc/bindings.cpp:321-337)."""
    if rc == TT_OK:
        return
    msg = last_error() or f"{what} failed with status {rc}"
    if rc == TT_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    if rc == TT_ERR_OUT_OF_RANGE:
        raise IndexError(msg)
    if rc == TT_ERR_NO_MEMORY:
        raise MemoryError(msg)
    raise RuntimeError(msg)
