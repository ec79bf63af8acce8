"""``tri_tier._C`` drop-in: the reference extension's Python surface over the gfx950 C ABI.

Same names, argument names, defaults and exception classes as the reference
module (csrc/bindings.cpp:317-626). The compute runs in
``libtritiercache_amd.so`` on the current HIP device, on torch's current stream.

Argument conventions follow the reference's ``get_contiguous_ptr``
(bindings.cpp:25-97): every tensor argument may be a raw integer address, a
torch tensor (must be contiguous) or a C-contiguous buffer-protocol object
(numpy array, memoryview). Device memory (ROCm tensors, device addresses) is
used in place. Host memory (CPU tensors, numpy arrays, host addresses) is
staged through device memory and, for output arguments, copied back before the
call returns, so the reference's host-side callers and tests keep working.

Differences from the reference, all documented in the C header:
  * the zero-copy getters return ROCm tensors viewing device memory (the
    reference returns numpy arrays viewing host memory);
  * num_q_heads must be a multiple of num_kv_heads and head_dim a multiple of
    16 of at most 256 (ValueError otherwise).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib

_L = _lib.load()

__all__ = [
    "TriTierCacheEngine",
    "fused_attention_decode",
    "quantize_k_block",
    "quantize_v_block",
    "dequantize_k",
    "dequantize_v",
    "device_count",
    "version",
]


def device_count() -> int:
    return int(_L.tt_device_count())


def version() -> str:
    return _L.tt_version().decode()


def _require_gpu() -> None:
    if device_count() == 0 or not torch.cuda.is_available():
        raise RuntimeError("tritiercache_amd: no HIP device is visible; the gfx950 kernels need an MI355X GPU.")


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _is_fp16(dtype_str: str, scale_obj) -> bool:
    """bindings.cpp:130-136: "fp16" selects half metadata, as does a scale
    object whose dtype string names float16/half."""
    fp16 = dtype_str == "fp16"
    dt = getattr(scale_obj, "dtype", None)
    if dt is not None:
        s = str(dt)
        if "float16" in s or "half" in s:
            fp16 = True
    return fp16


class _Staging:
    """Resolves arguments to device addresses, staging host memory."""

    def __init__(self):
        self._writeback = []
        self._keep = []

    def ptr(self, obj, name: str, nbytes: int, writable: bool = False, nullable: bool = False) -> int:
        if obj is None:
            if nullable:
                return 0
            raise ValueError(f"Argument '{name}' cannot be None.")
        if isinstance(obj, int) and not isinstance(obj, bool):
            if obj == 0:
                if nullable:
                    return 0
                raise ValueError(f"Argument '{name}' pointer address is NULL.")
            if int(_L.tt_pointer_kind(C.c_void_p(obj))) == 1:
                return obj
            return self._stage_raw(obj, nbytes, writable)
        if isinstance(obj, torch.Tensor):
            if not obj.is_contiguous():
                raise ValueError(
                    f"Argument '{name}' PyTorch tensor is not contiguous in memory. Call .contiguous() before passing.")
            if obj.is_cuda:
                p = obj.data_ptr()
                if p == 0 and not nullable:
                    raise ValueError(f"Argument '{name}' tensor data pointer is NULL.")
                return p
            return self._stage_tensor(obj, writable)
        if hasattr(obj, "data_ptr") and hasattr(obj, "is_contiguous"):
            if not obj.is_contiguous():
                raise ValueError(
                    f"Argument '{name}' PyTorch tensor is not contiguous in memory. Call .contiguous() before passing.")
            return int(obj.data_ptr())
        try:
            arr = np.asarray(memoryview(obj))
        except TypeError:
            raise ValueError(
                f"Argument '{name}' has unsupported type '{type(obj)}'. Expected PyTorch tensor, NumPy array, buffer "
                "object, or integer memory address.") from None
        if not arr.flags["C_CONTIGUOUS"]:
            raise ValueError(f"Argument '{name}' buffer is not C-contiguous in memory.")
        if writable and not arr.flags["WRITEABLE"]:
            raise ValueError(f"Argument '{name}' buffer is read-only.")
        return self._stage_numpy(arr, writable)

    def _device_copy(self, host_u8: torch.Tensor) -> torch.Tensor:
        dev = torch.empty(max(host_u8.numel(), 1), dtype=torch.uint8, device="cuda")
        if host_u8.numel():
            dev[: host_u8.numel()].copy_(host_u8)
        self._keep.append(dev)
        return dev

    def _stage_numpy(self, arr: np.ndarray, writable: bool) -> int:
        u8 = torch.from_numpy(arr.reshape(-1).view(np.uint8))
        dev = self._device_copy(u8)
        if writable:
            self._writeback.append(("numpy", arr, dev))
        return dev.data_ptr()

    def _stage_tensor(self, t: torch.Tensor, writable: bool) -> int:
        u8 = t.reshape(-1).view(torch.uint8)
        dev = self._device_copy(u8)
        if writable:
            self._writeback.append(("tensor", t, dev))
        return dev.data_ptr()

    def _stage_raw(self, addr: int, nbytes: int, writable: bool) -> int:
        buf = (C.c_uint8 * max(nbytes, 1)).from_address(addr)
        u8 = torch.from_numpy(np.frombuffer(buf, dtype=np.uint8, count=nbytes))
        dev = self._device_copy(u8)
        if writable:
            self._writeback.append(("raw", addr, dev, nbytes))
        return dev.data_ptr()

    def finish(self) -> None:
        if not self._writeback:
            return
        torch.cuda.current_stream().synchronize()
        for item in self._writeback:
            kind = item[0]
            if kind == "numpy":
                _, arr, dev = item
                n = arr.nbytes
                flat = arr.reshape(-1).view(np.uint8)
                flat[:] = dev[:n].cpu().numpy()
            elif kind == "tensor":
                _, t, dev = item
                n = t.numel() * t.element_size()
                t.reshape(-1).view(torch.uint8).copy_(dev[:n].cpu())
            else:
                _, addr, dev, n = item
                host = dev[:n].cpu().numpy()
                C.memmove(addr, host.ctypes.data, n)
        self._writeback.clear()
        self._keep.clear()


def fused_attention_decode(Q_ptr, dense_K_ptr, dense_V_ptr, dense_count, PBS_K_Packed_ptr, PBS_K_Scales_ptr,
                           PBS_K_Zeroes_ptr, PBS_V_Packed_ptr, PBS_V_Scales_ptr, PBS_V_Zeroes_ptr, PBS_token_ids_ptr,
                           num_blocks, num_q_heads, num_kv_heads, head_dim, attn_output_ptr,
                           mean_attn_weights_ptr=None, k_group_size=16, pbs_metadata_dtype="fp32"):
    """Fused decode attention over dense KV and 2-bit packed KV (bindings.cpp:99-178)."""
    dense_count, num_blocks = int(dense_count), int(num_blocks)
    Hq, Hkv, D, kgs = int(num_q_heads), int(num_kv_heads), int(head_dim), int(k_group_size)
    if dense_count < 0:
        raise ValueError("dense_count must be non-negative.")
    if num_blocks < 0:
        raise ValueError("num_blocks must be non-negative.")
    if Hq <= 0 or Hkv <= 0 or D <= 0:
        raise ValueError("num_q_heads, num_kv_heads, and head_dim must be positive integers.")
    _require_gpu()
    fp16 = _is_fp16(pbs_metadata_dtype, PBS_K_Scales_ptr)
    msz = 2 if fp16 else 4
    kvs = Hkv * D
    W = max(kgs // 16, 1)
    st = _Staging()
    nd0, nb0 = dense_count == 0, num_blocks == 0
    q = st.ptr(Q_ptr, "Q", Hq * D * 4)
    dk = st.ptr(dense_K_ptr, "dense_K", dense_count * kvs * 4, nullable=nd0)
    dv = st.ptr(dense_V_ptr, "dense_V", dense_count * kvs * 4, nullable=nd0)
    kp = st.ptr(PBS_K_Packed_ptr, "PBS_K_Packed", num_blocks * W * kvs * 4, nullable=nb0)
    vp = st.ptr(PBS_V_Packed_ptr, "PBS_V_Packed", num_blocks * kgs * Hkv * (D // 16) * 4, nullable=nb0)
    ids = st.ptr(PBS_token_ids_ptr, "PBS_token_ids", num_blocks * kgs * 8, nullable=nb0)
    out = st.ptr(attn_output_ptr, "attn_output", Hq * D * 4, writable=True)
    total = dense_count + num_blocks * kgs
    mw = st.ptr(mean_attn_weights_ptr, "mean_attn_weights", total * 4, writable=True, nullable=True)
    ks = st.ptr(PBS_K_Scales_ptr, "PBS_K_Scales", num_blocks * kvs * msz, nullable=nb0)
    kz = st.ptr(PBS_K_Zeroes_ptr, "PBS_K_Zeroes", num_blocks * kvs * msz, nullable=nb0)
    vs = st.ptr(PBS_V_Scales_ptr, "PBS_V_Scales", num_blocks * kgs * Hkv * msz, nullable=nb0)
    vz = st.ptr(PBS_V_Zeroes_ptr, "PBS_V_Zeroes", num_blocks * kgs * Hkv * msz, nullable=nb0)
    rc = _L.tt_fused_attention_decode(q, dk, dv, dense_count, kp, ks, kz, vp, vs, vz, ids, num_blocks, Hq, Hkv, D,
                                      out, mw or None, kgs, int(fp16), _stream())
    _lib.check(rc, "fused_attention_decode")
    st.finish()


_BATCH_FIELDS = ("Q", "dense_K", "dense_V", "dense_count", "PBS_K_Packed", "PBS_K_Scales", "PBS_K_Zeroes",
                 "PBS_V_Packed", "PBS_V_Scales", "PBS_V_Zeroes", "PBS_token_ids", "num_blocks", "attn_output",
                 "mean_attn_weights")


def fused_attention_decode_batched(batch, num_q_heads, num_kv_heads, head_dim, k_group_size=16,
                                   pbs_metadata_dtype="fp32"):
    """One decode step of many sequences in one split-K launch (plus one merge launch).

    `batch` holds one entry per sequence: a dict with the keys of
    ``_BATCH_FIELDS`` or a tuple in that order, i.e. the per-sequence
    arguments of fused_attention_decode (bindings.cpp:99-178); each
    sequence's outputs equal that call's. The sequences share the head
    counts, head_dim, k_group_size and metadata dtype. No counterpart in the
    reference, whose callers loop over sequences."""
    Hq, Hkv, D, kgs = int(num_q_heads), int(num_kv_heads), int(head_dim), int(k_group_size)
    if Hq <= 0 or Hkv <= 0 or D <= 0:
        raise ValueError("num_q_heads, num_kv_heads, and head_dim must be positive integers.")
    _require_gpu()
    entries = [dict(e) if isinstance(e, dict) else dict(zip(_BATCH_FIELDS, e)) for e in batch]
    if not entries:
        return
    fp16 = _is_fp16(pbs_metadata_dtype, entries[0].get("PBS_K_Scales"))
    msz = 2 if fp16 else 4
    kvs = Hkv * D
    W = max(kgs // 16, 1)
    st = _Staging()
    seqs = (_lib.DecodeSeq * len(entries))()
    for i, e in enumerate(entries):
        nd, nb = int(e.get("dense_count", 0)), int(e.get("num_blocks", 0))
        if nd < 0:
            raise ValueError("dense_count must be non-negative.")
        if nb < 0:
            raise ValueError("num_blocks must be non-negative.")
        nd0, nb0 = nd == 0, nb == 0
        s = seqs[i]
        s.Q = st.ptr(e.get("Q"), "Q", Hq * D * 4)
        s.dense_K = st.ptr(e.get("dense_K"), "dense_K", nd * kvs * 4, nullable=nd0) or None
        s.dense_V = st.ptr(e.get("dense_V"), "dense_V", nd * kvs * 4, nullable=nd0) or None
        s.PBS_K_Packed = st.ptr(e.get("PBS_K_Packed"), "PBS_K_Packed", nb * W * kvs * 4, nullable=nb0) or None
        s.PBS_K_Scales = st.ptr(e.get("PBS_K_Scales"), "PBS_K_Scales", nb * kvs * msz, nullable=nb0) or None
        s.PBS_K_Zeroes = st.ptr(e.get("PBS_K_Zeroes"), "PBS_K_Zeroes", nb * kvs * msz, nullable=nb0) or None
        s.PBS_V_Packed = st.ptr(e.get("PBS_V_Packed"), "PBS_V_Packed", nb * kgs * Hkv * (D // 16) * 4,
                                nullable=nb0) or None
        s.PBS_V_Scales = st.ptr(e.get("PBS_V_Scales"), "PBS_V_Scales", nb * kgs * Hkv * msz, nullable=nb0) or None
        s.PBS_V_Zeroes = st.ptr(e.get("PBS_V_Zeroes"), "PBS_V_Zeroes", nb * kgs * Hkv * msz, nullable=nb0) or None
        s.PBS_token_ids = st.ptr(e.get("PBS_token_ids"), "PBS_token_ids", nb * kgs * 8, nullable=nb0) or None
        s.attn_output = st.ptr(e.get("attn_output"), "attn_output", Hq * D * 4, writable=True)
        s.mean_attn_weights = st.ptr(e.get("mean_attn_weights"), "mean_attn_weights", (nd + nb * kgs) * 4,
                                     writable=True, nullable=True) or None
        s.dense_count, s.num_blocks = nd, nb
    n = len(entries)
    ws_bytes = int(_L.tt_batched_decode_workspace_bytes(seqs, n, Hq, Hkv, D, kgs))
    if ws_bytes == 0:
        _lib.check(_lib.TT_ERR_INVALID_ARGUMENT, "fused_attention_decode_batched")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    raw = np.frombuffer(bytes(seqs), dtype=np.uint8)
    seqs_dev = torch.from_numpy(raw.copy()).cuda()
    rc = _L.tt_fused_attention_decode_batched(seqs, seqs_dev.data_ptr(), n, Hq, Hkv, D, kgs, int(fp16), ws.data_ptr(),
                                              ws_bytes, _stream())
    _lib.check(rc, "fused_attention_decode_batched")
    st.finish()


def quantize_k_block(K, packed, scale, zero, num_heads, head_dim, k_group_size=16, pbs_metadata_dtype="fp32"):
    """2-bit per-channel quantisation of one K block (bindings.cpp:180-212)."""
    H, D, kgs = int(num_heads), int(head_dim), int(k_group_size)
    _require_gpu()
    fp16 = _is_fp16(pbs_metadata_dtype, scale)
    msz = 2 if fp16 else 4
    st = _Staging()
    k = st.ptr(K, "K", kgs * H * D * 4)
    p = st.ptr(packed, "packed", (kgs // 16) * H * D * 4, writable=True)
    s = st.ptr(scale, "scale", H * D * msz, writable=True)
    z = st.ptr(zero, "zero", H * D * msz, writable=True)
    _lib.check(_L.tt_quantize_k_block(k, p, s, z, 1, H, D, kgs, int(fp16), _stream()), "quantize_k_block")
    st.finish()


def quantize_k_blocks(K, packed, scale, zero, num_blocks, num_heads, head_dim, k_group_size=16,
                      pbs_metadata_dtype="fp32"):
    """Batched quantize_k_block over `num_blocks` consecutive blocks (one launch)."""
    nb, H, D, kgs = int(num_blocks), int(num_heads), int(head_dim), int(k_group_size)
    _require_gpu()
    fp16 = _is_fp16(pbs_metadata_dtype, scale)
    msz = 2 if fp16 else 4
    st = _Staging()
    k = st.ptr(K, "K", nb * kgs * H * D * 4)
    p = st.ptr(packed, "packed", nb * (kgs // 16) * H * D * 4, writable=True)
    s = st.ptr(scale, "scale", nb * H * D * msz, writable=True)
    z = st.ptr(zero, "zero", nb * H * D * msz, writable=True)
    _lib.check(_L.tt_quantize_k_block(k, p, s, z, nb, H, D, kgs, int(fp16), _stream()), "quantize_k_blocks")
    st.finish()


def quantize_v_block(V, packed, scale, zero, num_heads, head_dim, chunk_size=16, pbs_metadata_dtype="fp32"):
    """2-bit per-token quantisation of one V block (bindings.cpp:214-246)."""
    H, D, ch = int(num_heads), int(head_dim), int(chunk_size)
    _require_gpu()
    fp16 = _is_fp16(pbs_metadata_dtype, scale)
    msz = 2 if fp16 else 4
    st = _Staging()
    v = st.ptr(V, "V", ch * H * D * 4)
    p = st.ptr(packed, "packed", ch * H * ((D + 15) // 16) * 4, writable=True)
    s = st.ptr(scale, "scale", ch * H * msz, writable=True)
    z = st.ptr(zero, "zero", ch * H * msz, writable=True)
    _lib.check(_L.tt_quantize_v_block(v, p, s, z, ch, H, D, int(fp16), _stream()), "quantize_v_block")
    st.finish()


def dequantize_k(packed, scale, zero, out, num_blocks, num_heads, head_dim, k_group_size=16,
                 pbs_metadata_dtype="fp32"):
    """Dequantise K blocks: x = fmaf(q, scale, zero) (bindings.cpp:248-281)."""
    nb, H, D, kgs = int(num_blocks), int(num_heads), int(head_dim), int(k_group_size)
    _require_gpu()
    fp16 = _is_fp16(pbs_metadata_dtype, scale)
    msz = 2 if fp16 else 4
    st = _Staging()
    p = st.ptr(packed, "packed", nb * (kgs // 16) * H * D * 4)
    s = st.ptr(scale, "scale", nb * H * D * msz)
    z = st.ptr(zero, "zero", nb * H * D * msz)
    o = st.ptr(out, "out", nb * kgs * H * D * 4, writable=True)
    _lib.check(_L.tt_dequantize_k(p, s, z, o, nb, H, D, kgs, int(fp16), _stream()), "dequantize_k")
    st.finish()


def dequantize_v(packed, scale, zero, out, total_tokens, num_heads, head_dim, pbs_metadata_dtype="fp32"):
    """Dequantise V tokens (bindings.cpp:283-315)."""
    n, H, D = int(total_tokens), int(num_heads), int(head_dim)
    _require_gpu()
    fp16 = _is_fp16(pbs_metadata_dtype, scale)
    msz = 2 if fp16 else 4
    st = _Staging()
    p = st.ptr(packed, "packed", n * H * ((D + 15) // 16) * 4)
    s = st.ptr(scale, "scale", n * H * msz)
    z = st.ptr(zero, "zero", n * H * msz)
    o = st.ptr(out, "out", n * H * D * 4, writable=True)
    _lib.check(_L.tt_dequantize_v(p, s, z, o, n, H, D, int(fp16), _stream()), "dequantize_v")
    st.finish()


class _DeviceView:
    """__cuda_array_interface__ holder: torch.as_tensor keeps it (and through
    it the engine) alive for as long as the tensor lives."""

    def __init__(self, ptr: int, shape, typestr: str, owner):
        self._owner = owner
        self.__cuda_array_interface__ = {
            "shape": tuple(int(s) for s in shape),
            "typestr": typestr,
            "data": (int(ptr), False),
            "version": 3,
            "strides": None,
        }


_BUFFERS = {
    "S_K": 0, "S_V": 1, "RW_K": 2, "RW_V": 3, "HH_K": 4, "HH_V": 5, "HH_token_ids": 6, "HH_scores": 7, "WR_K": 8,
    "WR_V": 9, "WR_token_ids": 10, "PBS_K_Packed": 11, "PBS_K_Scales": 12, "PBS_K_Zeroes": 13, "PBS_V_Packed": 14,
    "PBS_V_Scales": 15, "PBS_V_Zeroes": 16, "PBS_token_ids": 17, "global_attn_scores": 18,
    "mean_attn_weights": 19,
}


class TriTierCacheEngine:
    """Device-resident tier engine (bindings.cpp:384-626, cache_engine.cpp)."""

    _COUNTER_NAMES = None

    def __init__(self, num_q_heads, num_kv_heads, head_dim, max_seq_len, sink_size=4, rw_size=64, h_ratio=0.1,
                 score_decay=0.999, update_interval=16, k_group_size=16, pbs_metadata_dtype="fp16"):
        _require_gpu()
        self._h = None
        h = C.c_void_p()
        self._pbs_metadata_dtype = str(pbs_metadata_dtype)
        rc = _L.tt_engine_create(C.byref(h), int(num_q_heads), int(num_kv_heads), int(head_dim), int(max_seq_len),
                                 int(sink_size), int(rw_size), float(h_ratio), float(score_decay),
                                 int(update_interval), int(k_group_size), self._pbs_metadata_dtype.encode(),
                                 _stream())
        _lib.check(rc, "TriTierCacheEngine")
        self._h = h
        self.h_ratio = float(np.float32(h_ratio))
        self.score_decay = float(np.float32(score_decay))
        c = self.counters()
        for k in ("num_q_heads", "num_kv_heads", "head_dim", "max_seq_len", "sink_size", "rw_size",
                  "update_interval", "k_group_size", "chunk_size", "quant_head_dim", "max_hh"):
            setattr(self, "_" + k, c[k])

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _L.tt_engine_destroy(h)
            self._h = None

    # ---- configuration (read-only) ----
    num_q_heads = property(lambda self: self._num_q_heads)
    num_kv_heads = property(lambda self: self._num_kv_heads)
    head_dim = property(lambda self: self._head_dim)
    max_seq_len = property(lambda self: self._max_seq_len)
    sink_size = property(lambda self: self._sink_size)
    rw_size = property(lambda self: self._rw_size)
    update_interval = property(lambda self: self._update_interval)
    k_group_size = property(lambda self: self._k_group_size)
    chunk_size = property(lambda self: self._chunk_size)
    quant_head_dim = property(lambda self: self._quant_head_dim)
    max_hh = property(lambda self: self._max_hh)
    pbs_metadata_dtype = property(lambda self: self._pbs_metadata_dtype)
    use_fp16_meta = property(lambda self: self._pbs_metadata_dtype == "fp16")

    # ---- counters (read from the device; synchronises the current stream) ----
    def counters(self) -> dict:
        if TriTierCacheEngine._COUNTER_NAMES is None:
            TriTierCacheEngine._COUNTER_NAMES = _L.tt_engine_counter_names().decode().split()
        out = np.zeros(23, np.int64)
        _lib.check(_L.tt_engine_counters(self._h, out.ctypes.data, _stream()), "counters")
        return dict(zip(TriTierCacheEngine._COUNTER_NAMES, (int(x) for x in out)))

    pbs_allocated_blocks = property(lambda self: self.counters()["pbs_allocated_blocks"])
    s_count = property(lambda self: self.counters()["s_count"])
    rw_count = property(lambda self: self.counters()["rw_count"])
    rw_head_index = property(lambda self: self.counters()["rw_head_index"])
    hh_count = property(lambda self: self.counters()["hh_count"])
    wr_count = property(lambda self: self.counters()["wr_count"])
    pbs_count = property(lambda self: self.counters()["pbs_count"])
    pbs_blocks_used = property(lambda self: self.counters()["pbs_blocks_used"])
    total_processed_tokens = property(lambda self: self.counters()["total_processed_tokens"])
    total_evictions = property(lambda self: self.counters()["total_evictions"])
    last_calc_pos = property(lambda self: self.counters()["last_calc_pos"])

    # ---- compute ----
    def step(self, q_ptr, k_ptr, v_ptr, out_ptr):
        """Ingest one token, attend, feed back scores (cache_engine.cpp:397-541)."""
        st = _Staging()
        Hq, Hkv, D = self._num_q_heads, self._num_kv_heads, self._head_dim
        q = st.ptr(q_ptr, "Q", Hq * D * 4)
        k = st.ptr(k_ptr, "K_new", Hkv * D * 4)
        v = st.ptr(v_ptr, "V_new", Hkv * D * 4)
        o = st.ptr(out_ptr, "attn_output", Hq * D * 4, writable=True)
        _lib.check(_L.tt_engine_step(self._h, q, k, v, o, _stream()), "step")
        st.finish()

    def step_deferred(self, q_ptr, k_ptr, v_ptr, out_ptr, prev=None):
        """step() for engines stepped one after another (a model's layers): this
        step runs up to its merged attention output and leaves its mean attention
        weights and score feedback pending; the pending feedback of `prev`
        (another TriTierCacheEngine on the same device, or None) runs in this
        step's finalize launch. A pending feedback also runs at the start of any
        later call on its engine, or in flush_feedback()."""
        if prev is self:
            raise ValueError("prev must be another engine.")
        st = _Staging()
        Hq, Hkv, D = self._num_q_heads, self._num_kv_heads, self._head_dim
        q = st.ptr(q_ptr, "Q", Hq * D * 4)
        k = st.ptr(k_ptr, "K_new", Hkv * D * 4)
        v = st.ptr(v_ptr, "V_new", Hkv * D * 4)
        o = st.ptr(out_ptr, "attn_output", Hq * D * 4, writable=True)
        ph = prev._h if prev is not None else None
        _lib.check(_L.tt_engine_step_deferred(self._h, q, k, v, o, ph, _stream()), "step_deferred")
        st.finish()

    def flush_feedback(self):
        """Runs this engine's pending mean weights and score feedback, if any."""
        _lib.check(_L.tt_engine_flush_feedback(self._h, _stream()), "flush_feedback")

    def step_with_weights(self, q_ptr, k_ptr, v_ptr, out_ptr) -> torch.Tensor:
        """step() that also returns this step's per-head softmax weights
        [num_q_heads, visible] in the engine's visible order."""
        st = _Staging()
        Hq, Hkv, D = self._num_q_heads, self._num_kv_heads, self._head_dim
        q = st.ptr(q_ptr, "Q", Hq * D * 4)
        k = st.ptr(k_ptr, "K_new", Hkv * D * 4)
        v = st.ptr(v_ptr, "V_new", Hkv * D * 4)
        o = st.ptr(out_ptr, "attn_output", Hq * D * 4, writable=True)
        # the step adds the new token, and a waiting-room flush makes up to
        # one more chunk of tokens visible
        cap = self.visible() + 1 + self._chunk_size
        w = torch.empty((Hq, cap), dtype=torch.float32, device="cuda")
        vis = C.c_int(0)
        _lib.check(_L.tt_engine_step_weights(self._h, q, k, v, o, w.data_ptr(), cap, C.byref(vis), _stream()),
                   "step_with_weights")
        st.finish()
        return w[:, : vis.value]

    def prefill(self, k_ptr, v_ptr, q_len):
        """Bulk prompt ingest (cache_engine.cpp:271-395)."""
        q_len = int(q_len)
        if q_len < 0:
            raise ValueError("q_len must be non-negative.")
        st = _Staging()
        n = q_len * self._num_kv_heads * self._head_dim * 4
        k = st.ptr(k_ptr, "K_all", n, nullable=q_len == 0)
        v = st.ptr(v_ptr, "V_all", n, nullable=q_len == 0)
        _lib.check(_L.tt_engine_prefill(self._h, k, v, q_len, _stream()), "prefill")
        st.finish()

    def ingest(self, k_ptr, v_ptr):
        """Tier maintenance only: ring ingest / eviction / routing / flush."""
        st = _Staging()
        n = self._num_kv_heads * self._head_dim * 4
        k = st.ptr(k_ptr, "K_new", n)
        v = st.ptr(v_ptr, "V_new", n)
        _lib.check(_L.tt_engine_ingest(self._h, k, v, _stream()), "ingest")
        st.finish()

    def feedback(self, mean_attn_weights):
        """Decayed score feedback with caller-supplied mean weights [visible]."""
        n = self.visible()
        size = getattr(mean_attn_weights, "numel", None)
        size = size() if callable(size) else getattr(mean_attn_weights, "size", None)
        if isinstance(size, int) and size < n:
            raise ValueError(f"mean_attn_weights has {size} elements; the engine attends {n} tokens.")
        st = _Staging()
        w = st.ptr(mean_attn_weights, "mean_attn_weights", n * 4)
        _lib.check(_L.tt_engine_feedback(self._h, w, _stream()), "feedback")
        st.finish()

    def visible(self) -> int:
        v = C.c_int(0)
        _lib.check(_L.tt_engine_visible(self._h, C.byref(v), _stream()), "visible")
        return int(v.value)

    def get_buffer_bytes(self) -> int:
        """The reference's tier-byte accounting (cache_engine.cpp:543-568)."""
        v = C.c_size_t(0)
        _lib.check(_L.tt_engine_buffer_bytes(self._h, C.byref(v), _stream()), "get_buffer_bytes")
        return int(v.value)

    # ---- zero-copy device views (bindings.cpp:461-626) ----
    def _view(self, name: str, shape, typestr: str) -> torch.Tensor:
        p = C.c_void_p()
        n = C.c_int64(0)
        es = C.c_int(0)
        _lib.check(_L.tt_engine_buffer(self._h, _BUFFERS[name], C.byref(p), C.byref(n), C.byref(es), _stream()),
                   name)
        assert int(np.prod(shape)) == n.value, (name, shape, n.value)
        if n.value == 0:
            return torch.empty(shape, dtype=torch.uint16 if typestr == "<u2" else {
                "<f4": torch.float32, "<i4": torch.int32, "<i8": torch.int64}[typestr], device="cuda")
        return torch.as_tensor(_DeviceView(p.value, shape, typestr, self), device="cuda")

    def _meta(self):
        return "<u2" if self.use_fp16_meta else "<f4"

    def get_global_attn_scores(self):
        return self._view("global_attn_scores", (self._max_seq_len,), "<f4")

    def get_S_K(self):
        return self._view("S_K", (self._sink_size, self._num_kv_heads, self._head_dim), "<f4")

    def get_S_V(self):
        return self._view("S_V", (self._sink_size, self._num_kv_heads, self._head_dim), "<f4")

    def get_RW_K(self):
        return self._view("RW_K", (self._rw_size, self._num_kv_heads, self._head_dim), "<f4")

    def get_RW_V(self):
        return self._view("RW_V", (self._rw_size, self._num_kv_heads, self._head_dim), "<f4")

    def get_HH_K(self):
        return self._view("HH_K", (self._max_hh, self._num_kv_heads, self._head_dim), "<f4")

    def get_HH_V(self):
        return self._view("HH_V", (self._max_hh, self._num_kv_heads, self._head_dim), "<f4")

    def get_HH_token_ids(self):
        return self._view("HH_token_ids", (self._max_hh,), "<i8")

    def get_HH_scores(self):
        return self._view("HH_scores", (self._max_hh,), "<f4")

    def get_WR_K(self):
        return self._view("WR_K", (self._chunk_size, self._num_kv_heads, self._head_dim), "<f4")

    def get_WR_V(self):
        return self._view("WR_V", (self._chunk_size, self._num_kv_heads, self._head_dim), "<f4")

    def get_WR_token_ids(self):
        return self._view("WR_token_ids", (self._chunk_size,), "<i8")

    def get_PBS_K_Packed(self):
        nb = self.pbs_allocated_blocks
        return self._view("PBS_K_Packed", (nb, self._k_group_size // 16, self._num_kv_heads, self._head_dim), "<i4")

    def get_PBS_K_Scales(self):
        nb = self.pbs_allocated_blocks
        return self._view("PBS_K_Scales", (nb, self._num_kv_heads, self._head_dim), self._meta())

    def get_PBS_K_Zeroes(self):
        nb = self.pbs_allocated_blocks
        return self._view("PBS_K_Zeroes", (nb, self._num_kv_heads, self._head_dim), self._meta())

    def get_PBS_V_Packed(self):
        nb = self.pbs_allocated_blocks
        return self._view("PBS_V_Packed", (nb * self._chunk_size, self._num_kv_heads, self._quant_head_dim), "<i4")

    def get_PBS_V_Scales(self):
        nb = self.pbs_allocated_blocks
        return self._view("PBS_V_Scales", (nb * self._chunk_size, self._num_kv_heads, 1), self._meta())

    def get_PBS_V_Zeroes(self):
        nb = self.pbs_allocated_blocks
        return self._view("PBS_V_Zeroes", (nb * self._chunk_size, self._num_kv_heads, 1), self._meta())

    def get_mean_attn_weights(self):
        """Mean attention weights of the last step, in visible order (engine extra)."""
        return self._view("mean_attn_weights", (self.visible(),), "<f4")

    def get_PBS_token_ids(self):
        nb = self.pbs_allocated_blocks
        return self._view("PBS_token_ids", (nb * self._chunk_size,), "<i8")
