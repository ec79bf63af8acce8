"""TriTierCache: the Python API of the reference (src/tri_tier/cache.py) on the gfx950 engine.

``TriTierCache`` keeps the reference constructor, attributes and methods. The
decode work goes through ``_C.TriTierCacheEngine`` (device-resident tiers,
HIP kernels); the tier buffers the reference exposes as zero-copy numpy views
(cache.py:50-59) are zero-copy ROCm tensor views here, and the counters the
reference mirrors after every call (cache.py:110-116) are read from the device
when accessed, so a decode step never waits for the GPU.

The reference's pure-PyTorch routing / packing / reconstruction methods
(cache.py:164-372) are kept with their reference semantics for callers that
use them directly. They are NOT a fallback for the engine: constructing a
TriTierCache without a usable GPU raises, unless the caller opts into the
reference's CPU reference mode with TRI_TIER_ALLOW_TORCH_FALLBACK=1 on a
machine with no GPU at all.
"""
from __future__ import annotations

import math
import os

import torch

from .constants import CHUNK_SIZE, DEVICE, SINK_SIZE, UPDATE_THRESHOLD

# Counters the reference copies from the engine after step()/prefill().
_ENGINE_COUNTERS = {
    "Total_Processed_Tokens": "total_processed_tokens",
    "total_evictions": "total_evictions",
    "PBS_count": "pbs_count",
    "RW_count": "rw_count",
    "RW_head_index": "rw_head_index",
    "S_count": "s_count",
    "HH_count": "hh_count",
    "WR_count": "wr_count",
}

# Python-side packed store of the reference's pure-PyTorch path (cache.py:82-96).
# Allocated on first use so engine users do not pay for it.
_PY_PBS = ("PBS_K_Packed", "PBS_K_Scales", "PBS_K_Zeroes", "PBS_V_Packed", "PBS_V_Scales", "PBS_V_Zeroes",
           "PBS_token_ids")


def _fallback_allowed() -> bool:
    if os.environ.get("TRI_TIER_ALLOW_TORCH_FALLBACK", "0") != "1":
        return False
    # Never on a machine with a GPU: there the HIP engine is the product path.
    return not torch.cuda.is_available()


class TriTierCache:
    def __init__(self, max_seq_len, head_dim, num_heads, R_size, H_ratio, num_q_heads=None, score_decay=0.999,
                 k_group_size=16, pbs_metadata_dtype="fp16"):
        """R_size: recent-window size; H_ratio: heavy-hitter fraction of max_seq_len."""
        d = self.__dict__
        d["_engine"] = None
        for name in _ENGINE_COUNTERS:
            d["_py_" + name] = 0
        self.R_size = R_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_q_heads = num_q_heads if num_q_heads is not None else num_heads
        self.score_decay = score_decay
        self.k_group_size = 32 if k_group_size == 32 else 16
        self.pbs_metadata_dtype = "fp32" if str(pbs_metadata_dtype).lower() == "fp32" else "fp16"
        self.current_threshold = 0.0
        self.max_seq_len = max_seq_len
        self.max_heavy_hitters = math.ceil(max_seq_len * H_ratio)
        self.max_background_tokens = max_seq_len - R_size - self.max_heavy_hitters

        engine_error = None
        try:
            from . import _C

            decay_val = 1.0 if score_decay is None else float(score_decay)
            d["_engine"] = _C.TriTierCacheEngine(
                self.num_q_heads, self.num_heads, self.head_dim, max_seq_len, SINK_SIZE, R_size, H_ratio, decay_val,
                UPDATE_THRESHOLD, self.k_group_size, self.pbs_metadata_dtype)
        except (ImportError, RuntimeError, ValueError, MemoryError) as e:
            engine_error = e
            d["_engine"] = None
        if self._engine is None and not _fallback_allowed():
            raise RuntimeError(
                "TriTierCache: the gfx950 engine could not be created "
                f"({engine_error}). Set TRI_TIER_ALLOW_TORCH_FALLBACK=1 on a CPU-only machine to use the "
                "reference's pure-PyTorch mode.")

        if self._engine is not None:
            e = self._engine
            self.S_K_Buffer = e.get_S_K()
            self.S_V_Buffer = e.get_S_V()
            self.RW_K_Buffer = e.get_RW_K()
            self.RW_V_Buffer = e.get_RW_V()
            self.HH_K_Buffer = e.get_HH_K()
            self.HH_V_Buffer = e.get_HH_V()
            self.HH_token_ids = e.get_HH_token_ids()
            self.HH_scores = e.get_HH_scores()
            self.Global_Attn_Scr = e.get_global_attn_scores()
            self.WR_K_Buffer = e.get_WR_K()
            self.WR_V_Buffer = e.get_WR_V()
            self.WR_token_ids = e.get_WR_token_ids()
        else:
            f32 = dict(dtype=torch.float32, device=DEVICE)
            self.S_K_Buffer = torch.empty((SINK_SIZE, num_heads, head_dim), **f32)
            self.S_V_Buffer = torch.empty((SINK_SIZE, num_heads, head_dim), **f32)
            self.RW_K_Buffer = torch.empty((R_size, num_heads, head_dim), **f32)
            self.RW_V_Buffer = torch.empty((R_size, num_heads, head_dim), **f32)
            self.HH_K_Buffer = torch.empty((self.max_heavy_hitters, num_heads, head_dim), **f32)
            self.HH_V_Buffer = torch.empty((self.max_heavy_hitters, num_heads, head_dim), **f32)
            self.HH_token_ids = torch.full((self.max_heavy_hitters,), -1, dtype=torch.int64, device=DEVICE)
            self.HH_scores = torch.empty((self.max_heavy_hitters,), **f32)
            self.Global_Attn_Scr = torch.zeros((max_seq_len,), **f32)
            self.WR_K_Buffer = torch.empty((CHUNK_SIZE, num_heads, head_dim), **f32)
            self.WR_V_Buffer = torch.empty((CHUNK_SIZE, num_heads, head_dim), **f32)
            self.WR_token_ids = torch.full((CHUNK_SIZE,), -1, dtype=torch.int64, device=DEVICE)

        self.num_blocks = math.ceil(self.max_background_tokens / CHUNK_SIZE)
        self.quant_head_dim = math.ceil(head_dim / 16)
        self.PBS_is_full = False
        self.PBS_block_head_index = 0

    # ------------------------------------------------------------------
    # Counters: read from the engine (device) when present, else Python state.
    # ------------------------------------------------------------------
    def _counter(self, name):
        e = self.__dict__.get("_engine")
        if e is not None:
            return e.counters()[_ENGINE_COUNTERS[name]]
        return self.__dict__["_py_" + name]

    def __getattr__(self, name):
        if name in _PY_PBS:
            self._alloc_python_pbs()
            return self.__dict__[name]
        raise AttributeError(f"'{type(self).__name__}' object has no attribute '{name}'")

    def _alloc_python_pbs(self):
        d = self.__dict__
        nb, H, D = self.num_blocks, self.num_heads, self.head_dim
        d["PBS_K_Packed"] = torch.empty((nb, H, D), dtype=torch.int32, device=DEVICE)
        d["PBS_K_Scales"] = torch.empty((nb, H, D), dtype=torch.float32, device=DEVICE)
        d["PBS_K_Zeroes"] = torch.empty((nb, H, D), dtype=torch.float32, device=DEVICE)
        d["PBS_V_Packed"] = torch.empty((nb * CHUNK_SIZE, H, self.quant_head_dim), dtype=torch.int32, device=DEVICE)
        d["PBS_V_Scales"] = torch.empty((nb * CHUNK_SIZE, H, 1), dtype=torch.float32, device=DEVICE)
        d["PBS_V_Zeroes"] = torch.empty((nb * CHUNK_SIZE, H, 1), dtype=torch.float32, device=DEVICE)
        d["PBS_token_ids"] = torch.full((nb * CHUNK_SIZE,), -1, dtype=torch.int64, device=DEVICE)

    # ------------------------------------------------------------------
    # Engine entry points (cache.py:101-154)
    # ------------------------------------------------------------------
    def step(self, Q: torch.Tensor, K_new: torch.Tensor, V_new: torch.Tensor, attn_output: torch.Tensor):
        """One decode step: ingest, attention over all tiers, score feedback."""
        if self._engine is None:
            raise NotImplementedError("C++ engine not initialized")
        self._engine.step(Q, K_new, V_new, attn_output)

    def step_with_weights(self, Q, K_new, V_new, attn_output):
        """step() returning this step's per-head attention weights and token ids,
        ordered like the reference's reconstruct_full_cache() (sinks, heavy
        hitters and packed tokens sorted by token id, recent window oldest first)."""
        if self._engine is None:
            raise NotImplementedError("C++ engine not initialized")
        w = self._engine.step_with_weights(Q, K_new, V_new, attn_output)
        ids = self._visible_token_ids(w.device)
        c = self._engine.counters()
        s, hh, rw = c["s_count"], c["hh_count"], c["rw_count"]
        nd = s + hh + rw
        mid_ids = torch.cat([ids[s:s + hh], ids[nd:]])
        order = torch.argsort(mid_ids)
        perm = torch.cat([torch.arange(s, device=w.device),
                          torch.cat([torch.arange(s, s + hh, device=w.device),
                                     torch.arange(nd, ids.numel(), device=w.device)])[order],
                          torch.arange(s + hh, nd, device=w.device)])
        return w[:, perm], ids[perm]

    def _visible_token_ids(self, device):
        e = self._engine
        c = e.counters()
        s, hh, rw, nb = c["s_count"], c["hh_count"], c["rw_count"], c["pbs_blocks_used"]
        total = c["total_processed_tokens"]
        parts = [torch.arange(s, device=device, dtype=torch.int64), e.get_HH_token_ids()[:hh].to(device),
                 torch.arange(total - rw, total, device=device, dtype=torch.int64),
                 e.get_PBS_token_ids()[: nb * e.chunk_size].to(device)]
        return torch.cat(parts)

    def prefill(self, K_tokens: torch.Tensor, V_tokens: torch.Tensor) -> None:
        """Ingest a batch of prompt tokens. K_tokens, V_tokens: [q_len, num_heads, head_dim]."""
        q_len = K_tokens.shape[0]
        if self._engine is not None:
            self._engine.prefill(K_tokens.to(torch.float32).contiguous(), V_tokens.to(torch.float32).contiguous(), q_len)
        else:
            for i in range(q_len):
                self.ingest_token(K_tokens[i], V_tokens[i])

    def get_buffer_bytes(self) -> int:
        """Allocated cache bytes (the engine's tier accounting when present)."""
        if self._engine is not None:
            return self._engine.get_buffer_bytes()
        tensors = [self.S_K_Buffer, self.S_V_Buffer, self.RW_K_Buffer, self.RW_V_Buffer, self.HH_K_Buffer,
                   self.HH_V_Buffer, self.HH_token_ids, self.HH_scores, self.WR_K_Buffer, self.WR_V_Buffer,
                   self.WR_token_ids, self.PBS_K_Packed, self.PBS_K_Scales, self.PBS_K_Zeroes, self.PBS_V_Packed,
                   self.PBS_V_Scales, self.PBS_V_Zeroes, self.PBS_token_ids, self.Global_Attn_Scr]
        return sum(t.element_size() * t.nelement() for t in tensors if t is not None)

    def assert_evictions_occurred(self) -> None:
        """Checks that a run reached the compressed tiers (cache.py:156-162)."""
        assert self.total_evictions > 0 or self.PBS_count > 0 or self.HH_count > 0, (
            f"TriTierCache ran with 0 evictions (total_tokens={self.Total_Processed_Tokens}, "
            f"R_size={self.R_size}, HH_count={self.HH_count}, PBS_count={self.PBS_count}). "
            "Quality benchmarks must run at context length >= 4x R_size to exercise compression tiers!")

    # ------------------------------------------------------------------
    # The reference's pure-PyTorch tier path (cache.py:164-372)
    # ------------------------------------------------------------------
    def accumulate_attn_scrs(self, attn_weights: torch.Tensor, full_ids=None) -> None:
        """Average attention over heads and add it to the global scores (undecayed)."""
        if attn_weights.dim() == 4:
            if attn_weights.shape[2] > 1:
                raise RuntimeError("Multi-token prefill not supported in single-step accumulate")
            per_token = attn_weights.squeeze(0).squeeze(1)
        elif attn_weights.dim() == 3:
            per_token = attn_weights.squeeze(1)
        else:
            per_token = attn_weights
        mean_scores = per_token.mean(dim=0)
        if full_ids is not None:
            keep = full_ids != -1
            self.Global_Attn_Scr.index_add_(0, full_ids[keep], mean_scores[keep])
        else:
            self.Global_Attn_Scr[0:mean_scores.shape[0]] += mean_scores

    def fetch_or_calc_thresh(self, total_processed_tokens: int):
        """95th-percentile threshold, recomputed every UPDATE_THRESHOLD tokens or while zero."""
        thr = self.current_threshold
        is_zero = (thr.item() == 0.0) if isinstance(thr, torch.Tensor) else (float(thr) == 0.0)
        if total_processed_tokens % UPDATE_THRESHOLD == 0 or is_zero:
            n = self.Total_Processed_Tokens if self.Total_Processed_Tokens > 0 else total_processed_tokens
            scores = self.Global_Attn_Scr[:n]
            if len(scores) > 0:
                self.current_threshold = torch.quantile(scores, 0.95)
        if isinstance(self.current_threshold, (int, float)):
            return torch.tensor(float(self.current_threshold))
        return self.current_threshold

    def ingest_token(self, K: torch.Tensor, V: torch.Tensor) -> None:
        """Sink / recent-window fill; ring eviction routes the oldest token."""
        if self.S_count < SINK_SIZE:
            self.S_K_Buffer[self.S_count] = K
            self.S_V_Buffer[self.S_count] = V
            self.S_count += 1
            self.Total_Processed_Tokens += 1
            return
        if self.RW_count < self.R_size:
            self.RW_K_Buffer[self.RW_count] = K
            self.RW_V_Buffer[self.RW_count] = V
            self.RW_count += 1
            self.Total_Processed_Tokens += 1
            return
        slot = self.RW_head_index
        evicted_id = self.Total_Processed_Tokens - self.R_size
        ek = self.RW_K_Buffer[slot].clone()
        ev = self.RW_V_Buffer[slot].clone()
        self.RW_K_Buffer[slot] = K
        self.RW_V_Buffer[slot] = V
        self.RW_head_index = (self.RW_head_index + 1) % self.R_size
        self.Total_Processed_Tokens += 1
        self.route_evicted_token(ek, ev, evicted_id)

    def route_evicted_token(self, K: torch.Tensor, V: torch.Tensor, token_id: int):
        """Heavy-hitter promotion / demotion against the cached threshold."""
        self.total_evictions += 1
        g = self.Global_Attn_Scr[token_id]
        score = g.item() if isinstance(g, torch.Tensor) else float(g)
        thr = self.current_threshold
        thr = thr.item() if isinstance(thr, torch.Tensor) else float(thr)
        if score >= thr:
            if self.HH_count < self.max_heavy_hitters:
                i = self.HH_count
                self.HH_K_Buffer[i] = K
                self.HH_V_Buffer[i] = V
                self.HH_token_ids[i] = token_id
                self.HH_scores[i] = score
                self.HH_count += 1
                return
            min_score, min_idx = torch.min(self.HH_scores[:self.HH_count], dim=0)
            if score > min_score.item():
                dk = self.HH_K_Buffer[min_idx].clone()
                dv = self.HH_V_Buffer[min_idx].clone()
                did = self.HH_token_ids[min_idx].clone()
                self.HH_K_Buffer[min_idx] = K
                self.HH_V_Buffer[min_idx] = V
                self.HH_token_ids[min_idx] = token_id
                self.HH_scores[min_idx] = score
                self.compress_and_store(dk, dv, did)
                return
        self.compress_and_store(K, V, token_id)

    def compress_and_store(self, K: torch.Tensor, V: torch.Tensor, token_id: int):
        """Waiting-room append; a full room is packed into the next block."""
        i = self.WR_count
        self.WR_K_Buffer[i] = K
        self.WR_V_Buffer[i] = V
        self.WR_token_ids[i] = token_id
        self.WR_count += 1
        if self.WR_count == CHUNK_SIZE:
            self._quantize_and_store()

    def _quantize_and_store(self):
        """Pure-PyTorch 2-bit packing of the waiting room (reference semantics:
        scale 0 -> 1, unfused dequant, FP32 metadata only)."""
        blk = self.PBS_block_head_index
        dev = self.WR_K_Buffer.device
        k = self.WR_K_Buffer.unsqueeze(0)
        v = self.WR_V_Buffer.unsqueeze(0)
        kmin = k.min(dim=1, keepdim=True).values
        kscale = (k.max(dim=1, keepdim=True).values - kmin) / 3.0
        kscale[kscale == 0] = 1.0
        kq = torch.clamp(torch.round((k - kmin) / kscale), 0, 3).to(torch.int32)
        tshift = torch.arange(0, 32, 2, dtype=torch.int32, device=dev).view(1, CHUNK_SIZE, 1, 1)
        self.PBS_K_Packed[blk] = torch.bitwise_left_shift(kq, tshift).sum(dim=1).squeeze(0)
        self.PBS_K_Scales[blk] = kscale.squeeze(0).squeeze(0)
        self.PBS_K_Zeroes[blk] = kmin.squeeze(0).squeeze(0)

        vmin = v.min(dim=-1, keepdim=True).values
        vscale = (v.max(dim=-1, keepdim=True).values - vmin) / 3.0
        vscale[vscale == 0] = 1.0
        vq = torch.clamp(torch.round((v - vmin) / vscale), 0, 3).to(torch.int32)
        padded = self.quant_head_dim * 16
        if self.head_dim < padded:
            vq = torch.nn.functional.pad(vq, (0, padded - self.head_dim))
        vq = vq.view(1, CHUNK_SIZE, self.num_heads, self.quant_head_dim, 16)
        cshift = torch.arange(0, 32, 2, dtype=torch.int32, device=dev).view(1, 1, 1, 16)
        lo, hi = blk * CHUNK_SIZE, (blk + 1) * CHUNK_SIZE
        self.PBS_V_Packed[lo:hi] = torch.bitwise_left_shift(vq, cshift).sum(dim=-1).squeeze(0)
        self.PBS_V_Scales[lo:hi] = vscale.squeeze(0)
        self.PBS_V_Zeroes[lo:hi] = vmin.squeeze(0)
        self.PBS_token_ids[lo:hi] = self.WR_token_ids.clone()
        self.PBS_count += CHUNK_SIZE
        self.PBS_block_head_index = (self.PBS_block_head_index + 1) % self.num_blocks
        self.WR_count = 0
        self.WR_token_ids.fill_(-1)

    def reconstruct_full_cache(self):
        """Dequantised view of every attended token: sinks, heavy hitters and
        valid packed tokens sorted by id, then the recent window oldest first
        (cache.py:326-372 of the reference). With the device engine the tiers
        are read from the engine (either block size, either metadata type)."""
        if self._engine is not None:
            return self._reconstruct_engine()
        dev = self.S_K_Buffer.device
        sk = self.S_K_Buffer[0:self.S_count]
        sv = self.S_V_Buffer[0:self.S_count]
        sids = torch.arange(0, self.S_count, device=dev)

        tshift = torch.arange(0, 32, 2, dtype=torch.int32, device=dev).view(1, 16, 1, 1)
        kq = torch.bitwise_and(torch.bitwise_right_shift(self.PBS_K_Packed.unsqueeze(1), tshift), 0b11)
        kq = kq.reshape(self.num_blocks * CHUNK_SIZE, self.num_heads, self.head_dim)
        t3k = (kq.float() * self.PBS_K_Scales.repeat_interleave(CHUNK_SIZE, dim=0)
               + self.PBS_K_Zeroes.repeat_interleave(CHUNK_SIZE, dim=0))
        cshift = torch.arange(0, 32, 2, dtype=torch.int32, device=dev)
        vq = torch.bitwise_and(torch.bitwise_right_shift(self.PBS_V_Packed.unsqueeze(-1), cshift), 0b11)
        vq = vq.reshape(self.num_blocks * CHUNK_SIZE, self.num_heads, self.quant_head_dim * 16)[..., :self.head_dim]
        t3v = vq.float() * self.PBS_V_Scales + self.PBS_V_Zeroes
        keep = self.PBS_token_ids != -1
        t3k, t3v, t3ids = t3k[keep], t3v[keep], self.PBS_token_ids[keep]

        mk = torch.cat([self.HH_K_Buffer[0:self.HH_count], t3k], dim=0)
        mv = torch.cat([self.HH_V_Buffer[0:self.HH_count], t3v], dim=0)
        mids = torch.cat([self.HH_token_ids[0:self.HH_count], t3ids], dim=0)
        if len(mids) > 0:
            perm = torch.argsort(mids)
            mk, mv, mids = mk[perm], mv[perm], mids[perm]

        if self.RW_count < self.R_size:
            rk = self.RW_K_Buffer[0:self.RW_count]
            rv = self.RW_V_Buffer[0:self.RW_count]
            rids = torch.arange(self.S_count, self.S_count + self.RW_count, device=dev)
        else:
            rk = torch.roll(self.RW_K_Buffer, shifts=-self.RW_head_index, dims=0)
            rv = torch.roll(self.RW_V_Buffer, shifts=-self.RW_head_index, dims=0)
            rids = torch.arange(self.Total_Processed_Tokens - self.R_size, self.Total_Processed_Tokens, device=dev)

        return (torch.cat([sk, mk, rk], dim=0), torch.cat([sv, mv, rv], dim=0),
                torch.cat([sids, mids, rids], dim=0))


def _meta_f32(t: torch.Tensor) -> torch.Tensor:
    """Scale / zero metadata as f32 (FP16 metadata is kept as uint16 bits)."""
    return t.view(torch.float16).float() if t.dtype == torch.uint16 else t


def _reconstruct_engine(self):
    """reconstruct_full_cache() over the engine's device tiers."""
    e = self._engine
    c = e.counters()
    s, hh, rw, nb = c["s_count"], c["hh_count"], c["rw_count"], c["pbs_blocks_used"]
    total, head = c["total_processed_tokens"], c["rw_head_index"]
    H, D, kgs = self.num_heads, self.head_dim, e.k_group_size
    sk, sv = e.get_S_K()[:s], e.get_S_V()[:s]
    dev = sk.device
    sids = torch.arange(0, s, device=dev, dtype=torch.int64)

    # K words: [block][kgs / 16][H][D], token 16 w + t of a block at bits 2t of word w
    kp = e.get_PBS_K_Packed()[:nb]
    tshift = torch.arange(0, 32, 2, dtype=torch.int32, device=dev).view(1, 1, 16, 1, 1)
    kq = torch.bitwise_and(torch.bitwise_right_shift(kp.unsqueeze(2), tshift), 0b11).reshape(nb * kgs, H, D)
    t3k = (kq.float() * _meta_f32(e.get_PBS_K_Scales()[:nb]).repeat_interleave(kgs, dim=0)
           + _meta_f32(e.get_PBS_K_Zeroes()[:nb]).repeat_interleave(kgs, dim=0))
    # V words: [slot][H][D / 16], channel 16 g + i at bits 2i of word g
    vp = e.get_PBS_V_Packed()[: nb * kgs]
    cshift = torch.arange(0, 32, 2, dtype=torch.int32, device=dev)
    vq = torch.bitwise_and(torch.bitwise_right_shift(vp.unsqueeze(-1), cshift), 0b11).reshape(nb * kgs, H, -1)[..., :D]
    t3v = vq.float() * _meta_f32(e.get_PBS_V_Scales()[: nb * kgs]) + _meta_f32(e.get_PBS_V_Zeroes()[: nb * kgs])
    pids = e.get_PBS_token_ids()[: nb * kgs]
    keep = pids != -1
    mk = torch.cat([e.get_HH_K()[:hh], t3k[keep]], dim=0)
    mv = torch.cat([e.get_HH_V()[:hh], t3v[keep]], dim=0)
    mids = torch.cat([e.get_HH_token_ids()[:hh], pids[keep]], dim=0)
    if mids.numel() > 0:
        perm = torch.argsort(mids)
        mk, mv, mids = mk[perm], mv[perm], mids[perm]

    R = self.R_size
    if rw < R:
        rk, rv = e.get_RW_K()[:rw], e.get_RW_V()[:rw]
        rids = torch.arange(s, s + rw, device=dev, dtype=torch.int64)
    else:
        rk = torch.roll(e.get_RW_K(), shifts=-head, dims=0)
        rv = torch.roll(e.get_RW_V(), shifts=-head, dims=0)
        rids = torch.arange(total - R, total, device=dev, dtype=torch.int64)
    return (torch.cat([sk, mk, rk], dim=0), torch.cat([sv, mv, rv], dim=0), torch.cat([sids, mids, rids], dim=0))


TriTierCache._reconstruct_engine = _reconstruct_engine


def _counter_property(name):
    def get(self):
        return self._counter(name)

    def set(self, value):
        if self.__dict__.get("_engine") is not None:
            raise AttributeError(f"{name} is owned by the device engine and read-only")
        self.__dict__["_py_" + name] = value

    return property(get, set)


for _n in _ENGINE_COUNTERS:
    setattr(TriTierCache, _n, _counter_property(_n))
del _n
