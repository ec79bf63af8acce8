"""TriTierCache: the Python API of the reference (src/tri_tier/cache.py) over the gfx950 engine.

Every TriTierCache owns one ``_C.TriTierCacheEngine``: the sink, recent-window,
heavy-hitter, waiting-room and packed tiers live in device memory and every
decode step runs as HIP kernels on the current stream. The constructor
arguments, attribute names and methods are the reference's
(cache.py:11-162 there); what differs is where the data lives:

* the tier buffers the reference exposes as zero-copy numpy views of host
  memory (cache.py:50-59) are zero-copy ROCm tensors viewing device memory;
* the counters the reference copies from the engine after each call
  (cache.py:110-116, 133-139) are read from the device when accessed, so a
  decode step never waits for the GPU;
* there is no CPU mode: constructing a TriTierCache without the native library
  or without a visible GPU raises RuntimeError. The reference's pure-PyTorch
  tier path (its ingest/route/pack methods, cache.py:164-372) is not part of
  this package; the engine's own routing (cache_engine.cpp) is the contract.
"""
from __future__ import annotations

import math

import torch

from .constants import SINK_SIZE, UPDATE_THRESHOLD

# Reference attribute name -> engine counter.
_COUNTERS = {
    "Total_Processed_Tokens": "total_processed_tokens",
    "total_evictions": "total_evictions",
    "PBS_count": "pbs_count",
    "RW_count": "rw_count",
    "RW_head_index": "rw_head_index",
    "S_count": "s_count",
    "HH_count": "hh_count",
    "WR_count": "wr_count",
}

# Reference attribute name -> engine getter of the device buffer it views.
_VIEWS = {
    "S_K_Buffer": "get_S_K", "S_V_Buffer": "get_S_V", "RW_K_Buffer": "get_RW_K", "RW_V_Buffer": "get_RW_V",
    "HH_K_Buffer": "get_HH_K", "HH_V_Buffer": "get_HH_V", "HH_token_ids": "get_HH_token_ids",
    "HH_scores": "get_HH_scores", "Global_Attn_Scr": "get_global_attn_scores", "WR_K_Buffer": "get_WR_K",
    "WR_V_Buffer": "get_WR_V", "WR_token_ids": "get_WR_token_ids",
}
# The packed store grows with the engine's allocation, so its views are taken
# at each access rather than once.
_PBS_VIEWS = {
    "PBS_K_Packed": "get_PBS_K_Packed", "PBS_K_Scales": "get_PBS_K_Scales", "PBS_K_Zeroes": "get_PBS_K_Zeroes",
    "PBS_V_Packed": "get_PBS_V_Packed", "PBS_V_Scales": "get_PBS_V_Scales", "PBS_V_Zeroes": "get_PBS_V_Zeroes",
    "PBS_token_ids": "get_PBS_token_ids",
}


class TriTierCache:
    def __init__(self, max_seq_len, head_dim, num_heads, R_size, H_ratio, num_q_heads=None, score_decay=0.999,
                 k_group_size=16, pbs_metadata_dtype="fp16"):
        """R_size: recent-window size; H_ratio: heavy-hitter fraction of max_seq_len.
        The engine is created on the current HIP device."""
        self.R_size = R_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_q_heads = num_q_heads if num_q_heads is not None else num_heads
        self.score_decay = score_decay
        self.k_group_size = 32 if k_group_size == 32 else 16
        self.pbs_metadata_dtype = "fp32" if str(pbs_metadata_dtype).lower() == "fp32" else "fp16"
        self.current_threshold = 0.0
        self.H_ratio = H_ratio
        self.max_seq_len = max_seq_len
        self.max_heavy_hitters = math.ceil(max_seq_len * H_ratio)
        self.max_background_tokens = max_seq_len - R_size - self.max_heavy_hitters
        self.num_blocks = math.ceil(self.max_background_tokens / self.k_group_size)
        self.quant_head_dim = math.ceil(head_dim / 16)
        self.PBS_is_full = False
        self.PBS_block_head_index = 0
        try:
            from . import _C

            decay = 1.0 if score_decay is None else float(score_decay)
            self._engine = _C.TriTierCacheEngine(self.num_q_heads, num_heads, head_dim, max_seq_len, SINK_SIZE,
                                                 R_size, H_ratio, decay, UPDATE_THRESHOLD, self.k_group_size,
                                                 self.pbs_metadata_dtype)
        except (ImportError, RuntimeError, ValueError, MemoryError) as e:
            raise RuntimeError(f"TriTierCache: the gfx950 engine could not be created: {e}") from e
        for name, getter in _VIEWS.items():
            setattr(self, name, getattr(self._engine, getter)())

    def __getattr__(self, name):
        # only reached for names not set in __init__
        if name in _PBS_VIEWS and "_engine" in self.__dict__:
            return getattr(self._engine, _PBS_VIEWS[name])()
        raise AttributeError(f"'{type(self).__name__}' object has no attribute '{name}'")

    # ------------------------------------------------------------------
    # Decode and prefill (cache.py:101-139)
    # ------------------------------------------------------------------
    def step(self, Q: torch.Tensor, K_new: torch.Tensor, V_new: torch.Tensor, attn_output: torch.Tensor):
        """One decode step: ingest the new token, attention over every tier, score feedback.
        Q [num_q_heads * head_dim], K_new / V_new [num_heads * head_dim], attn_output
        [num_q_heads * head_dim]; f32, contiguous, on the engine's device."""
        self._engine.step(Q, K_new, V_new, attn_output)

    def step_deferred(self, Q, K_new, V_new, attn_output, prev=None):
        """step() for the caches of a model's layers stepped one after another: the
        context vector is written as by step(), while this step's mean attention
        weights and score feedback stay pending and run in the finalize launch of
        the next cache stepped this way (`prev` is the cache stepped just before,
        on the same device, or None), or at the start of any later call on this
        cache. The tier state afterwards is the state step() leaves."""
        self._engine.step_deferred(Q, K_new, V_new, attn_output, None if prev is None else prev._engine)

    def flush_feedback(self):
        """Runs the pending mean weights and score feedback of the last step_deferred()."""
        self._engine.flush_feedback()

    def step_with_weights(self, Q, K_new, V_new, attn_output):
        """step() plus this step's per-head attention weights [num_q_heads, visible] and the
        token id of each column, ordered as reconstruct_full_cache() orders tokens (sinks,
        heavy hitters and packed tokens by token id, recent window oldest first)."""
        w = self._engine.step_with_weights(Q, K_new, V_new, attn_output)
        ids, perm = self._visible_order(w.device)
        return w[:, perm], ids[perm]

    def prefill(self, K_tokens: torch.Tensor, V_tokens: torch.Tensor) -> None:
        """Ingest a batch of prompt tokens. K_tokens, V_tokens: [q_len, num_heads, head_dim]."""
        q_len = K_tokens.shape[0]
        self._engine.prefill(K_tokens.to(torch.float32).contiguous(), V_tokens.to(torch.float32).contiguous(), q_len)

    def get_buffer_bytes(self) -> int:
        """The engine's accounting of allocated tier bytes (cache_engine.cpp:543-568)."""
        return self._engine.get_buffer_bytes()

    def assert_evictions_occurred(self) -> None:
        """Checks that a run reached the compressed tiers (cache.py:156-162)."""
        assert self.total_evictions > 0 or self.PBS_count > 0 or self.HH_count > 0, (
            f"TriTierCache ran with 0 evictions (total_tokens={self.Total_Processed_Tokens}, "
            f"R_size={self.R_size}, HH_count={self.HH_count}, PBS_count={self.PBS_count}). "
            "Quality benchmarks must run at context length >= 4x R_size to exercise compression tiers!")

    # ------------------------------------------------------------------
    # Views over the device tiers
    # ------------------------------------------------------------------
    def _visible_order(self, device):
        """Token ids of the engine's visible columns (sinks, heavy-hitter slots, recent
        window oldest first, packed slots) and the permutation that sorts the heavy
        hitters and packed slots by id between the sinks and the recent window."""
        e = self._engine
        c = e.counters()
        s, hh, rw, nb = c["s_count"], c["hh_count"], c["rw_count"], c["pbs_blocks_used"]
        total = c["total_processed_tokens"]
        ids = torch.cat([torch.arange(s, device=device, dtype=torch.int64),
                         e.get_HH_token_ids()[:hh].to(device),
                         torch.arange(total - rw, total, device=device, dtype=torch.int64),
                         e.get_PBS_token_ids()[: nb * e.chunk_size].to(device)])
        nd = s + hh + rw
        middle = torch.cat([torch.arange(s, s + hh, device=device), torch.arange(nd, ids.numel(), device=device)])
        middle = middle[torch.argsort(ids[middle])]
        perm = torch.cat([torch.arange(s, device=device), middle, torch.arange(s + hh, nd, device=device)])
        return ids, perm

    def reconstruct_full_cache(self):
        """(K, V, ids) of every token the next step attends to, dequantised: sinks, then
        heavy hitters and valid packed tokens sorted by token id, then the recent window
        oldest first (the order of the reference's cache.py:326-372). Either block size,
        either metadata dtype."""
        e = self._engine
        c = e.counters()
        s, hh, rw, nb = c["s_count"], c["hh_count"], c["rw_count"], c["pbs_blocks_used"]
        total, head = c["total_processed_tokens"], c["rw_head_index"]
        H, D, kgs = self.num_heads, self.head_dim, e.k_group_size
        sk, sv = e.get_S_K()[:s], e.get_S_V()[:s]
        dev = sk.device
        # Packed store through the library's own dequantisers (bit-exact with the
        # reference's dequantize_k / dequantize_v).
        from . import _C

        t3k = torch.empty((nb * kgs, H, D), dtype=torch.float32, device=dev)
        t3v = torch.empty((nb * kgs, H, D), dtype=torch.float32, device=dev)
        if nb > 0:
            _C.dequantize_k(e.get_PBS_K_Packed()[:nb], e.get_PBS_K_Scales()[:nb], e.get_PBS_K_Zeroes()[:nb], t3k,
                            nb, H, D, kgs, self.pbs_metadata_dtype)
            _C.dequantize_v(e.get_PBS_V_Packed()[: nb * kgs], e.get_PBS_V_Scales()[: nb * kgs],
                            e.get_PBS_V_Zeroes()[: nb * kgs], t3v, nb * kgs, H, D, self.pbs_metadata_dtype)
        pids = e.get_PBS_token_ids()[: nb * kgs]
        keep = pids != -1
        mk = torch.cat([e.get_HH_K()[:hh], t3k[keep]])
        mv = torch.cat([e.get_HH_V()[:hh], t3v[keep]])
        mids = torch.cat([e.get_HH_token_ids()[:hh], pids[keep]])
        order = torch.argsort(mids)
        mk, mv, mids = mk[order], mv[order], mids[order]
        ring = (torch.arange(rw, device=dev) + (head if rw == self.R_size else 0)) % max(rw, 1)
        rk, rv = e.get_RW_K()[ring], e.get_RW_V()[ring]
        rids = torch.arange(total - rw, total, device=dev, dtype=torch.int64)
        sids = torch.arange(s, device=dev, dtype=torch.int64)
        return torch.cat([sk, mk, rk]), torch.cat([sv, mv, rv]), torch.cat([sids, mids, rids])


def _counter_property(name):
    key = _COUNTERS[name]

    def get(self):
        return self._engine.counters()[key]

    def set(self, value):
        raise AttributeError(f"{name} is owned by the device engine and read-only")

    return property(get, set, doc=f"Engine counter {key} (read from the device).")


for _n in _COUNTERS:
    setattr(TriTierCache, _n, _counter_property(_n))
del _n
