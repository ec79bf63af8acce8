"""Per-tier KV-cache memory accounting.

``measure_cache_bytes`` is the reference's canonical accounting
(benchmarks/common.py:184-307 there): same arguments, same defaults, same keys,
same arithmetic. Given a token count it partitions the tokens into the tiers the
way a full cache holds them (4 sinks, then the recent window, then
ceil(total * h_ratio) heavy hitters, the rest 2-bit packed) and prices each tier
per layer:

* sinks and recent window: K + V in FP32;
* heavy hitters: K + V in FP32, plus an int64 token id and an FP32 score each;
* packed payload: 2 bits per element for K and for V;
* packed metadata: a scale and a zero per (K block, head, channel) and per
  (V token, head), in FP16 or FP32, plus an int64 token id per packed token.

It also reports the uncompressed FP16 / FP32 K+V sizes and the compression ratios
against them.

``live_cache_bytes`` prices what an engine actually holds, from its device
counters (sinks, ring, heavy hitters and flushed blocks as they are, the waiting
room separately), with the same per-tier rules and the same keys.
"""
from __future__ import annotations

import math
from typing import Any, Dict, Optional

_MB = 1024.0 * 1024.0


def _tier_bytes(sinks: int, rw: int, hh: int, pbs: int, kv_heads: int, head_dim: int, k_group_size: int,
                meta_bytes: int) -> Dict[str, float]:
    """Bytes of one layer's tiers holding the given token counts."""
    row = kv_heads * head_dim  # elements of one token's K (or V)
    k_blocks = math.ceil(pbs / k_group_size) if pbs > 0 else 0
    return {
        "sink": 2 * sinks * row * 4,
        "rw": 2 * rw * row * 4,
        "hh": 2 * hh * row * 4 + hh * (8 + 4),
        "payload": 2 * pbs * row * 0.25,
        "metadata": k_blocks * row * 2 * meta_bytes + pbs * kv_heads * 2 * meta_bytes + pbs * 8,
    }


def _report(total_tokens, num_layers, kv_heads, head_dim, counts, per_layer) -> Dict[str, Any]:
    sinks, rw, hh, pbs = counts
    layer_total = sum(per_layer.values())
    total = layer_total * num_layers
    vanilla = 2 * num_layers * total_tokens * kv_heads * head_dim
    return {
        "total_tokens": total_tokens,
        "num_layers": num_layers,
        "num_kv_heads": kv_heads,
        "head_dim": head_dim,
        "actual_sinks": sinks,
        "actual_rw": rw,
        "actual_hh": hh,
        "actual_pbs": pbs,
        "sink_bytes": per_layer["sink"] * num_layers,
        "rw_bytes": per_layer["rw"] * num_layers,
        "hh_bytes": per_layer["hh"] * num_layers,
        "pbs_payload_bytes": per_layer["payload"] * num_layers,
        "pbs_metadata_bytes": per_layer["metadata"] * num_layers,
        "total_bytes": total,
        "total_mb": total / _MB,
        "vanilla_fp16_bytes": vanilla * 2,
        "vanilla_fp16_mb": vanilla * 2 / _MB,
        "vanilla_fp32_bytes": vanilla * 4,
        "vanilla_fp32_mb": vanilla * 4 / _MB,
        "compression_ratio_vs_fp16": vanilla * 2 / max(1.0, total),
        "compression_ratio_vs_fp32": vanilla * 4 / max(1.0, total),
    }


def measure_cache_bytes(cache_obj: Any = None, total_tokens: Optional[int] = None, config: Optional[Any] = None,
                        num_kv_heads: Optional[int] = None, head_dim: Optional[int] = None, num_layers: int = 1,
                        sink_size: int = 4, r_size: int = 256, h_ratio: float = 0.05, chunk_size: int = 16,
                        k_group_size: int = 16, pbs_metadata_dtype: str = "fp16") -> Dict[str, Any]:
    """Per-tier byte breakdown of a cache holding `total_tokens` tokens, summed over
    `num_layers` layers (benchmarks/common.py:184-307 of the reference).

    Shapes come from, in order of precedence: `cache_obj` (its num_heads, head_dim,
    R_size, H_ratio, and Total_Processed_Tokens when total_tokens is None), an HF
    `config` (num_hidden_layers, num_key_value_heads, head_dim or hidden_size /
    num_attention_heads), the keyword arguments, and finally 3 KV heads of
    head_dim 64 when none gives them. `chunk_size` is accepted for the
    reference's signature and not used (the packed blocks are k_group_size
    tokens)."""
    if config is not None:
        num_layers = getattr(config, "num_hidden_layers", num_layers)
        num_kv_heads = getattr(config, "num_key_value_heads", getattr(config, "num_attention_heads", num_kv_heads))
        head_dim = getattr(config, "head_dim",
                           getattr(config, "hidden_size", 0) // getattr(config, "num_attention_heads", 1))
    if cache_obj is not None:
        num_kv_heads = getattr(cache_obj, "num_heads", num_kv_heads)
        head_dim = getattr(cache_obj, "head_dim", head_dim)
        r_size = getattr(cache_obj, "R_size", r_size)
        h_ratio = getattr(cache_obj, "H_ratio", h_ratio)
        if total_tokens is None:
            total_tokens = getattr(cache_obj, "Total_Processed_Tokens", 0)
    if num_kv_heads is None or head_dim is None:
        num_kv_heads, head_dim = 3, 64
    total_tokens = total_tokens or 0

    # the canonical partition of a full cache
    sinks = min(sink_size, total_tokens)
    rw = min(r_size, max(0, total_tokens - sinks))
    hh = min(math.ceil(total_tokens * h_ratio), max(0, total_tokens - sinks - rw))
    pbs = max(0, total_tokens - sinks - rw - hh)
    meta = 2 if pbs_metadata_dtype == "fp16" else 4
    per_layer = _tier_bytes(sinks, rw, hh, pbs, num_kv_heads, head_dim, k_group_size, meta)
    return _report(total_tokens, num_layers, num_kv_heads, head_dim, (sinks, rw, hh, pbs), per_layer)


def live_cache_bytes(cache: Any, num_layers: int = 1) -> Dict[str, Any]:
    """The same breakdown for what a TriTierCache's engine holds now, read from its
    device counters: its sinks, recent window and heavy hitters as counted, its
    flushed packed tokens (pbs_count, priced per k_group_size block), and the
    waiting room's FP32 rows under "wr_bytes" (not part of total_bytes, like the
    reference's accounting, which has no waiting-room tier). `num_layers` scales
    one cache to a model whose layers hold the same state."""
    c = cache._engine.counters()
    kv_heads, head_dim = cache.num_heads, cache.head_dim
    meta = 2 if cache.pbs_metadata_dtype == "fp16" else 4
    counts = (c["s_count"], c["rw_count"], c["hh_count"], c["pbs_count"])
    per_layer = _tier_bytes(*counts, kv_heads, head_dim, c["k_group_size"], meta)
    out = _report(c["total_processed_tokens"], num_layers, kv_heads, head_dim, counts, per_layer)
    out["actual_wr"] = c["wr_count"]
    out["wr_bytes"] = 2 * c["wr_count"] * kv_heads * head_dim * 4 * num_layers
    return out
