"""HF attention patch for the LLaMA, Mistral, Qwen2 and Qwen3 families on the gfx950 engine.

Public surface of the reference's src/tri_tier/integration/patch_model.py: the
module constants, ``patched_forward``, ``apply_patch``, ``remove_patch``,
``reset_caches``, ``is_patched``, ``HAS_CPP_EXT``, the per-module
``tri_tier_cache`` attribute and the ``capture_needle_pos`` hook.

Design: each patched attention module owns one TriTierCache, created lazily on
the module's own device. The projections, optional q/k norm and the family's
rotary embedding (the model file's own ``apply_rotary_pos_emb``) run as in the
unpatched model; then

* a prompt (q_len > 1) is attended causally with SDPA over its own keys
  (grouped-query heads shared in place, no repeated K/V) and bulk-ingested into
  the engine, whose tiers it fills in one prefill launch per tier;
* a decode token (q_len == 1) goes to the engine as three flat f32 device
  vectors; the engine's step (ring ingest, routing, packing, fused attention
  over every tier, score feedback) writes the context vector in device memory,
  which feeds ``o_proj`` directly. No tensor leaves the device and no step
  synchronises the host. The layers' steps are chained: each layer's mean
  attention weights and score feedback run in the next layer's finalize
  launch (the state afterwards is the state a per-layer step leaves). With
  output_attentions=True the step also returns the per-head weights over the
  attended tokens.

There is no path without the engine: a layer whose cache cannot be created
raises.
"""
from __future__ import annotations

import sys
import weakref
from typing import Any, Dict, List, Optional, Tuple, Type

import torch
import torch.nn.functional as F

from ..cache import TriTierCache

try:
    from .. import _C  # noqa: F401

    HAS_CPP_EXT = True
except ImportError:
    _C = None
    HAS_CPP_EXT = False

MAX_SEQ_LEN = 32768
R_SIZE = 256
H_RATIO = 0.05
SCORE_DECAY = 0.999
K_GROUP_SIZE = 16
PBS_METADATA_DTYPE = "fp16"

# (modeling module, attention class) of every family the patch serves.
_FAMILIES = (
    ("transformers.models.llama.modeling_llama", "LlamaAttention"),
    ("transformers.models.mistral.modeling_mistral", "MistralAttention"),
    ("transformers.models.qwen2.modeling_qwen2", "Qwen2Attention"),
    ("transformers.models.qwen3.modeling_qwen3", "Qwen3Attention"),
)


def _resolve_families() -> List[Type]:
    found = []
    for mod, name in _FAMILIES:
        try:
            found.append(getattr(__import__(mod, fromlist=[name]), name))
        except (ImportError, AttributeError):
            continue
    return found


_SUPPORTED_ATTENTION_CLASSES: List[Type] = _resolve_families()
_ORIGINAL_FORWARDS: Dict[Type, Any] = {}
# The cache a decode step last went through, per device: the next layer's step
# runs that cache's mean weights and score feedback in its own finalize launch.
_LAST_STEPPED: Dict[int, "weakref.ref"] = {}


def _shape(module) -> Tuple[int, int, int]:
    """(query heads, KV heads, head_dim) of an attention module."""
    cfg = module.config
    hq = cfg.num_attention_heads
    hkv = getattr(cfg, "num_key_value_heads", None) or hq
    d = getattr(module, "head_dim", None) or cfg.hidden_size // hq
    return hq, hkv, d


def _layer_cache(module, device: torch.device) -> TriTierCache:
    cache = getattr(module, "tri_tier_cache", None)
    if cache is None:
        hq, hkv, d = _shape(module)
        capacity = max(MAX_SEQ_LEN, getattr(module.config, "max_position_embeddings", MAX_SEQ_LEN))
        with torch.cuda.device(device):
            cache = TriTierCache(max_seq_len=capacity, head_dim=d, num_heads=hkv, R_size=R_SIZE, H_ratio=H_RATIO,
                                 num_q_heads=hq, score_decay=SCORE_DECAY, k_group_size=K_GROUP_SIZE,
                                 pbs_metadata_dtype=PBS_METADATA_DTYPE)
        module.tri_tier_cache = cache
    return cache


def _rotated_qkv(module, hidden_states, position_embeddings):
    """Q [1, Hq, q_len, D], K and V [1, Hkv, q_len, D] after projection, the
    family's q/k norm (Qwen3) and its rotary embedding."""
    hq, hkv, d = _shape(module)
    n = hidden_states.shape[1]
    q = module.q_proj(hidden_states).view(1, n, hq, d)
    k = module.k_proj(hidden_states).view(1, n, hkv, d)
    v = module.v_proj(hidden_states).view(1, n, hkv, d)
    if getattr(module, "q_norm", None) is not None:
        q = module.q_norm(q)
    if getattr(module, "k_norm", None) is not None:
        k = module.k_norm(k)
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    cos, sin = position_embeddings
    rope = _family_rope(type(module))
    if rope is not None:
        q, k = rope(q, k, cos, sin)
    else:
        q, k = _rotate_half_rope(q, cos, sin), _rotate_half_rope(k, cos, sin)
    return q, k, v


def _family_rope(cls):
    """The ``apply_rotary_pos_emb`` of the model file that defines the patched
    family class ``cls`` derives from (found through the MRO, so a subclass from
    another module, e.g. remote code, uses its family's), or None."""
    for base in cls.__mro__:
        if base in _SUPPORTED_ATTENTION_CLASSES or base is cls:
            fn = getattr(sys.modules.get(base.__module__), "apply_rotary_pos_emb", None)
            if fn is not None:
                return fn
    return None


def _rotate_half_rope(x, cos, sin):
    """x * cos + rotate_half(x) * sin with cos/sin [1, q_len, D] broadcast over the
    heads, the rotation the reference applies inline (patch_model.py:104-116)."""
    if cos.ndim == 3:
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rot * sin


def patched_forward(self, hidden_states: torch.Tensor,
                    position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                    attention_mask: Optional[torch.Tensor] = None, past_key_values: Optional[Any] = None, **kwargs):
    """Forward of a patched LlamaAttention / MistralAttention / Qwen2Attention / Qwen3Attention.
    Returns (output, attention weights or None) like the unpatched forward."""
    bsz, q_len, _ = hidden_states.shape
    assert bsz == 1, "TriTierCache only supports batch_size=1"
    cache = _layer_cache(self, hidden_states.device)
    hq, hkv, d = _shape(self)
    q, k, v = _rotated_qkv(self, hidden_states, position_embeddings)

    if q_len > 1:
        ctx = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=hq != hkv)
        k_tok = k[0].transpose(0, 1).contiguous()  # [q_len, Hkv, D]
        v_tok = v[0].transpose(0, 1).contiguous()
        pos = getattr(self, "capture_needle_pos", None)
        if pos is not None:
            self.captured_needle_k = k_tok[pos].clone()
            self.captured_needle_v = v_tok[pos].clone()
        cache.prefill(k_tok, v_tok)
        return self.o_proj(ctx.transpose(1, 2).reshape(1, q_len, hq * d)), None

    q_vec = q.reshape(hq * d).float().contiguous()
    k_vec = k.reshape(hkv * d).float().contiguous()
    v_vec = v.reshape(hkv * d).float().contiguous()
    ctx = torch.empty(hq * d, dtype=torch.float32, device=hidden_states.device)
    weights = None
    if kwargs.get("output_attentions", False):
        w, _ = cache.step_with_weights(q_vec, k_vec, v_vec, ctx)
        weights = w.to(hidden_states.dtype).view(1, hq, 1, -1)
    else:
        # Chained through the model's layers: this layer's mean attention weights
        # and score feedback run in the next layer's finalize launch (or at this
        # cache's next call), so a decode step pays one finalize launch per layer.
        key = hidden_states.device.index if hidden_states.device.index is not None else -1
        ref = _LAST_STEPPED.get(key)
        prev = ref() if ref is not None else None
        cache.step_deferred(q_vec, k_vec, v_vec, ctx, prev=prev if prev is not cache else None)
        _LAST_STEPPED[key] = weakref.ref(cache)
    return self.o_proj(ctx.view(1, 1, hq * d).to(hidden_states.dtype)), weights


def apply_patch():
    """Route every supported attention class's forward through patched_forward."""
    for cls in _SUPPORTED_ATTENTION_CLASSES:
        _ORIGINAL_FORWARDS.setdefault(cls, cls.forward)
        cls.forward = patched_forward


def remove_patch():
    """Restore the forwards apply_patch replaced."""
    for cls, forward in _ORIGINAL_FORWARDS.items():
        cls.forward = forward


def reset_caches(model):
    """Drop the TriTierCache of every attention module of `model` (a new one is
    created on the next forward)."""
    for module in model.modules():
        if hasattr(module, "tri_tier_cache"):
            delattr(module, "tri_tier_cache")
    _LAST_STEPPED.clear()


def is_patched(model_or_module=None) -> bool:
    """True while any supported attention class runs patched_forward."""
    return any(cls.forward is patched_forward for cls in _SUPPORTED_ATTENTION_CLASSES)
