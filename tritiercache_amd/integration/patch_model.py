"""HF attention patch for LLaMA / Mistral / Qwen2 / Qwen3 (reference src/tri_tier/integration/patch_model.py).

``patched_forward`` replaces the ``forward`` of the supported attention
classes. Prefill runs SDPA over the prompt and bulk-ingests the prompt's K/V
into the layer's TriTierCache; decode hands Q and the new K/V to the
device-resident engine, which runs the fused tiered attention on the GPU.
Tensors stay on the model's device: on a ROCm model nothing crosses to the
host (the reference flattens to FP32 CPU tensors, patch_model.py:151-155).

With output_attentions=True the engine also returns this step's per-head
attention weights (ordered like the reference's reconstruct_full_cache()).
Without an engine (CPU-only opt-in mode) the reference's pure-PyTorch path is
used, as in the reference.
"""
from typing import Any, Dict, List, Optional, Tuple, Type

import torch

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


def _reference_attention_path(self, cache: TriTierCache, Q: torch.Tensor, num_q_heads: int, num_kv_heads: int,
                              head_dim: int):
    """Dense attention over the reconstructed cache (patch_model.py:33-51)."""
    K_full, V_full, full_ids = cache.reconstruct_full_cache()
    if num_q_heads != num_kv_heads:
        rep = num_q_heads // num_kv_heads
        K_full = K_full.repeat_interleave(rep, dim=1)
        V_full = V_full.repeat_interleave(rep, dim=1)
    K_full = K_full.transpose(0, 1).unsqueeze(0).to(dtype=Q.dtype)
    V_full = V_full.transpose(0, 1).unsqueeze(0).to(dtype=Q.dtype)
    scaling = getattr(self, "scaling", None) or (head_dim ** -0.5)
    scores = torch.matmul(Q, K_full.transpose(-2, -1).contiguous()) * scaling
    weights = torch.softmax(scores, dim=-1)
    cache.accumulate_attn_scrs(weights, full_ids)
    return torch.matmul(weights, V_full), weights


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def patched_forward(self, hidden_states: torch.Tensor,
                    position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                    attention_mask: Optional[torch.Tensor] = None, past_key_values: Optional[Any] = None, **kwargs):
    """Forward of LlamaAttention / MistralAttention / Qwen2Attention / Qwen3Attention."""
    bsz, q_len, _ = hidden_states.shape
    assert bsz == 1, "TriTierCache only supports batch_size=1"

    num_q_heads = self.config.num_attention_heads
    num_kv_heads = getattr(self.config, "num_key_value_heads", num_q_heads)
    head_dim = getattr(self, "head_dim", None) or (self.config.hidden_size // num_q_heads)
    max_pos = getattr(self.config, "max_position_embeddings", MAX_SEQ_LEN)
    seq_len_cap = max(MAX_SEQ_LEN, max_pos)

    if getattr(self, "tri_tier_cache", None) is None:
        self.tri_tier_cache = TriTierCache(
            max_seq_len=seq_len_cap, head_dim=head_dim, num_heads=num_kv_heads, R_size=R_SIZE, H_ratio=H_RATIO,
            num_q_heads=num_q_heads, score_decay=SCORE_DECAY, k_group_size=K_GROUP_SIZE,
            pbs_metadata_dtype=PBS_METADATA_DTYPE)
    cache = self.tri_tier_cache

    q = self.q_proj(hidden_states).view(bsz, q_len, num_q_heads, head_dim)
    k = self.k_proj(hidden_states).view(bsz, q_len, num_kv_heads, head_dim)
    v = self.v_proj(hidden_states).view(bsz, q_len, num_kv_heads, head_dim)
    if getattr(self, "q_norm", None) is not None:
        q = self.q_norm(q)
    if getattr(self, "k_norm", None) is not None:
        k = self.k_norm(k)
    Q = q.transpose(1, 2)
    K_new = k.transpose(1, 2)
    V_new = v.transpose(1, 2)

    cos, sin = position_embeddings
    if cos.ndim == 3:
        cos = cos.unsqueeze(1)
        sin = sin.unsqueeze(1)
    Q = (Q * cos) + (_rotate_half(Q) * sin)
    K_new = (K_new * cos) + (_rotate_half(K_new) * sin)

    need_weights = kwargs.get("output_attentions", False)

    if q_len > 1:
        rep = num_q_heads // num_kv_heads
        K_exp = K_new.repeat_interleave(rep, dim=1) if rep > 1 else K_new
        V_exp = V_new.repeat_interleave(rep, dim=1) if rep > 1 else V_new
        ctx = torch.nn.functional.scaled_dot_product_attention(Q, K_exp, V_exp, is_causal=True)
        K_tokens = K_new.squeeze(0).transpose(0, 1).contiguous()
        V_tokens = V_new.squeeze(0).transpose(0, 1).contiguous()
        if getattr(self, "capture_needle_pos", None) is not None:
            pos = self.capture_needle_pos
            self.captured_needle_k = K_tokens[pos].clone()
            self.captured_needle_v = V_tokens[pos].clone()
        cache.prefill(K_tokens.float(), V_tokens.float())
        ctx = ctx.transpose(1, 2).reshape(bsz, q_len, -1)
        return self.o_proj(ctx), None

    if cache._engine is not None:
        Q_flat = Q.reshape(num_q_heads * head_dim).contiguous().float()
        K_flat = K_new.reshape(num_kv_heads * head_dim).contiguous().float()
        V_flat = V_new.reshape(num_kv_heads * head_dim).contiguous().float()
        out = torch.empty((num_q_heads * head_dim,), dtype=torch.float32, device=Q_flat.device)
        weights = None
        if need_weights:
            w, _ = cache.step_with_weights(Q_flat, K_flat, V_flat, out)
            weights = w.to(Q.device, dtype=Q.dtype).view(1, num_q_heads, 1, -1)
        else:
            cache.step(Q_flat, K_flat, V_flat, out)
        ctx = out.view(bsz, q_len, -1).to(dtype=hidden_states.dtype)
        return self.o_proj(ctx), weights

    cache.ingest_token(K_new.squeeze(0).squeeze(1).float(), V_new.squeeze(0).squeeze(1).float())
    ctx, weights = _reference_attention_path(self, cache, Q, num_q_heads, num_kv_heads, head_dim)
    ctx = ctx.transpose(1, 2).reshape(bsz, q_len, -1).to(dtype=hidden_states.dtype)
    return self.o_proj(ctx), weights


_SUPPORTED_ATTENTION_CLASSES: List[Type] = []
_ORIGINAL_FORWARDS: Dict[Type, Any] = {}
_IS_PATCHED: bool = False

for _mod, _cls in (("transformers.models.llama.modeling_llama", "LlamaAttention"),
                   ("transformers.models.mistral.modeling_mistral", "MistralAttention"),
                   ("transformers.models.qwen2.modeling_qwen2", "Qwen2Attention"),
                   ("transformers.models.qwen3.modeling_qwen3", "Qwen3Attention")):
    try:
        _SUPPORTED_ATTENTION_CLASSES.append(getattr(__import__(_mod, fromlist=[_cls]), _cls))
    except (ImportError, AttributeError):
        pass


def apply_patch():
    """Patch every supported attention class."""
    global _IS_PATCHED
    for cls in _SUPPORTED_ATTENTION_CLASSES:
        if cls not in _ORIGINAL_FORWARDS:
            _ORIGINAL_FORWARDS[cls] = cls.forward
        cls.forward = patched_forward
    _IS_PATCHED = True


def remove_patch():
    """Restore the original forwards."""
    global _IS_PATCHED
    for cls, fwd in _ORIGINAL_FORWARDS.items():
        cls.forward = fwd
    _IS_PATCHED = False


def reset_caches(model):
    """Drop every lazily created TriTierCache on the model's layers."""
    for module in model.modules():
        if hasattr(module, "tri_tier_cache"):
            delattr(module, "tri_tier_cache")


def is_patched(model_or_module=None) -> bool:
    """True while the patch is active."""
    if _IS_PATCHED:
        return True
    return any(getattr(cls, "forward", None) == patched_forward for cls in _SUPPORTED_ATTENTION_CLASSES)
