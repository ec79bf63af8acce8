"""The HF patch's rotary-embedding lookup (CPU only): a patched family class and a
subclass of it from another module both use the family's own
apply_rotary_pos_emb, and the inline rotate-half fallback (the rotation the
reference applies inline, src/tri_tier/integration/patch_model.py:104-116)
equals the LLaMA file's function."""
import pytest
import torch

transformers = pytest.importorskip("transformers")


def test_family_rope_found_through_the_mro():
    from transformers.models.llama import modeling_llama
    from transformers.models.qwen2 import modeling_qwen2

    from tritiercache_amd.integration import patch_model

    class RemoteAttention(modeling_llama.LlamaAttention):  # defined in a module without the function
        pass

    assert patch_model._family_rope(modeling_llama.LlamaAttention) is modeling_llama.apply_rotary_pos_emb
    assert patch_model._family_rope(RemoteAttention) is modeling_llama.apply_rotary_pos_emb
    assert patch_model._family_rope(modeling_qwen2.Qwen2Attention) is modeling_qwen2.apply_rotary_pos_emb
    assert patch_model._family_rope(torch.nn.Module) is None


def test_inline_rope_matches_the_family_function():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    from tritiercache_amd.integration import patch_model

    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 8, 5, 64, generator=g)
    k = torch.randn(1, 2, 5, 64, generator=g)
    cos, sin = torch.randn(1, 5, 64, generator=g), torch.randn(1, 5, 64, generator=g)
    wq, wk = apply_rotary_pos_emb(q, k, cos, sin)
    assert torch.equal(patch_model._rotate_half_rope(q, cos, sin), wq)
    assert torch.equal(patch_model._rotate_half_rope(k, cos, sin), wk)
