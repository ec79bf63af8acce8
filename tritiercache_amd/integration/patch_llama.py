"""Import path of the reference's LLaMA patcher (src/tri_tier/integration/patch_llama.py),
kept so callers of ``tri_tier.integration.patch_llama`` find the same functions and
constants. The patch itself lives in patch_model."""
from .patch_model import (  # noqa: F401
    H_RATIO,
    HAS_CPP_EXT,
    K_GROUP_SIZE,
    MAX_SEQ_LEN,
    PBS_METADATA_DTYPE,
    R_SIZE,
    SCORE_DECAY,
    apply_patch,
    is_patched,
    patched_forward,
    remove_patch,
    reset_caches,
)

__all__ = ["apply_patch", "remove_patch", "reset_caches", "is_patched", "patched_forward", "MAX_SEQ_LEN", "R_SIZE",
           "H_RATIO", "SCORE_DECAY", "K_GROUP_SIZE", "PBS_METADATA_DTYPE", "HAS_CPP_EXT"]
