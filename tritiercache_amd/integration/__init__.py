from .patch_model import apply_patch, is_patched, patched_forward, remove_patch, reset_caches

__all__ = ["apply_patch", "remove_patch", "reset_caches", "is_patched", "patched_forward"]
