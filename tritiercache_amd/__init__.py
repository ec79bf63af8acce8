"""TriTierCache on AMD Instinct MI355X (gfx950).

Drop-in for the reference package ``tri_tier``: ``TriTierCache`` (cache.py),
the constants, the HF attention patch (``integration``) and the native module
``_C`` -- here a ctypes layer over ``libtritiercache_amd.so``, whose HIP
kernels run the fused tiered decode step on the GPU.

The reference gates its extension on AVX2 (src/tri_tier/__init__.py:91-109);
this package gates on a visible HIP device. ``HAS_CPP_EXT`` is True when the
native library loads; the kernels additionally need a GPU at call time and
raise RuntimeError without one.
"""
from __future__ import annotations

import os

from .constants import CHUNK_SIZE, DEVICE, SINK_SIZE, UPDATE_THRESHOLD

try:
    from . import _C

    HAS_CPP_EXT = True
except ImportError:  # the native library was not built
    _C = None  # type: ignore[assignment]
    HAS_CPP_EXT = False


def is_gpu_supported() -> bool:
    """True when the native library is loaded and a HIP device is visible."""
    return HAS_CPP_EXT and _C.device_count() > 0


from .accounting import live_cache_bytes, measure_cache_bytes  # noqa: E402
from .cache import TriTierCache  # noqa: E402

__version__ = "0.1.0"

__all__ = [
    "TriTierCache",
    "measure_cache_bytes",
    "live_cache_bytes",
    "DEVICE",
    "UPDATE_THRESHOLD",
    "CHUNK_SIZE",
    "SINK_SIZE",
    "is_gpu_supported",
    "HAS_CPP_EXT",
    "_C",
    "__version__",
]
