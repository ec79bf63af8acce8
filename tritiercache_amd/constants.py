"""Constants of the TriTierCache Python API (reference src/tri_tier/constants.py:1-7).

DEVICE names the device the engine's tiers live on when a GPU is visible
(the reference uses it for its Python-side buffers).
"""
import torch

DEVICE = "cuda" if torch.cuda.is_available() else "cpu"

UPDATE_THRESHOLD = 32

CHUNK_SIZE = 16

SINK_SIZE = 4
