"""Constants of the TriTierCache Python API (reference src/tri_tier/constants.py:1-7).

DEVICE is where the Python-side buffers live: the ROCm device when one is
visible (the engine's tiers are device-resident), else the CPU.
"""
import torch

DEVICE = "cuda" if torch.cuda.is_available() else "cpu"

UPDATE_THRESHOLD = 32

CHUNK_SIZE = 16

SINK_SIZE = 4
