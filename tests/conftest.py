"""Test configuration: the `gpu` marker and import paths.

GPU tests (marked `gpu`) need an MI355X and the built native library; they call
the HIP path through the C ABI and compare with the oracle (oracle/) on the
same seeded inputs. Everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def oracle():
    from oracle.binding import load_oracle

    return load_oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle.binding import load_reference

    ref = load_reference()
    if ref is None:
        pytest.skip("compiled reference (oracle/_ref/libttref.so) not built here")
    return ref


@pytest.fixture(scope="session")
def golden():
    import json

    import numpy as np

    g = os.path.join(HERE, "golden")
    data = {
        "qv_kat": json.load(open(os.path.join(g, "quantize_v_kat.json"))),
        "tie_kat": json.load(open(os.path.join(g, "tie_kat.json"))),
        "kernels": dict(np.load(os.path.join(g, "kernels_small.npz"), allow_pickle=False)),
        "kernels_index": json.load(open(os.path.join(g, "kernels_small.json"))),
        "engine": json.load(open(os.path.join(g, "engine_digests.json"))),
    }
    return data
