import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "dsh-moss-tts_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path through the C ABI")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference compiled from its sources (oracle/_ref); skipped where it was never built."""
    from oracle import REF_SO, RefCpu
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref/libmossref.so not built here")
    return RefCpu(a16_mode="decode")


def golden(name):
    return np.load(os.path.join(GOLDEN, name))


@pytest.fixture(scope="session")
def golden_model():
    """The seeded synthetic model of tests/golden/model_small.npz, checked against its sha256."""
    import hashlib
    from mosship import moss_format as mf
    g = golden("model_small.npz")
    blob = mf.synth_model(int(g["seed"][0]), ln_random=True)
    assert hashlib.sha256(blob).digest() == g["sha256"].tobytes(), "synthetic model generator changed"
    return blob, g


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch


def max_rel(a, b):
    """max |a - b| / max |b| -- the tolerance metric used throughout (<= 1e-3 for fp)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))
