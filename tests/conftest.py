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


def q8t_rows(buf, m, K):
    """Rows [m][K] of an int8 GEMM operand in the matrix-core order: row r, column k at byte
    ((r // 16) * (K // 32) + k // 32) * 512 + 8 * (r % 16 + 16 * ((k % 32) // 8)) + k % 8."""
    r = np.arange(m)[:, None]
    k = np.arange(K)[None, :]
    off = ((r // 16) * (K // 32) + k // 32) * 512 + 8 * (r % 16 + 16 * ((k % 32) // 8)) + k % 8
    return np.asarray(buf).view(np.int8)[off]


def d8t_rows(buf, m, K):
    """Block scales [m][K / 32] of such an operand: block b of row r at float
    ((r // 16) * (K // 32) + b) * 16 + r % 16."""
    r = np.arange(m)[:, None]
    b = np.arange(K // 32)[None, :]
    return np.asarray(buf).view(np.float32)[((r // 16) * (K // 32) + b) * 16 + r % 16]


def check_quant(oracle, x, q, d, what):
    """Int8 values q (any integer dtype or integer-valued floats) and fp32 scales d of x
    against the oracle's quantize_row of x (quant.cpp:28-54), bit for bit; returns the
    count of values at +-127."""
    qr, _, dr = oracle.quantize_row(np.ascontiguousarray(x, np.float32))
    q = np.asarray(q)
    assert np.all(q == np.round(q)), what
    assert np.array_equal(q.astype(np.int32), qr.astype(np.int32)), f"{what}: int8 values differ"
    assert np.array_equal(np.asarray(d, np.float32).view(np.uint32), dr.view(np.uint32)), f"{what}: scales differ"
    return int(np.count_nonzero(np.abs(qr) == 127))


def max_rel(a, b):
    """max |a - b| / max |b| -- the tolerance metric used throughout (<= 1e-3 for fp)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))
