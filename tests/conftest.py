"""pytest configuration: the `gpu` marker and shared helpers.

`-m "not gpu"` runs the oracle checks, host logic and ABI checks (no device);
`-m gpu` runs the parity tests through the C ABI on an MI355X.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")
FIXTURES = os.path.join(GOLDEN, "ds5_synthetic")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libds5hip.so on the device)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def hip():
    import qw3_amd.hip as H
    return H


@pytest.fixture(scope="session")
def ctx(hip):
    c = hip.Ctx.init(0)
    yield c
    c.deinit()


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def f16_ulp_diff(a_bits, b_bits) -> np.ndarray:
    """|a - b| in units of f16 ulp (bit-pattern distance on the monotone f16 line)."""
    def mono(x):
        x = np.asarray(x, np.uint16).astype(np.int32)
        return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + x)
    return np.abs(mono(a_bits) - mono(b_bits))


def attention_f64(q, kc_bits, vc_bits, scale):
    """Causal softmax(q k^T * scale) v in float64 for one head: q [T, d] f32, caches
    [T, d] f16 bits (the token at row t attends rows 0..t)."""
    qd = np.asarray(q, np.float64)
    kd = np.asarray(kc_bits, np.uint16).view(np.float16).astype(np.float64)
    vd = np.asarray(vc_bits, np.uint16).view(np.float16).astype(np.float64)
    s = (qd @ kd.T) * float(np.float32(scale))
    T = s.shape[0]
    s[np.triu_indices(T, 1)] = -np.inf
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p @ vd) / p.sum(axis=1, keepdims=True)
