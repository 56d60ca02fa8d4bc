"""Shared test setup: import paths, the `gpu` marker, seeded input helpers.

`-m "not gpu"` tests run on any host (oracle pins, host-side API, C-ABI
symbols); `-m gpu` tests call the HIP library through its C ABI on a gfx950
device and compare with the CPU oracle (oracle/), which is the checker only.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "sme-gemm_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


@pytest.fixture(scope="session")
def smg():
    """The product library; GPU tests fail (not skip) when it cannot run."""
    import smegemm
    if not smegemm.available():
        raise RuntimeError("libsmegemm_gpu.so did not load or no gfx950 device is visible")
    return smegemm


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


def max_rel(got_bits, want_bits, bf16=False):
    """max |g - w| / (1 + |w|) (tests/correctness/main.rs:63-68), both given as
    16-bit patterns (w = the oracle's rounded output)."""
    import oracle
    cv = oracle.bf16_to_f32 if bf16 else oracle.f16_to_f32
    g = cv(got_bits).astype(np.float64)
    w = cv(want_bits).astype(np.float64)
    if np.any(np.isnan(g) != np.isnan(w)):
        return float("inf")
    ok = ~np.isnan(w)
    if not ok.any():
        return 0.0
    return float(np.max(np.abs(g[ok] - w[ok]) / (1.0 + np.abs(w[ok]))))


def f16_tol(k):
    """The north star's float tolerance: max rel err <= 2e-3 * sqrt(K)/64,
    floored at 2e-3 (K <= 4096)."""
    return 2e-3 * max(1.0, np.sqrt(max(k, 1)) / 64.0)


def bf16_tol(k):
    """bf16 keeps 8 mantissa bits to f16's 11: 8x the f16 bound."""
    return 8.0 * f16_tol(k)


def rng_f16(rng, size, scale=1.0):
    return (rng.standard_normal(size) * scale).astype(np.float16).view(np.uint16)


def ulp_dist(a, b):
    """Largest distance in 16-bit ulps between two arrays of f16/bf16 bit
    patterns (sign-magnitude mapped to a monotonic integer line)."""
    def line(x):
        x = np.asarray(x, np.uint16).astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return int(np.max(np.abs(line(a) - line(b)))) if np.size(a) else 0
