"""Seeded synthetic inputs for the benchmark configurations (host numpy arrays,
f16 values as uint16 bit patterns). Shared by bench.py and the parity tests so
both see identical data.

Config 1 (Q4 GEMV): nibbles uniform 0..15 (code = two's complement of the
nibble, src/kernels/q4/mod.rs:213-214), one f16 scale per column per 32-block
~ U[0.005, 0.02], A ~ N(0, 1).
Config 2 (Q2): codes uniform in {0, 1, 2} (ternary -1/0/+1), scales ~ U[0.01, 0.05]
per 128-block.
Config 3 (Q1): signs Bernoulli(0.5), scales ~ U[0.01, 0.05] per 128-block,
bias ~ N(0, 0.1).
Config 4 (Q4 GEMM): as config 1 with m = 512, plus mul_col s ~ U[0.5, 1.5] and
add_col b ~ N(0, 0.1).
"""
from __future__ import annotations

import numpy as np


def f16(x) -> np.ndarray:
    return np.asarray(x, np.float64).astype(np.float16).view(np.uint16)


def q4_inputs(m: int, n: int, k: int, block: int = 32, seed: int = 0, scale_lo=0.005,
              scale_hi=0.02, affine: bool = False):
    rng = np.random.default_rng(seed)
    quants = rng.integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
    nbk = -(-k // block)
    scales = f16(rng.uniform(scale_lo, scale_hi, size=n * nbk))
    mins = f16(rng.uniform(-0.1, 0.1, size=n * nbk)) if affine else None
    a = f16(rng.standard_normal(m * k))
    return a, quants, scales, mins


def q2_inputs(m: int, n: int, k: int, block: int = 128, seed: int = 0):
    rng = np.random.default_rng(seed)
    codes2 = rng.integers(0, 3, size=k * n, dtype=np.uint8)  # ternary codes 0,1,2
    pad = (-codes2.size) % 4
    c = np.concatenate([codes2, np.zeros(pad, np.uint8)]).reshape(-1, 4)
    codes = (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8)
    nbk = -(-k // block)
    scales = f16(rng.uniform(0.01, 0.05, size=n * nbk))
    a = f16(rng.standard_normal(m * k))
    return a, codes, scales


def q1_inputs(m: int, n: int, k: int, block: int = 128, seed: int = 0):
    rng = np.random.default_rng(seed)
    signs = rng.integers(0, 256, size=(k * n + 7) // 8, dtype=np.uint8)
    nbk = -(-k // block)
    scales = f16(rng.uniform(0.01, 0.05, size=n * nbk))
    a = f16(rng.standard_normal(m * k))
    bias = f16(rng.normal(0.0, 0.1, size=n))
    return a, signs, scales, bias


def q4_gemm_epilogue_inputs(n: int, seed: int = 1):
    rng = np.random.default_rng(seed)
    s = f16(rng.uniform(0.5, 1.5, size=n))
    b = f16(rng.normal(0.0, 0.1, size=n))
    return s, b


# Algorithmic bytes per call (packed weights + scales + A + C [+ epilogue
# vectors]), counted once each.
def q4_bytes(m, n, k, block=32, affine=False):
    nbk = -(-k // block)
    return (k * n + 1) // 2 + 2 * n * nbk * (2 if affine else 1) + 2 * m * k + 2 * m * n


def q2_bytes(m, n, k, block=128):
    nbk = -(-k // block)
    return (k * n + 3) // 4 + 2 * n * nbk + 2 * m * k + 2 * m * n


def q1_bytes(m, n, k, block=128, n_col_vectors=1):
    nbk = -(-k // block)
    return (k * n + 7) // 8 + 2 * n * nbk + 2 * m * k + 2 * m * n + 2 * n * n_col_vectors
