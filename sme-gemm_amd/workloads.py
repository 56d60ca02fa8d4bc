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


# Config 5: one Llama-style decoder block at one row (src/block.rs path).
CONFIG5 = dict(d=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336, past=4096, theta=10000.0,
               eps=1e-5)


def block_inputs(d: int, heads: int, kv_heads: int, head_dim: int, ffn: int, past: int,
                 seed: int = 0, cap_extra: int = 8):
    """The decode block's weights and state (config 5 at its default sizes):
    Q4 linears as config 1 (nibbles uniform 0..15, scales ~ U[0.005, 0.02] per
    32-block, row-major public input) -- qkv ((heads + 2 kv_heads) * head_dim
    outputs, [q | k | v]), out, gate, up (ffn outputs each) and down --, RMSNorm
    weights ~ U[0.9, 1.1] (f32), `past` cached positions of f16 keys and values
    ~ N(0, 1) (capacity past + cap_extra), and a residual row x ~ N(0, 1) (f32)."""
    rng = np.random.default_rng(seed)

    def q4(n, k):
        quants = rng.integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
        scales = f16(rng.uniform(0.005, 0.02, size=n * -(-k // 32)))
        return quants, scales, n, k

    nq = (heads + 2 * kv_heads) * head_dim
    ld = kv_heads * head_dim
    cap = past + cap_extra
    out = dict(
        qkv=q4(nq, d), out=q4(d, heads * head_dim), gate=q4(ffn, d), up=q4(ffn, d), down=q4(d, ffn),
        norm1=rng.uniform(0.9, 1.1, d).astype(np.float32),
        norm2=rng.uniform(0.9, 1.1, d).astype(np.float32),
        cache_k=np.zeros((cap, ld), np.uint16), cache_v=np.zeros((cap, ld), np.uint16),
        x=rng.standard_normal(d).astype(np.float32))
    out["cache_k"][:past] = f16(rng.standard_normal((past, ld)))
    out["cache_v"][:past] = f16(rng.standard_normal((past, ld)))
    return out


def block_stage_bytes(d, heads, kv_heads, head_dim, ffn, kv_len, block=32):
    """block_bytes split by the decode step's HBM-reading stages: each Q4
    projection's codes and scales, and the cached keys and values."""
    q4 = lambda n, k: n * k // 2 + n * (-(-k // block)) * 2  # noqa: E731
    return {"qkv": q4((heads + 2 * kv_heads) * head_dim, d), "kv_cache": 2 * 2 * kv_len * kv_heads * head_dim,
            "out": q4(d, heads * head_dim), "gate_up": q4(2 * ffn, d), "down": q4(d, ffn)}


def block_bytes(d, heads, kv_heads, head_dim, ffn, kv_len, block=32):
    """Algorithmic HBM bytes of one decode step: every Q4 weight (0.5 B) and
    its f16 scale (2 B per 32-block), and the f16 keys and values read."""
    weights = d * (heads + 2 * kv_heads) * head_dim + heads * head_dim * d + 2 * ffn * d + ffn * d
    return weights // 2 + weights // block * 2 + 2 * 2 * kv_len * kv_heads * head_dim
