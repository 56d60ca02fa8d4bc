"""Python harness over the C oracle (``oracle.c`` -> ``liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg, as the checker. Every function restates a
piece of the reference crate's portable path; the C source cites file:line for
each. Arrays of f16/bf16 values travel as ``np.uint16`` bit patterns.

Epilogues are described as ``(nodes, act)``: ``nodes`` a list of
``(op, aux, scalar, operand_or_None, ld)`` tuples in builder order (operand a
``np.uint16`` array of f16/bf16 bits) and ``act`` the trailing activation kind
or ``None`` -- the fields of the reference's ``Epilogue`` (src/epilogue/graph.rs:33).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
_lib = None

P = C.c_void_p
SZ = C.c_size_t


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        _lib = C.CDLL(_LIB)
        L = _lib
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_f64_to_f16.restype = C.c_uint16
        L.or_f64_to_f16.argtypes = [C.c_double]
        L.or_f32_to_bf16.restype = C.c_uint16
        L.or_f32_to_bf16.argtypes = [C.c_float]
        L.or_act_f64.restype = C.c_double
        L.or_act_f64.argtypes = [C.c_uint32, C.c_double, C.c_double]
        L.or_act_f32.restype = C.c_float
        L.or_act_f32.argtypes = [C.c_uint32, C.c_float, C.c_float]
        for name in ("or_f32_to_f16_array", "or_f64_to_f16_array", "or_f16_to_f32_array",
                     "or_f32_to_bf16_array"):
            getattr(L, name).argtypes = [P, P, SZ]
            getattr(L, name).restype = None
        L.or_act_f32_array.argtypes = [C.c_uint32, P, P, SZ, C.c_float]
        L.or_q4_quantize.argtypes = [P, C.c_int, SZ, SZ, SZ, C.c_int, P, P, P]
        L.or_q4_quantize.restype = None
        L.or_q2_quantize.argtypes = [P, C.c_int, SZ, SZ, SZ, P, P, P]
        L.or_q2_quantize.restype = C.c_int
        L.or_q1_quantize.argtypes = [P, C.c_int, SZ, SZ, SZ, P, P]
        L.or_q1_quantize.restype = None
        L.or_q4_dequant_f16.argtypes = [P, P, P, SZ, SZ, SZ, P]
        L.or_q4_dequant_bf16.argtypes = [P, P, P, SZ, SZ, SZ, P]
        L.or_gemm_f16.argtypes = [SZ, SZ, SZ, P, P, P, C.c_uint16, C.c_int, P]
        L.or_gemm_bf16.argtypes = [SZ, SZ, SZ, P, P, P, C.c_uint16, C.c_int, P]
        L.or_gemm_strided.argtypes = [C.c_int, SZ, SZ, SZ, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, C.c_uint16,
                                      C.c_uint16, P]
        L.or_gemm_strided.restype = None
        L.or_apply_ep.argtypes = [P, SZ, SZ, SZ, SZ, P, SZ, C.c_int, C.c_int]
        L.or_quantize_row.argtypes = [P, SZ, SZ, P, P]
        L.or_lowbit_reference.argtypes = [C.c_int, P, P, P, P, C.c_int, SZ, SZ, SZ, SZ, P, P, P]
        L.or_lowbit_reference_cols.argtypes = [C.c_int, P, P, P, P, C.c_int, SZ, SZ, SZ, SZ, P,
                                               SZ, SZ, P, P]
        L.or_lowbit_dequant_f16.argtypes = [C.c_int, P, P, P, C.c_int, SZ, SZ, SZ, P]
        L.or_q4_band_sizes.argtypes = [SZ, SZ, SZ, C.POINTER(SZ), C.POINTER(SZ)]
        L.or_q4_band_sizes.restype = SZ
        L.or_q4_pack_band.argtypes = [P, P, P, SZ, SZ, SZ, P, P, P]
        L.or_lowbit_band_sizes.argtypes = [C.c_int, SZ, SZ, SZ, C.POINTER(SZ), C.POINTER(SZ)]
        L.or_lowbit_pack_band.argtypes = [C.c_int, P, P, C.c_int, SZ, SZ, SZ, P, P]
        L.or_rms_norm_row.argtypes = [P, P, SZ, C.c_float, P]
        L.or_rms_norm_f16.argtypes = [P, P, SZ, SZ, C.c_float, P, P]
        L.or_layer_norm_row.argtypes = [P, P, P, SZ, C.c_float, P]
        L.or_layer_norm_f16.argtypes = [P, P, P, SZ, SZ, C.c_float, P, P]
        L.or_rope_inv_freq.argtypes = [SZ, C.c_double, P]
        L.or_rope_angles.argtypes = [P, SZ, SZ, P, P]
        L.or_rope_apply.argtypes = [P, SZ, P, P, SZ]
        L.or_attention_kv_f16.argtypes = [P, P, P, SZ, SZ, SZ, SZ, C.c_float, P, P, P]
        L.or_glu_f16.argtypes = [P, P, SZ, SZ, C.c_int]
        L.or_matmul_mt.argtypes = [C.c_int, P, P, P, P, SZ, SZ, SZ, SZ, P, C.c_int]
        L.or_matmul_mt.restype = C.c_int
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(P)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---- conversions -----------------------------------------------------------

def f32_to_f16(x) -> np.ndarray:
    x = _c(np.asarray(x, np.float32).ravel(), np.float32)
    y = np.empty(x.size, np.uint16)
    lib().or_f32_to_f16_array(_p(x), _p(y), x.size)
    return y


def f64_to_f16(x) -> np.ndarray:
    x = _c(np.asarray(x, np.float64).ravel(), np.float64)
    y = np.empty(x.size, np.uint16)
    lib().or_f64_to_f16_array(_p(x), _p(y), x.size)
    return y


def f16_to_f32(h) -> np.ndarray:
    h = _c(np.asarray(h, np.uint16).ravel(), np.uint16)
    y = np.empty(h.size, np.float32)
    lib().or_f16_to_f32_array(_p(h), _p(y), h.size)
    return y


def f32_to_bf16(x) -> np.ndarray:
    x = _c(np.asarray(x, np.float32).ravel(), np.float32)
    y = np.empty(x.size, np.uint16)
    lib().or_f32_to_bf16_array(_p(x), _p(y), x.size)
    return y


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def act_f32(kind: int, x, alpha: float = 0.0) -> np.ndarray:
    x = _c(np.asarray(x, np.float32).ravel(), np.float32)
    y = np.empty_like(x)
    lib().or_act_f32_array(kind, _p(x), _p(y), x.size, alpha)
    return y


# ---- load-time quantizers ----------------------------------------------------

def q4_quantize(w, layout, n, k, block, affine=False):
    """Q4Weights::quantize (src/kernels/q4/quantize.rs:29-81): (quants, scales, mins)."""
    w = _c(w, np.float32)
    nbk = -(-k // block)
    quants = np.zeros(-(-(k * n) // 2), np.uint8)
    scales = np.zeros(n * nbk, np.uint16)
    mins = np.zeros(n * nbk, np.uint16) if affine else None
    lib().or_q4_quantize(_p(w), layout, n, k, block, int(affine), _p(quants), _p(scales),
                         _p(mins) if affine else None)
    return quants, scales, mins


def q2_quantize(w, layout, n, k, block, codebook=(-1, 0, 1, 0)):
    """Q2Weights::quantize (src/kernels/lowbit/q2.rs:110-143): (codes, scales)."""
    w = _c(w, np.float32)
    nbk = -(-k // block)
    codes = np.zeros(-(-(k * n) // 4), np.uint8)
    scales = np.zeros(n * nbk, np.uint16)
    cb = np.asarray(codebook, np.int8)
    if lib().or_q2_quantize(_p(w), layout, n, k, block, _p(cb), _p(codes), _p(scales)) != 0:
        raise ValueError("q2 codebook is all zeros")
    return codes, scales


def q1_quantize(w, layout, n, k, block):
    """Q1Weights::quantize (src/kernels/lowbit/q1.rs:116-147): (signs OutIn, scales)."""
    w = _c(w, np.float32)
    nbk = -(-k // block)
    signs = np.zeros(-(-(k * n) // 8), np.uint8)
    scales = np.zeros(n * nbk, np.uint16)
    lib().or_q1_quantize(_p(w), layout, n, k, block, _p(signs), _p(scales))
    return signs, scales


# ---- Q4 --------------------------------------------------------------------

def q4_dequant(quants, scales, mins, n, k, block, bf16=False) -> np.ndarray:
    """Row-major k x n weights as the portable path multiplies them
    (src/kernels/q4/mod.rs:193-224; weights.rs:190-259)."""
    quants = _c(quants, np.uint8)
    scales = _c(scales, np.uint16)
    mins = _c(mins, np.uint16)
    out = np.empty(k * n, np.uint16)
    fn = lib().or_q4_dequant_bf16 if bf16 else lib().or_q4_dequant_f16
    fn(_p(quants), _p(scales), _p(mins), n, k, block, _p(out))
    return out


def gemm16(a, b, m, n, k, beta_bits=None, col_major=False, bf16=False) -> np.ndarray:
    """reference::gemm_f16 / gemm_bf16 (src/reference.rs:308-387) with
    alpha = 0, as the packed fallback calls it (src/exec/macros.rs:188-203)."""
    a = _c(a, np.uint16)
    b = _c(b, np.uint16)
    if beta_bits is None:
        beta_bits = 0x3F80 if bf16 else 0x3C00
    c = np.zeros(m * n, np.uint16)
    acc = np.empty(max(n, 1), np.float32)
    fn = lib().or_gemm_bf16 if bf16 else lib().or_gemm_f16
    fn(m, n, k, _p(c), _p(a), _p(b), beta_bits, int(col_major), _p(acc))
    return c


def gemm_strided(c, c_rs, c_cs, a, a_rs, a_cs, b, b_rs, b_cs, m, n, k, alpha_bits, beta_bits,
                 bf16=False) -> np.ndarray:
    """reference::gemm_f16 / gemm_bf16 (src/reference.rs:308-387) in full:
    C = alpha*C + beta*(A@B) over strided uint16 arrays (C is read only when
    alpha != 0). Returns an updated copy of c."""
    c = np.array(c, np.uint16, copy=True)
    a = _c(a, np.uint16)
    b = _c(b, np.uint16)
    acc = np.empty(max(n, 1), np.float32)
    lib().or_gemm_strided(int(bf16), m, n, k, _p(c), c_rs, c_cs, _p(a), a_rs, a_cs, _p(b), b_rs, b_cs,
                          alpha_bits, beta_bits, _p(acc))
    return c


class _EpNode(C.Structure):
    _fields_ = [("op", C.c_uint32), ("aux", C.c_uint32), ("scalar", C.c_float),
                ("ptr", C.c_void_p), ("ld", C.c_size_t)]


def apply_ep(c, m, n, nodes, act, bf16=False, col_major=False) -> np.ndarray:
    """apply_ep_scalar (src/exec/scalar.rs:125-140) on a copy of c."""
    c = np.array(c, np.uint16, copy=True)
    keep = []
    arr = (_EpNode * max(len(nodes), 1))()
    for t, (op, aux, scalar, operand, ld) in enumerate(nodes):
        ptr = None
        if operand is not None:
            operand = _c(operand, np.uint16)
            keep.append(operand)
            ptr = operand.ctypes.data
        arr[t] = _EpNode(op, aux, scalar, ptr, ld)
    rs, cs = (1, m) if col_major else (n, 1)
    lib().or_apply_ep(_p(c), m, n, rs, cs, C.cast(arr, P), len(nodes),
                      -1 if act is None else int(act), int(bf16))
    return c


def _has_ep(nodes, act):
    return len(nodes) > 0 or act is not None


def packed_ep(a, b, m, n, k, nodes=(), act=None, beta_bits=None, col_major=False, bf16=False):
    """f16/bf16_packed_ep_impl's portable branch (src/exec/macros.rs:188-206):
    reference GEMM, then the scalar epilogue iff the graph is non-empty."""
    c = gemm16(a, b, m, n, k, beta_bits, col_major, bf16)
    if _has_ep(nodes, act):
        c = apply_ep(c, m, n, list(nodes), act, bf16, col_major)
    return c


def matmul_q4_ep(a, quants, scales, mins, m, n, k, block, nodes=(), act=None, bf16=False):
    """matmul_q4_ep / matmul_q4_bf16_ep off-Apple (src/kernels/q4/matmul.rs:91-102,
    :258-270): dequant to row-major, then the dense packed path."""
    if m == 0 or n == 0:
        return np.zeros(m * n, np.uint16)
    b = q4_dequant(quants, scales, mins, n, k, block, bf16)
    return packed_ep(a, b, m, n, k, nodes, act, None, False, bf16)


# ---- low-bit -----------------------------------------------------------------

def quantize_row(a, k, block):
    """quantize_row (src/kernels/lowbit/matmul.rs:354-371)."""
    a = _c(a, np.uint16)
    nbk = -(-k // block)
    q = np.empty(max(k, 1), np.int8)
    s = np.empty(max(nbk, 1), np.float32)
    lib().or_quantize_row(_p(a), k, block, _p(q), _p(s))
    return q[:k], s[:nbk]


def lowbit_reference(kind, a, codes, scales, m, n, k, block, codebook=(-1, 0, 1, 0),
                     inout=False, cols=None):
    """reference (src/kernels/lowbit/matmul.rs:376-398) on the public input
    formats: kind 2 = Q2 (q2.rs:43-47), kind 1 = Q1 (q1.rs:35-41)."""
    a = _c(a, np.uint16)
    codes = _c(codes, np.uint8)
    scales = _c(scales, np.uint16)
    cb = np.asarray(codebook, np.int8)
    c = np.zeros(m * n, np.uint16)
    q = np.empty(max(k, 1), np.int8)
    s = np.empty(max(-(-k // block), 1), np.float32)
    if cols is None:
        lib().or_lowbit_reference(kind, _p(a), _p(codes), _p(scales), _p(cb), int(inout), m, n,
                                  k, block, _p(c), _p(q), _p(s))
    else:
        lib().or_lowbit_reference_cols(kind, _p(a), _p(codes), _p(scales), _p(cb), int(inout),
                                       m, n, k, block, _p(c), cols[0], cols[1], _p(q), _p(s))
    return c


def matmul_lowbit_ep(kind, a, codes, scales, m, n, k, block, nodes=(), act=None,
                     codebook=(-1, 0, 1, 0), inout=False):
    """lowbit_impl off-Apple (matmul.rs:326-337): reference, then apply_ep_scalar
    (always called; the empty graph is the identity)."""
    if m == 0 or n == 0:
        return np.zeros(m * n, np.uint16)
    c = lowbit_reference(kind, a, codes, scales, m, n, k, block, codebook, inout)
    return apply_ep(c, m, n, list(nodes), act)


def lowbit_dequant(kind, codes, scales, n, k, block, codebook=(-1, 0, 1, 0), inout=False):
    """Codes::dequant (matmul.rs:178-197)."""
    codes = _c(codes, np.uint8)
    scales = _c(scales, np.uint16)
    cb = np.asarray(codebook, np.int8)
    out = np.empty(k * n, np.uint16)
    lib().or_lowbit_dequant_f16(kind, _p(codes), _p(scales), _p(cb), int(inout), n, k, block,
                                _p(out))
    return out


def matmul_lowbit_mopa_ep(kind, a, codes, scales, m, n, k, block, nodes=(), act=None,
                          codebook=(-1, 0, 1, 0), inout=False):
    """mopa_impl off-Apple (matmul.rs:339-350): eager dequant, dense f16 path."""
    if m == 0 or n == 0:
        return np.zeros(m * n, np.uint16)
    b = lowbit_dequant(kind, codes, scales, n, k, block, codebook, inout)
    return packed_ep(a, b, m, n, k, nodes, act)


# ---- the reference's band-major resident packs ------------------------------

def q4_band_sizes(n, k, block):
    """(nibble bytes, scale entries) of the band-major Q4 arrays."""
    nl, sl = SZ(), SZ()
    lib().or_q4_band_sizes(n, k, block, C.byref(nl), C.byref(sl))
    return nl.value, sl.value


def lowbit_band_sizes(kind, n, k, block):
    """(code bytes, scale entries) of the band-major Q2 (kind 2) / Q1 arrays."""
    cl, sl = SZ(), SZ()
    lib().or_lowbit_band_sizes(kind, n, k, block, C.byref(cl), C.byref(sl))
    return cl.value, sl.value


def q4_pack_band(quants, scales, mins, n, k, block):
    nl, sl = SZ(), SZ()
    lib().or_q4_band_sizes(n, k, block, C.byref(nl), C.byref(sl))
    nib = np.empty(nl.value, np.uint8)
    sc = np.empty(sl.value, np.uint16)
    mn = np.empty(sl.value, np.uint16) if mins is not None else None
    lib().or_q4_pack_band(_p(_c(quants, np.uint8)), _p(_c(scales, np.uint16)),
                          _p(_c(mins, np.uint16)), n, k, block, _p(nib), _p(sc), _p(mn))
    return nib, sc, mn


def lowbit_pack_band(kind, codes, scales, n, k, block, inout=False):
    cl, sl = SZ(), SZ()
    lib().or_lowbit_band_sizes(kind, n, k, block, C.byref(cl), C.byref(sl))
    packed = np.empty(cl.value, np.uint8)
    sc = np.empty(sl.value, np.uint16)
    lib().or_lowbit_pack_band(kind, _p(_c(codes, np.uint8)), _p(_c(scales, np.uint16)),
                              int(inout), n, k, block, _p(packed), _p(sc))
    return packed, sc


# ---- the reference's test-data generators -----------------------------------

def lcg_bytes(seed: int, length: int) -> np.ndarray:
    """`data`/`bytes`/`byte` of the reference tests
    (src/kernels/lowbit/matmul.rs:409-417, tests/correctness/q4.rs:18-21):
    s = s*6364136223846793005 + 1 (mod 2^64), byte = (s >> 40) as u8."""
    out = np.empty(length, np.uint8)
    s = seed & 0xFFFFFFFFFFFFFFFF
    for i in range(length):
        s = (s * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
        out[i] = (s >> 40) & 0xFF
    return out


def lcg_fill(seed: int, length: int):
    """`fill` of tests/correctness/main.rs:36-46: returns (f16 bits, new seed)."""
    vals = np.empty(length, np.float32)
    s = seed & 0xFFFFFFFFFFFFFFFF
    for i in range(length):
        s = (s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        vals[i] = np.float32(s >> 40) / np.float32(1 << 24) - np.float32(0.5)
    return f32_to_f16(vals), s


def lcg_fill_f32(seed: int, length: int):
    """`fill_f32` of tests/correctness/main.rs:152-161: returns (f32 values,
    new seed)."""
    vals = np.empty(length, np.float32)
    s = seed & 0xFFFFFFFFFFFFFFFF
    for i in range(length):
        s = (s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        vals[i] = np.float32(s >> 40) / np.float32(1 << 24) - np.float32(0.5)
    return vals, s


# ---- the decode block's row-wise passes (config 5) ---------------------------

def rms_norm_row(x, w, eps):
    """norm_row with rms (src/nn.rs:127-144), f32 out."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    out = np.empty(x.size, np.float32)
    lib().or_rms_norm_row(_p(x), _p(w), x.size, eps, _p(out))
    return out


def rms_norm_f16(x, w, eps, rows=1):
    """nn::rms_norm into f16 (src/nn.rs:159): rows of len(w)."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    y = np.empty(x.size, np.uint16)
    scratch = np.empty(w.size, np.float32)
    lib().or_rms_norm_f16(_p(x), _p(w), rows, w.size, eps, _p(y), _p(scratch))
    return y


def layer_norm_row(x, w, b, eps):
    """norm_row with rms = false (src/nn.rs:133-143), f32 out; b may be None."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    bb = None if b is None else _c(b, np.float32)
    out = np.empty(x.size, np.float32)
    lib().or_layer_norm_row(_p(x), _p(w), None if bb is None else _p(bb), x.size, eps, _p(out))
    return out


def layer_norm_f16(x, w, b, eps, rows=1):
    """nn::layer_norm into f16 (src/nn.rs:73-86): rows of len(w); b may be None."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    bb = None if b is None else _c(b, np.float32)
    y = np.empty(x.size, np.uint16)
    scratch = np.empty(w.size, np.float32)
    lib().or_layer_norm_f16(_p(x), _p(w), None if bb is None else _p(bb), rows, w.size, eps, _p(y),
                            _p(scratch))
    return y


def norm_f16(x, p, which):
    """The block's norm `which` (1 or 2): Norm::layer when p["norm"] is "layer"
    (weights p["norm<which>"], optional bias p["bias<which>"]), else Norm::rms."""
    if p.get("norm") == "layer":
        return layer_norm_f16(x, p[f"norm{which}"], p.get(f"bias{which}"), p["eps"])
    return rms_norm_f16(x, p[f"norm{which}"], p["eps"])


def rope_inv_freq(dim, base=10000.0):
    """Rope::new without YaRN (examples/bonsai/model.rs:38-51)."""
    out = np.empty(dim // 2, np.float32)
    lib().or_rope_inv_freq(dim, base, _p(out))
    return out


def rope_angles(inv_freq, pos):
    """Rope::angles (model.rs:77-85): (cos, sin) per frequency."""
    inv_freq = _c(inv_freq, np.float32)
    c = np.empty(inv_freq.size, np.float32)
    s = np.empty(inv_freq.size, np.float32)
    lib().or_rope_angles(_p(inv_freq), inv_freq.size, pos, _p(c), _p(s))
    return c, s


def rope_apply(x, cos_v, sin_v):
    """Rope::apply (model.rs:87-99) on a copy of x (heads of 2*len(cos_v))."""
    x = np.array(x, np.float32, copy=True)
    cos_v = _c(cos_v, np.float32)
    sin_v = _c(sin_v, np.float32)
    lib().or_rope_apply(_p(x), x.size, _p(cos_v), _p(sin_v), cos_v.size)
    return x


def attention_kv_f16(q, k, v, length, heads, kv_heads, hd, scale):
    """attention_kv_f16's portable one_row (src/kernels/kv_attention.rs:282-325):
    q f32 [heads*hd], k/v f16 bits [length][kv_heads*hd]; returns f32."""
    q = _c(q, np.float32)
    k = _c(k, np.uint16)
    v = _c(v, np.uint16)
    out = np.empty(heads * hd, np.float32)
    scores = np.empty(max(length, 1), np.float32)
    qh = np.empty(hd, np.float32)
    lib().or_attention_kv_f16(_p(q), _p(k), _p(v), length, heads, kv_heads, hd, scale, _p(out),
                              _p(scores), _p(qh))
    return out


def glu_f16(both, m, n, gelu=False):
    """glu (src/linear.rs:804-826) over m rows of 2n interleaved gate/up f16."""
    both = _c(both, np.uint16)
    y = np.empty(m * n, np.uint16)
    lib().or_glu_f16(_p(y), _p(both), m, n, int(gelu))
    return y


def interleave32(g, u, n, k):
    """GatedLinear's interleave (src/linear.rs:601-619) of two InOut k x n
    arrays (any dtype): k x 2n, each 32-column chunk of g then of u."""
    g = np.asarray(g).reshape(k, n)
    u = np.asarray(u).reshape(k, n)
    parts = []
    for c0 in range(0, n, 32):
        c1 = min(c0 + 32, n)
        parts += [g[:, c0:c1], u[:, c0:c1]]
    return np.concatenate(parts, axis=1)


class Q4Lin:
    """A 4-bit Linear as the reference's portable path runs it at one row
    (Linear::forward -> matmul_q4_ep, src/linear.rs:533-552): the public
    row-major arrays of Q4Weights (block 32, Scale form)."""

    def __init__(self, quants, scales, n, k, block=32):
        self.quants, self.scales, self.n, self.k, self.block = quants, scales, n, k, block

    def forward(self, x16, m=1, nodes=(), act=None):
        return matmul_q4_ep(x16, self.quants, self.scales, None, m, self.n, self.k, self.block,
                            nodes, act)


def block_decode(x, cache_k, cache_v, pos, p, parts=None):
    """One row of Block::accumulate (src/block.rs:90-106) with RoPE inserted as
    examples/bonsai/model.rs:329-349 applies it (q and k rotated in f32 after
    the qkv projection, k stored rotated; no q/k norm):
      h = rms_norm(x, norm1) -> f16;  qkv = Q4 qkv(h) -> f16
      q, k = rope(f32(q16), pos), rope(f32(k16), pos); cache[pos] = f16(k), v16
      att = attention_kv_f16(q, K[0..=pos], V[0..=pos]) -> f16;  x += f32(out(att))
      h = rms_norm(x, norm2) -> f16;  hid = glu(gate_up(h)) -> f16;  x += f32(down(hid))
    x: f32 [d] (updated copy returned); cache_k / cache_v: f16 [cap][kv*hd]
    (row pos written). p: dict of the block's parts (see tests). parts: a
    dict that receives the two f16 terms added to the residual, as f32
    ("attn", "mlp"), and the residual between them ("x1")."""
    d, H, KV, hd, eps = p["d"], p["heads"], p["kv_heads"], p["head_dim"], p["eps"]
    x = np.array(x, np.float32, copy=True)
    h = norm_f16(x, p, 1)
    qkv = p["qkv"].forward(h)
    ql, kl = H * hd, KV * hd
    q32 = f16_to_f32(qkv[:ql])
    k32 = f16_to_f32(qkv[ql:ql + kl])
    if p.get("theta"):
        cs, sn = rope_angles(rope_inv_freq(hd, p["theta"]), pos)
        q32 = rope_apply(q32, cs, sn)
        k32 = rope_apply(k32, cs, sn)
    cache_k[pos] = f32_to_f16(k32)
    cache_v[pos] = qkv[ql + kl:]
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    att = attention_kv_f16(q32, cache_k[:pos + 1], cache_v[:pos + 1], pos + 1, H, KV, hd, scale)
    o = p["out"].forward(f32_to_f16(att))
    if parts is not None:
        parts["attn"] = f16_to_f32(o)
    x = (x + f16_to_f32(o)).astype(np.float32)
    o = block_mlp_term(x, p)
    if parts is not None:
        parts["x1"] = x.copy()
        parts["mlp"] = o
    return (x + o).astype(np.float32)


def block_mlp_term(x, p):
    """The MLP half's term of Block::accumulate (src/block.rs:90-106) for the
    f32 residual row x: f32(down(glu(gate_up(norm2(x) -> f16)))) (Mlp::gated),
    or with p["up"], f32(down(act(up(h)))) (Mlp::new, the activation at the up
    projection's f16 store: src/mlp.rs:113-149, act p["act"])."""
    h = norm_f16(np.asarray(x, np.float32), p, 2)
    if "up" in p:
        hid = p["up"].forward(h, 1, (), p["act"])
    else:
        both = p["gate_up"].forward(h)
        hid = glu_f16(both, 1, p["ffn"], p.get("gelu", False))
    return f16_to_f32(p["down"].forward(hid))


def block_rows(x, cache_k, cache_v, pos, rows, p):
    """Block::accumulate for `rows` rows at positions pos .. pos + rows - 1
    (src/block.rs:90-106): every output row depends on its own input row and
    on the cache -- the qkv, out and MLP products and the norms act row by
    row, and attend_causal gives row r the portable one_row over positions
    0 .. pos + r (kv_attention.rs:214-238) -- so the block of rows is
    block_decode applied to the rows in order. x: f32 [rows][d] (updated copy
    returned); cache rows pos .. pos + rows - 1 written."""
    d = p["d"]
    x = np.array(x, np.float32, copy=True).reshape(rows, d)
    for r in range(rows):
        x[r] = block_decode(x[r], cache_k, cache_v, pos + r, p)
    return x.ravel()


def attention_kv_causal_f16(q, k, v, start, rows, heads, kv_heads, hd, scale):
    """attention_kv_causal_f16's portable path (src/kernels/kv_attention.rs:214-238):
    query row i is one_row over keys 0 .. start + i. q f32 [rows][heads*hd],
    k/v f16 bits [start + rows][kv_heads*hd]; returns f32 [rows][heads*hd]."""
    q = _c(q, np.float32).reshape(rows, heads * hd)
    ld = kv_heads * hd
    k = _c(k, np.uint16).reshape(-1, ld)
    v = _c(v, np.uint16).reshape(-1, ld)
    out = np.empty((rows, heads * hd), np.float32)
    for i in range(rows):
        out[i] = attention_kv_f16(q[i], k[:start + i + 1], v[:start + i + 1], start + i + 1, heads, kv_heads,
                                  hd, scale)
    return out.ravel()


def q4_interleave32(gq, gs, uq, us, n, k, block=32):
    """The Q4 row-major arrays (quants, scales) of gate | up interleaved 32
    columns at a time, as GatedLinear::quantize lays out its 2n outputs
    (src/linear.rs:601-619): every column keeps its codes and scales (Q4 blocks
    run along K), so this is the quantization of the interleaved weights."""
    nbk = -(-k // block)
    if n % 32 == 0:
        # 32 columns of a depth are 16 whole bytes: move bytes, not nibbles
        g = np.asarray(gq, np.uint8).reshape(k, n // 32, 1, 16)
        u = np.asarray(uq, np.uint8).reshape(k, n // 32, 1, 16)
        quants = np.ascontiguousarray(np.concatenate([g, u], axis=2)).ravel()
    else:
        idx = np.arange(k * n)

        def nibs(q):
            return np.where(idx % 2 == 0, q[idx // 2] & 15, q[idx // 2] >> 4).astype(np.uint8).reshape(k, n)
        both = interleave32(nibs(gq), nibs(uq), n, k).ravel()
        lo, hi = both[0::2], np.append(both[1::2], np.uint8(0))[:both[0::2].size]
        quants = (lo | (hi << 4)).astype(np.uint8)
    sc = interleave32(np.asarray(gs).reshape(n, nbk).T, np.asarray(us).reshape(n, nbk).T, n, nbk).T.ravel()
    return quants, np.ascontiguousarray(sc)


def matmul_mt(kind, a, codes, scales, m, n, k, block, threads, codebook=(-1, 0, 1, 0)):
    """The CPU baseline's threaded mode: matmul_q4 (kind 4) or matmul_q2 / q1
    (kind 2 / 1, Q1 OutIn), no epilogue, split over column ranges on `threads`
    host threads; the bits of the single-threaded path."""
    a = _c(a, np.uint16)
    codes = _c(codes, np.uint8)
    scales = _c(scales, np.uint16)
    cb = np.asarray(codebook, np.int8)
    c = np.empty(m * n, np.uint16)
    if lib().or_matmul_mt(kind, _p(a), _p(codes), _p(scales), _p(cb), m, n, k, block, _p(c), threads) != 0:
        raise MemoryError("or_matmul_mt: a thread's buffers could not be allocated")
    return c
