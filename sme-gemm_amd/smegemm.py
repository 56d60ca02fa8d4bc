"""Python mirror of the reference crate's quantized-matmul API over the gfx950
C ABI (``include/smegemm_gpu.h`` -> ``libsmegemm_gpu.so``).

Names, argument meaning and panics follow the Rust API this path replaces:
``Q4Params``/``Q4Weights``/``matmul_q4*`` (src/kernels/q4/), ``Q2Params``/
``Q2Weights``/``Q1Weights``/``matmul_q{1,2}{,_ep,_mopa,_mopa_ep}``
(src/kernels/lowbit/), ``Epilogue`` (src/epilogue/graph.rs), ``prepack_f16``/
``Packed`` and the ``Gemm`` builder (src/exec/builder.rs). Length checks raise
``ValueError`` where the Rust code panics.

Arrays are f16/bf16 bit patterns (``np.uint16``) in host memory, or torch CUDA
tensors (int16/float16/bfloat16) for the asynchronous device-pointer entry
points, which run on torch's current stream. There is no CPU fallback: when the
library or a gfx950 device is missing every call raises ``SmeGemmError``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBPATH = os.path.join(_HERE, "libsmegemm_gpu.so")
_lib = None

P = C.c_void_p
SZ = C.c_size_t

Q4_BLOCK = 32          # src/kernels/q4/mod.rs:34
Q2_BLOCK = 256         # src/kernels/lowbit/mod.rs:26
Q2_TERNARY = (-1, 0, 1, 0)  # src/kernels/lowbit/mod.rs:30


class SmeGemmError(RuntimeError):
    pass


def build() -> None:
    """Compile the HIP library for gfx950 in-tree."""
    subprocess.run(["make", "-s", "-C", _HERE, "-j8"], check=True)


def lib() -> C.CDLL:
    """The loaded C ABI. Raises if the library has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIBPATH):
        raise SmeGemmError(f"{_LIBPATH} is not built (run make -C {_HERE})")
    # PyTorch-ROCm ships its own libamdhip64; loading torch first makes this
    # library resolve to that same runtime, so one HIP runtime serves the
    # process and torch streams / device pointers are valid here. (With two
    # runtimes loaded, the second one to initialise sees no GPU.)
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(_LIBPATH)
    W = C.POINTER(C.c_void_p)
    L.smg_available.restype = C.c_int
    L.smg_last_error.restype = C.c_char_p
    L.smg_q4_gemv_max_rows.restype = SZ
    L.smg_q4_create.argtypes = [P, P, P, SZ, SZ, SZ, W]
    L.smg_q4_create_band.argtypes = [P, P, P, SZ, SZ, SZ, W]
    L.smg_q2_create.argtypes = [P, P, P, SZ, SZ, SZ, W]
    L.smg_q2_create_band.argtypes = [P, P, P, SZ, SZ, SZ, W]
    L.smg_q1_create.argtypes = [P, P, C.c_int, SZ, SZ, SZ, W]
    L.smg_q1_create_band.argtypes = [P, P, SZ, SZ, SZ, W]
    L.smg_q4_quantize.argtypes = [P, C.c_int, SZ, SZ, SZ, C.c_int, P, P, P]
    L.smg_q2_quantize.argtypes = [P, C.c_int, SZ, SZ, SZ, P, P, P]
    L.smg_q1_quantize.argtypes = [P, C.c_int, SZ, SZ, SZ, P, P]
    L.smg_f16_prepack.argtypes = [P, SZ, SZ, C.c_long, C.c_long, W]
    L.smg_bf16_prepack.argtypes = [P, SZ, SZ, C.c_long, C.c_long, W]
    L.smg_q4_dequant.argtypes = [P, C.c_int, W]
    L.smg_weights_clone.argtypes = [P, W]
    L.smg_q4_permute_columns.argtypes = [P, P, W]
    L.smg_q1_interleave.argtypes = [P, P, W]
    L.smg_weights_destroy.argtypes = [P]
    L.smg_weights_destroy.restype = None
    L.smg_weights_info.argtypes = [P, C.POINTER(SZ), C.POINTER(SZ), C.POINTER(SZ), C.POINTER(SZ)]
    L.smg_weights_device.argtypes = [P, C.POINTER(C.c_int)]
    for name in ("gemm_gpu_f16f16_q4", "gemm_gpu_b16b16_q4", "gemm_gpu_f16_q2", "gemm_gpu_f16_q1",
                 "gemm_gpu_f16f16_q2", "gemm_gpu_f16f16_q1"):
        getattr(L, name).argtypes = [SZ, P, P, P, P]
    for name in ("gemm_gpu_f16f16_run_packed", "gemm_gpu_b16b16_run_packed"):
        getattr(L, name).argtypes = [SZ, SZ, SZ, P, C.c_long, C.c_long, C.c_int, P, C.c_long,
                                     C.c_long, P, C.c_uint16, C.c_uint16, P]
    L.gemm_gpu_f16f16_q4_single.argtypes = [SZ, SZ, SZ]
    L.smg_q4_matmul_dev.argtypes = [SZ, P, P, P, P, C.c_int, P]
    L.gemm_gpu_f16f16_q4_chained.argtypes = [SZ, P, P, P, P, P, P]
    L.smg_q4_chained_dev.argtypes = [SZ, P, P, P, P, P, P, P, C.c_uint, P]
    L.smg_lowbit_matmul_dev.argtypes = [SZ, P, P, P, P, P]
    L.smg_lowbit_mopa_dev.argtypes = [SZ, P, P, P, P, P]
    L.smg_packed_matmul_dev.argtypes = [SZ, P, P, C.c_long, C.c_long, P, C.c_long, C.c_long,
                                        C.c_uint16, P, C.c_int, P]
    for name in ("gemm_gpu_f16f16_run", "gemm_gpu_f16f32_run", "gemm_gpu_b16b16_run", "gemm_gpu_bf16f32_run"):
        getattr(L, name).argtypes = [SZ, SZ, SZ, P, C.c_long, C.c_long, C.c_int, P, C.c_long, C.c_long,
                                     P, C.c_long, C.c_long, C.c_uint16, C.c_uint16]
    L.smg_gemm_run_dev.argtypes = [C.c_int, SZ, SZ, SZ, P, C.c_long, C.c_long, C.c_int, P, C.c_long,
                                   C.c_long, P, C.c_long, C.c_long, C.c_uint16, C.c_uint16, P]
    L.smg_ep_check.argtypes = [P, SZ]
    L.smg_q4_interleave.argtypes = [P, P, W]
    # the decode block
    L.smg_kv_cache_create.argtypes = [SZ, SZ, SZ, SZ, W]
    L.smg_kv_cache_destroy.argtypes = [P]
    L.smg_kv_cache_destroy.restype = None
    L.smg_kv_cache_info.argtypes = [P, C.POINTER(SZ), C.POINTER(SZ), C.POINTER(C.c_float)]
    L.smg_kv_cache_truncate.argtypes = [P, SZ]
    L.smg_kv_cache_set_scale.argtypes = [P, C.c_float]
    L.smg_kv_cache_storage.argtypes = [P, W, W]
    L.smg_kv_cache_read_dev.argtypes = [P, P, P, P]
    L.smg_kv_cache_extend_dev.argtypes = [P, P, P, SZ, P]
    L.smg_kv_cache_attend_dev.argtypes = [P, P, P, P]
    L.smg_attention_kv_f16_dev.argtypes = [P, P, P, SZ, SZ, SZ, SZ, C.c_float, P, P]
    L.smg_rms_norm_f16_dev.argtypes = [P, P, SZ, SZ, C.c_float, P, P]
    L.smg_layer_norm_f16_dev.argtypes = [P, P, P, SZ, SZ, C.c_float, P, P]
    L.smg_attention_kv_causal_f16_dev.argtypes = [P, P, P, SZ, SZ, SZ, SZ, SZ, C.c_float, P, P]
    L.smg_kv_cache_attend_causal_dev.argtypes = [P, P, SZ, P, P]
    L.smg_glu_f16_dev.argtypes = [P, SZ, SZ, C.c_uint32, P, P]
    L.smg_q4_accumulate_dev.argtypes = [SZ, P, P, P, P]
    L.smg_attn_create.argtypes = [P, P, SZ, SZ, SZ, C.c_double, W]
    L.smg_attn_destroy.argtypes = [P]
    L.smg_attn_destroy.restype = None
    L.smg_attn_accumulate_dev.argtypes = [P, P, P, P, SZ, P]
    L.smg_mlp_create.argtypes = [P, P, C.c_uint32, C.c_int, W]
    L.smg_mlp_destroy.argtypes = [P]
    L.smg_mlp_destroy.restype = None
    L.smg_mlp_accumulate_dev.argtypes = [P, P, P, SZ, P]
    L.smg_block_create.argtypes = [P, C.c_float, P, C.c_float, SZ, P, P, W]
    L.smg_block_create_norms.argtypes = [P, P, C.c_float, C.c_int, P, P, C.c_float, C.c_int, SZ, P, P, W]
    L.smg_block_destroy.argtypes = [P]
    L.smg_block_destroy.restype = None
    L.smg_block_accumulate_dev.argtypes = [P, P, P, SZ, P]
    # host-slice forms of the model parts
    L.smg_q4_accumulate.argtypes = [SZ, P, P, P]
    L.smg_attn_accumulate.argtypes = [P, P, P, P, SZ]
    L.smg_mlp_accumulate.argtypes = [P, P, P, SZ]
    L.smg_block_accumulate.argtypes = [P, P, P, SZ]
    L.smg_kv_cache_extend.argtypes = [P, P, P, SZ]
    L.smg_kv_cache_read.argtypes = [P, P, P]
    L.smg_kv_cache_attend.argtypes = [P, P, P]
    L.smg_kv_cache_attend_causal.argtypes = [P, P, SZ, P]
    L.smg_attention_kv_f16.argtypes = [P, P, P, SZ, SZ, SZ, SZ, C.c_float, P]
    L.smg_attention_kv_causal_f16.argtypes = [P, P, P, SZ, SZ, SZ, SZ, SZ, C.c_float, P]
    L.smg_rms_norm_f16.argtypes = [P, P, SZ, SZ, C.c_float, P]
    L.smg_layer_norm_f16.argtypes = [P, P, P, SZ, SZ, C.c_float, P]
    L.smg_stream_read_dev.argtypes = [P, SZ, P]
    L.smg_stream_read_store_dev.argtypes = [P, SZ, P, SZ, P]
    L.smg_clock_probe_dev.argtypes = [P, C.c_uint, P]
    _lib = L
    return L


def available() -> bool:
    try:
        return bool(lib().smg_available())
    except (OSError, SmeGemmError):
        return False


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise SmeGemmError(f"{what} failed (rc={rc}): {lib().smg_last_error().decode()}")


def _require_device() -> None:
    if not lib().smg_available():
        raise SmeGemmError("no gfx950 device: the HIP path is required (there is no CPU fallback)")


# ---- array plumbing ---------------------------------------------------------

def _is_dev(x) -> bool:
    return hasattr(x, "is_cuda") and x.is_cuda


def _host16(x, n: int, what: str) -> np.ndarray:
    a = np.ascontiguousarray(x)
    if a.dtype != np.uint16:
        if a.dtype == np.float16:
            a = a.view(np.uint16)
        else:
            raise TypeError(f"{what}: expected uint16 bit patterns or float16")
    if a.size != n:
        raise ValueError(f"{what} has {a.size} elements, expected {n}")
    return a


def _ptr(a) -> int:
    if _is_dev(a):
        return a.data_ptr()
    return a.ctypes.data


def _dev16(x, n: int | None, what: str, device: int | None, bf16: bool | None = None):
    """A device tensor the kernels read or write as `n` contiguous 16-bit
    elements on `device`: anything else (a 1- or 4-byte dtype, a strided view,
    another GPU) would make them read or store the wrong bytes."""
    if x.element_size() != 2:
        raise TypeError(f"{what}: expected a 16-bit tensor (float16/bfloat16/int16), got {x.dtype}")
    if bf16 is not None:
        import torch
        if (bf16 and x.dtype == torch.float16) or (not bf16 and x.dtype == torch.bfloat16):
            raise TypeError(f"{what}: {x.dtype} where {'bf16' if bf16 else 'f16'} values are expected")
    if not x.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if device is not None and x.device.index != device:
        raise ValueError(f"{what} is on cuda:{x.device.index}, the weights on cuda:{device}")
    if n is not None and x.numel() != n:
        raise ValueError(f"{what} has {x.numel()} elements, expected {n}")
    return x


def _host_x16(x, n: int, what: str) -> np.ndarray:
    """A host input of a model part as f16 bits: float16 / uint16 as they are,
    float32 rounded to nearest even as the reference's ModelFloat::as_f16
    does for f32 callers (src/linear.rs:61-66)."""
    a = np.asarray(x)
    if a.dtype == np.float32:
        with np.errstate(over="ignore"):  # past the f16 range: infinity, as the conversion rounds
            a = np.ascontiguousarray(a).astype(np.float16)
    return _host16(a, n, what)


def _host_out(x, n: int | None, dtypes, what: str) -> np.ndarray:
    """A host array a host-slice call writes in place: a contiguous, writable
    numpy array of one of `dtypes` with n elements."""
    if not isinstance(x, np.ndarray) or x.dtype not in dtypes:
        raise TypeError(f"{what}: expected a numpy array of {' or '.join(np.dtype(d).name for d in dtypes)}")
    if not x.flags["C_CONTIGUOUS"] or not x.flags["WRITEABLE"]:
        raise ValueError(f"{what} must be contiguous and writable")
    if n is not None and x.size != n:
        raise ValueError(f"{what} has {x.size} elements, expected {n}")
    return x


def _host_f32(x, n: int | None, what: str) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    if n is not None and a.size != n:
        raise ValueError(f"{what} has {a.size} elements, expected {n}")
    return a


def _same_side(*xs):
    """True for device tensors, False for host arrays; mixing them raises."""
    dev = {_is_dev(x) for x in xs if x is not None}
    if len(dev) > 1:
        raise ValueError("the arrays must all be host arrays or all device tensors")
    return dev == {True}


def _stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream


# ---- epilogue ---------------------------------------------------------------

EP_ACT = dict(relu=1, gelu=2, silu=3, tanh=4, sigmoid=5, leaky_relu=6, relu6=7, hardsigmoid=8,
              hardswish=9, abs=10, neg=11, square=12, sign=13, sqrt=14, softsign=15, recip=16,
              rsqrt=17, exp=18, log=19, elu=20, selu=21, softplus=22, mish=23, gelu_exact=24)
EP_OP = dict(add_scalar=0, mul_scalar=1, add_row=2, mul_row=3, add_col=4, mul_col=5,
             add_tensor=6, mul_tensor=7, act=8, max_scalar=9, min_scalar=10, sub_scalar=11,
             sub_row=12, sub_col=13, sub_tensor=14, div_scalar=15, div_row=16, div_col=17,
             div_tensor=18, max_row=19, max_col=20, max_tensor=21, min_row=22, min_col=23,
             min_tensor=24)
_ROW = {2, 3, 12, 16, 19, 22}
_COL = {4, 5, 13, 17, 20, 23}
_TENSOR = {6, 7, 14, 18, 21, 24}


class EpNode(C.Structure):
    """csrc/epilogue.h:214-221 (32 bytes)."""
    _fields_ = [("op", C.c_uint32), ("aux", C.c_uint32), ("scalar", C.c_float),
                ("ptr", C.c_void_p), ("ld", C.c_size_t)]


class EpDesc16(C.Structure):
    _fields_ = [("n_nodes", C.c_uint32), ("nodes", C.POINTER(EpNode))]


def _host_operand(v, bf16: bool) -> np.ndarray:
    """A host epilogue operand as contiguous 16-bit patterns: uint16 bits, or
    float16 values for an f16 graph. Any other dtype is refused rather than
    cast by value (a float32 bias cast to uint16 would be the wrong bits)."""
    a = np.ascontiguousarray(v)
    if a.dtype == np.uint16:
        return a
    if a.dtype == np.float16 and not bf16:
        return a.view(np.uint16)
    raise TypeError(f"epilogue operand: expected {'uint16 bf16 bits' if bf16 else 'float16 or uint16 bits'}, "
                    f"got {a.dtype}")


def _bf16_round(x: float) -> float:
    """f32 -> bf16 RNE -> f32 (NaN kept)."""
    u = int(np.float32(x).view(np.uint32))
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return float(np.float32(x))
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return float(np.uint32(u).view(np.float32))


def _scalar_to_f32(v, bf16: bool) -> float:
    """A scalar operand is stored as `v.ep_to_f32()` of a T (graph.rs:86-96):
    pass a number (int or float, rounded to T here) or T's bit pattern given
    explicitly as np.uint16."""
    if isinstance(v, np.uint16):
        if bf16:
            return float(np.uint32(int(v) << 16).view(np.float32))
        return float(v.view(np.float16))
    if isinstance(v, bool) or not isinstance(v, (int, float, np.floating, np.integer)):
        raise TypeError(f"scalar operand: a number or np.uint16 bits, got {type(v).__name__}")
    return _bf16_round(float(v)) if bf16 else float(np.float16(float(v)))


class Epilogue:
    """The ordered op-graph builder (src/epilogue/graph.rs:33). Operands are
    uint16 f16/bf16 bit arrays (host) or CUDA tensors (device calls).
    Named activations (.relu/.gelu/.silu/.tanh/.sigmoid) set the trailing
    activation, applied last; the others push in-order nodes."""

    def __init__(self, bf16: bool = False):
        self.bf16 = bf16  # element type T of the operands: f16 (default) or bf16
        self.nodes = []   # (op, aux, scalar, operand, ld)
        self.act = None

    def _scalar(self, op, v):
        self.nodes.append((op, 0, _scalar_to_f32(v, self.bf16), None, 0))
        return self

    def _vec(self, op, v, ld=0):
        self.nodes.append((op, 0, 0.0, v, ld))
        return self

    def _push_act(self, kind, alpha=0.0):
        self.nodes.append((8, kind, float(np.float32(alpha)), None, 0))
        return self

    # scalar / vector ops (graph.rs:103-331)
    def add_scalar(self, v): return self._scalar(0, v)
    def mul_scalar(self, v): return self._scalar(1, v)
    def sub_scalar(self, v): return self._scalar(11, v)
    def div_scalar(self, v): return self._scalar(15, v)
    def max(self, lo): return self._scalar(9, lo)
    def min(self, hi): return self._scalar(10, hi)
    def clamp(self, lo, hi): return self.max(lo).min(hi)
    def add_row(self, r): return self._vec(2, r)
    def mul_row(self, r): return self._vec(3, r)
    def sub_row(self, r): return self._vec(12, r)
    def div_row(self, r): return self._vec(16, r)
    def max_row(self, r): return self._vec(19, r)
    def min_row(self, r): return self._vec(22, r)
    def add_col(self, c): return self._vec(4, c)
    def mul_col(self, c): return self._vec(5, c)
    def sub_col(self, c): return self._vec(13, c)
    def div_col(self, c): return self._vec(17, c)
    def max_col(self, c): return self._vec(20, c)
    def min_col(self, c): return self._vec(23, c)
    def add_tensor(self, t, ld=0): return self._vec(6, t, ld)
    def mul_tensor(self, t, ld=0): return self._vec(7, t, ld)
    def sub_tensor(self, t, ld=0): return self._vec(14, t, ld)
    def div_tensor(self, t, ld=0): return self._vec(18, t, ld)
    def max_tensor(self, t, ld=0): return self._vec(21, t, ld)
    def min_tensor(self, t, ld=0): return self._vec(24, t, ld)
    # *_tensor_strided (graph.rs / builder.rs:634-670): the ld argument above
    add_tensor_strided = add_tensor
    mul_tensor_strided = mul_tensor
    sub_tensor_strided = sub_tensor
    div_tensor_strided = div_tensor
    max_tensor_strided = max_tensor
    min_tensor_strided = min_tensor

    # trailing activations (graph.rs:193-223)
    def relu(self): self.act = 1; return self
    def gelu(self): self.act = 2; return self
    def silu(self): self.act = 3; return self
    def tanh(self): self.act = 4; return self
    def sigmoid(self): self.act = 5; return self

    # in-order activation nodes (graph.rs:334-431)
    def leaky_relu(self, alpha): return self._push_act(6, alpha)
    def relu6(self): return self._push_act(7)
    def hardsigmoid(self): return self._push_act(8)
    def hardswish(self): return self._push_act(9)
    def abs(self): return self._push_act(10)
    def neg(self): return self._push_act(11)
    def square(self): return self._push_act(12)
    def sign(self): return self._push_act(13)
    def sqrt(self): return self._push_act(14)
    def softsign(self): return self._push_act(15)
    def recip(self): return self._push_act(16)
    def rsqrt(self): return self._push_act(17)
    def exp(self): return self._push_act(18)
    def log(self): return self._push_act(19)
    def elu(self, alpha): return self._push_act(20, alpha)
    def selu(self): return self._push_act(21)
    def softplus(self): return self._push_act(22)
    def mish(self): return self._push_act(23)
    def gelu_exact(self): return self._push_act(24)

    def is_empty(self) -> bool:
        return not self.nodes and self.act is None

    def validate(self, m: int, n: int, device: int | None = None) -> None:
        """validate_ep (src/exec/guard.rs:112-147), plus where the operands
        live: a host-pointer call (`device` None) stages host arrays of f16 /
        bf16 bit patterns; a device call on GPU `device` hands its operands to
        the kernels, so they must be 16-bit, contiguous tensors on that GPU (a
        host array there would be read through a host address by the kernel)."""
        for op, _aux, _s, v, ld in self.nodes:
            if v is not None and device is None:
                if _is_dev(v):
                    raise TypeError("host call: an epilogue operand is a device tensor (pass host arrays, "
                                    "or call with device tensors for A and C)")
                _host_operand(v, self.bf16)
            elif v is not None:
                if not _is_dev(v):
                    raise TypeError(f"device call: an epilogue operand is a host array (pass tensors on "
                                    f"cuda:{device})")
                _dev16(v, None, "epilogue operand", device, self.bf16)
            length = None if v is None else (v.numel() if _is_dev(v) else np.asarray(v).size)
            if op in _ROW and length != m:
                raise ValueError("row operand is per-M (length m)")
            if op in _COL and length != n:
                raise ValueError("col operand is per-N (length n)")
            if op in _TENSOR:
                eld = n if ld == 0 else ld
                if eld < n:
                    raise ValueError("tensor row stride must be >= n")
                if m != 0 and length < (m - 1) * eld + n:
                    raise ValueError("tensor must hold m*n elements (stride ld)")

    def desc(self, n: int):
        """resolve_nodes (src/exec/scalar.rs:28-53): tensor ld 0 -> n, the
        trailing activation appended as a final ACT node. Returns
        (EpDesc16 or None, keepalive)."""
        nodes = []
        keep = []
        for op, aux, scalar, v, ld in self.nodes:
            ptr = None
            if v is not None:
                if not _is_dev(v):
                    v = _host_operand(v, self.bf16)
                keep.append(v)
                ptr = _ptr(v)
            if op in _TENSOR and ld == 0:
                ld = n
            nodes.append(EpNode(op, aux, scalar, ptr, ld))
        if self.act is not None:
            nodes.append(EpNode(8, self.act, 0.0, None, 0))
        if not nodes:
            return None, keep
        arr = (EpNode * len(nodes))(*nodes)
        keep.append(arr)
        d = EpDesc16(len(nodes), C.cast(arr, C.POINTER(EpNode)))
        keep.append(d)
        return d, keep


def _ep_ptr(ep, n):
    if ep is None:
        return None, []
    d, keep = ep.desc(n)
    return (None if d is None else C.addressof(d)), keep


# ---- weight handles -----------------------------------------------------------

class _Handle:
    def __init__(self, h: C.c_void_p, n: int, k: int):
        self._h = h
        self._n = n
        self._k = k

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.smg_weights_destroy(h)
            self._h = None

    def n(self) -> int:
        return self._n

    def k(self) -> int:
        return self._k

    def clone(self):
        """Another device copy of the same weights (device-to-device)."""
        import copy
        h = C.c_void_p()
        _check(lib().smg_weights_clone(self._h, C.byref(h)), "smg_weights_clone")
        c = copy.copy(self)
        c._h = h
        return c

    def device_bytes(self) -> int:
        b = SZ()
        _check(lib().smg_weights_info(self._h, None, None, None, C.byref(b)), "smg_weights_info")
        return b.value

    def device(self) -> int:
        """The GPU ordinal the weights live on (device tensors passed with
        them must be there too)."""
        d = C.c_int()
        _check(lib().smg_weights_device(self._h, C.byref(d)), "smg_weights_device")
        return d.value


class Q4Params:
    """src/kernels/q4/mod.rs:56-103."""

    def __init__(self, block: int = Q4_BLOCK):
        if block <= 0 or block & (block - 1):
            raise ValueError(f"q4 block size must be a power of two, got {block}")
        self._block = block
        self._affine = False

    def affine(self) -> "Q4Params":
        p = Q4Params(self._block)
        p._affine = True
        return p

    def block(self) -> int:
        return self._block

    def is_affine(self) -> bool:
        return self._affine


def _f32(w, size: int) -> np.ndarray:
    w = np.ascontiguousarray(np.asarray(w, dtype=np.float32).ravel())
    if w.size != size:
        raise ValueError("w holds n * k weights")
    return w


def _quantize_q4(w, layout: int, n: int, k: int, p: "Q4Params"):
    """Q4Weights::quantize's arrays (src/kernels/q4/quantize.rs:29-81), on the host."""
    w = _f32(w, n * k)
    nbk = -(-k // p.block())
    quants = np.zeros(-(-(k * n) // 2), np.uint8)
    scales = np.zeros(n * nbk, np.uint16)
    mins = np.zeros(n * nbk, np.uint16) if p.is_affine() else None
    _check(lib().smg_q4_quantize(_ptr(w), layout, n, k, p.block(), int(p.is_affine()), _ptr(quants),
                                 _ptr(scales), None if mins is None else _ptr(mins)), "smg_q4_quantize")
    return quants, scales, mins


def _u8(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.uint8)


def q4_band_sizes(n: int, k: int, block: int):
    """(nibble bytes, scale entries) of Q4Weights' band-major arrays
    (src/kernels/q4/weights.rs:89-113): 128-column bands, 64 bytes a depth,
    scales [band][block][128]."""
    bands, nbk = -(-n // 128), -(-k // block)
    return bands * k * 64, bands * nbk * 128


def lowbit_band_sizes(kind: int, n: int, k: int, block: int):
    """(code bytes, scale entries) of Q2Weights / Q1Weights' band-major arrays
    (src/kernels/lowbit/q2.rs:12-20,148-161, q1.rs:186-201): 64-column bands,
    K padded to a multiple of 16, 16 (Q2) or 8 (Q1) bytes a band per depth,
    scales [band][block][64]."""
    bands, kp, nbk = -(-n // 64), -(-k // 16) * 16, -(-k // block)
    return bands * kp * (16 if kind == 2 else 8), bands * nbk * 64


class Q4Weights(_Handle):
    """Q4 weights kept 4-bit resident on the device (src/kernels/q4/weights.rs:26)."""

    def __init__(self, quants, scales, n: int, k: int, params: Q4Params | None = None,
                 mins=None, _band=False):
        p = params or Q4Params()
        nbk = -(-k // p.block())
        quants = _u8(quants)
        # the library reads exactly these lengths from the host arrays
        q_len, sc_len = q4_band_sizes(n, k, p.block()) if _band else (-(-(k * n) // 2), n * nbk)
        scales = _host16(scales, sc_len, "scales")
        if p.is_affine() != (mins is not None):
            raise ValueError("Q4Form::Affine requires a mins array" if p.is_affine()
                             else "Q4Form::Scale takes no mins array")
        if mins is not None:
            mins = _host16(mins, sc_len, "mins")
        if quants.size != q_len:
            raise ValueError(f"quants is {q_len} bytes" + (" (band-major)" if _band else " (ceil(k*n/2))"))
        _require_device()
        h = C.c_void_p()
        fn = lib().smg_q4_create_band if _band else lib().smg_q4_create
        _check(fn(_ptr(quants), _ptr(scales), None if mins is None else _ptr(mins), n, k,
                  p.block(), C.byref(h)), "smg_q4_create")
        super().__init__(h, n, k)
        self._params = p

    @classmethod
    def new(cls, quants, scales, n, k):
        return cls(quants, scales, n, k)

    @classmethod
    def with_params(cls, quants, scales, mins, n, k, p: Q4Params):
        return cls(quants, scales, n, k, p, mins)

    @classmethod
    def from_band(cls, nibbles, scales, mins, n, k, p: Q4Params):
        """From the reference's band-major resident arrays (what src/ffi.rs passes)."""
        return cls(nibbles, scales, n, k, p, mins, _band=True)

    @classmethod
    def quantize(cls, w, layout: int, n: int, k: int, p: Q4Params | None = None):
        """Q4Weights::quantize (src/kernels/q4/quantize.rs:29): f32 weights in
        `layout` (WeightLayout.OutIn / InOut) to Q4_0 (p.affine() for Q4_1)."""
        p = p or Q4Params()
        quants, scales, mins = _quantize_q4(w, layout, n, k, p)
        return cls(quants, scales, n, k, p, mins)

    def params(self) -> Q4Params:
        return self._params

    def permute_columns(self, perm) -> "Q4Weights":
        """Q4Weights::permute_columns (src/kernels/q4/weights.rs:128): output
        column j is column perm[j]; codes, scales and mins move unchanged."""
        import copy
        perm = np.ascontiguousarray(perm, dtype=np.uintp)
        if perm.size != self._n:
            raise ValueError("perm reorders all n columns")
        h = C.c_void_p()
        _check(lib().smg_q4_permute_columns(self._h, _ptr(perm), C.byref(h)), "smg_q4_permute_columns")
        c = copy.copy(self)
        c._h = h
        return c


class Q2Params:
    """src/kernels/lowbit/mod.rs:38-94."""

    def __init__(self, block: int = Q2_BLOCK):
        if block & (block - 1) or not (16 <= block <= 1 << 16):
            raise ValueError(f"q2 block size must be a power of two from 16 to 65536, got {block}")
        self._block = block
        self._codebook = tuple(Q2_TERNARY)

    def with_codebook(self, values) -> "Q2Params":
        """Q2Params::with_codebook (src/kernels/lowbit/mod.rs:74-81): the four
        int8 values codes 0..3 stand for (an `[i8; 4]` in the reference)."""
        vals = tuple(int(v) for v in values)
        if len(vals) != 4 or any(not -128 <= v <= 127 for v in vals):
            raise ValueError(f"a Q2 codebook is exactly 4 int8 values, got {values!r}")
        p = Q2Params(self._block)
        p._codebook = vals
        return p

    def block(self) -> int:
        return self._block

    def codebook(self):
        return self._codebook


class WeightLayout:
    OutIn = 0
    InOut = 1


class Q2Weights(_Handle):
    """2-bit weights resident on the device (src/kernels/lowbit/q2.rs:31)."""

    def __init__(self, codes, scales, n: int, k: int, p: Q2Params | None = None, _band=False):
        p = p or Q2Params()
        nbk = -(-k // p.block())
        codes = _u8(codes)
        c_len, sc_len = lowbit_band_sizes(2, n, k, p.block()) if _band else (-(-(k * n) // 4), n * nbk)
        if codes.size != c_len:
            raise ValueError(f"codes is {c_len} bytes" + (" (band-major)" if _band else " (ceil(k*n/4))"))
        scales = _host16(scales, sc_len, "scales")
        cb = np.asarray(p.codebook(), np.int8)
        _require_device()
        h = C.c_void_p()
        fn = lib().smg_q2_create_band if _band else lib().smg_q2_create
        _check(fn(_ptr(codes), _ptr(scales), _ptr(cb), n, k, p.block(), C.byref(h)),
               "smg_q2_create")
        super().__init__(h, n, k)
        self._params = p

    @classmethod
    def from_band(cls, codes, scales, n, k, p: Q2Params):
        return cls(codes, scales, n, k, p, _band=True)

    @classmethod
    def quantize(cls, w, layout: int, n: int, k: int, p: Q2Params | None = None):
        """Q2Weights::quantize (src/kernels/lowbit/q2.rs:110): each weight to the
        nearest scaled codebook value, scale = f16(amax / max|codebook|)."""
        p = p or Q2Params()
        codes, scales = quantize_q2_arrays(w, layout, n, k, p)
        return cls(codes, scales, n, k, p)

    def params(self) -> Q2Params:
        return self._params


class Q1Weights(_Handle):
    """1-bit weights resident on the device (src/kernels/lowbit/q1.rs:23)."""

    def __init__(self, signs, scales, layout: int, n: int, k: int, block: int, _band=False):
        if block & (block - 1) or not (16 <= block <= 1 << 16):
            raise ValueError(f"q1 block size must be a power of two from 16 to 65536, got {block}")
        nbk = -(-k // block)
        signs = _u8(signs)
        s_len, sc_len = lowbit_band_sizes(1, n, k, block) if _band else (-(-(k * n) // 8), n * nbk)
        if signs.size != s_len:
            raise ValueError(f"signs is {s_len} bytes" + (" (band-major)" if _band else " (ceil(k*n/8))"))
        scales = _host16(scales, sc_len, "scales")
        _require_device()
        h = C.c_void_p()
        if _band:
            rc = lib().smg_q1_create_band(_ptr(signs), _ptr(scales), n, k, block, C.byref(h))
        else:
            rc = lib().smg_q1_create(_ptr(signs), _ptr(scales), int(layout), n, k, block,
                                     C.byref(h))
        _check(rc, "smg_q1_create")
        super().__init__(h, n, k)
        self._block = block

    @classmethod
    def from_band(cls, signs, scales, n, k, block):
        return cls(signs, scales, 0, n, k, block, _band=True)

    @classmethod
    def quantize(cls, w, layout: int, n: int, k: int, block: int):
        """Q1Weights::quantize (src/kernels/lowbit/q1.rs:116): scale = the block's
        mean magnitude, sign = w >= 0."""
        signs, scales = quantize_q1_arrays(w, layout, n, k, block)
        return cls(signs, scales, WeightLayout.OutIn, n, k, block)

    def block(self) -> int:
        return self._block

    @classmethod
    def interleave(cls, gate: "Q1Weights", up: "Q1Weights") -> "Q1Weights":
        """Q1Weights::interleave (src/kernels/lowbit/q1.rs:149): 2n columns,
        each 32-column chunk of gate followed by the same chunk of up."""
        import copy
        h = C.c_void_p()
        _check(lib().smg_q1_interleave(gate._h, up._h, C.byref(h)), "smg_q1_interleave")
        c = copy.copy(gate)
        c._h = h
        c._n = 2 * gate.n()
        return c


def quantize_q4_arrays(w, layout: int, n: int, k: int, p: Q4Params | None = None):
    """(quants, scales, mins) of Q4Weights::quantize, host arrays (no device)."""
    return _quantize_q4(w, layout, n, k, p or Q4Params())


def quantize_q2_arrays(w, layout: int, n: int, k: int, p: Q2Params | None = None):
    """(codes, scales) of Q2Weights::quantize, host arrays (no device)."""
    p = p or Q2Params()
    w = _f32(w, n * k)
    nbk = -(-k // p.block())
    codes = np.zeros(-(-(k * n) // 4), np.uint8)
    scales = np.zeros(n * nbk, np.uint16)
    cb = np.asarray(p.codebook(), np.int8)
    _check(lib().smg_q2_quantize(_ptr(w), layout, n, k, p.block(), _ptr(cb), _ptr(codes), _ptr(scales)),
           "smg_q2_quantize")
    return codes, scales


def quantize_q1_arrays(w, layout: int, n: int, k: int, block: int):
    """(signs in WeightLayout.OutIn, scales) of Q1Weights::quantize, host arrays."""
    w = _f32(w, n * k)
    nbk = -(-k // block)
    signs = np.zeros(-(-(k * n) // 8), np.uint8)
    scales = np.zeros(n * nbk, np.uint16)
    _check(lib().smg_q1_quantize(_ptr(w), layout, n, k, block, _ptr(signs), _ptr(scales)),
           "smg_q1_quantize")
    return signs, scales


class Packed(_Handle):
    """Packed<f16> / Packed<bf16> (src/element.rs:87) held on the device."""

    def __init__(self, h, n, k, bf16):
        super().__init__(h, n, k)
        self.bf16 = bf16


def prepack_f16(b, n: int, k: int) -> Packed:
    """prepack_f16 (src/kernels/f16.rs:212): b is row-major k x n."""
    b = _host16(b, k * n, "b")
    _require_device()
    h = C.c_void_p()
    _check(lib().smg_f16_prepack(_ptr(b), n, k, n, 1, C.byref(h)), "smg_f16_prepack")
    return Packed(h, n, k, False)


def prepack_bf16(b, n: int, k: int) -> Packed:
    b = _host16(b, k * n, "b")
    _require_device()
    h = C.c_void_p()
    _check(lib().smg_bf16_prepack(_ptr(b), n, k, n, 1, C.byref(h)), "smg_bf16_prepack")
    return Packed(h, n, k, True)


def _dequant(w: Q4Weights, bf16: bool) -> Packed:
    h = C.c_void_p()
    _check(lib().smg_q4_dequant(w._h, int(bf16), C.byref(h)), "smg_q4_dequant")
    return Packed(h, w.n(), w.k(), bf16)


def dequant_q4(quants, scales, n, k) -> Packed:
    """dequant_q4 (src/kernels/q4/mod.rs:145): eager dequant on the device."""
    return _dequant(Q4Weights(quants, scales, n, k), False)


def dequant_q4_with(quants, scales, mins, n, k, p: Q4Params) -> Packed:
    return _dequant(Q4Weights(quants, scales, n, k, p, mins), False)


def dequant_q4_bf16(quants, scales, n, k) -> Packed:
    return _dequant(Q4Weights(quants, scales, n, k), True)


def dequant_q4_bf16_with(quants, scales, mins, n, k, p: Q4Params) -> Packed:
    return _dequant(Q4Weights(quants, scales, n, k, p, mins), True)


# ---- matmuls --------------------------------------------------------------------

def _run_host_or_dev(name_host, dev_fn, a, w, c, m, ep, extra_dev=()):
    n, k = w.n(), w.k()
    ep = ep or Epilogue()
    if (_is_dev(a)) != (_is_dev(c)):
        raise ValueError("a and c must both be host arrays or both device tensors")
    if _is_dev(a):
        dev = w.device()
        _dev16(a, m * k, "a (m*k)", dev)
        _dev16(c, m * n, "c (m*n)", dev)
        ep.validate(m, n, dev)
        eptr, keep = _ep_ptr(ep, n)
        _check(dev_fn(m, w._h, c.data_ptr(), a.data_ptr(), eptr, *extra_dev, _stream()), name_host)
        return c
    a = _host16(a, m * k, "a")
    if not isinstance(c, np.ndarray) or c.dtype not in (np.uint16, np.float16) or c.size != m * n:
        raise ValueError("c is m*n (uint16/float16 numpy array)")
    if not c.flags["C_CONTIGUOUS"]:
        raise ValueError("c must be contiguous")
    ep.validate(m, n)
    eptr, keep = _ep_ptr(ep, n)
    _check(getattr(lib(), name_host)(m, w._h, c.ctypes.data, a.ctypes.data, eptr), name_host)
    return c


def matmul_q4_ep(a, w: Q4Weights, c, m: int, ep: Epilogue):
    """src/kernels/q4/matmul.rs:21."""
    return _run_host_or_dev("gemm_gpu_f16f16_q4", lambda *x: lib().smg_q4_matmul_dev(*x[:5], 0, x[5]),
                            a, w, c, m, ep)


def q4_chained(a, w: Q4Weights, c, ep: Epilogue | None = None, done=None, ready=None, *, m: int = 1,
               sync=None, wait_us: int = 0) -> bool:
    """One row of matmul_q4_ep as a link of a chain (src/kernels/q4/matmul.rs:116-164).

    Host arrays: ``done`` / ``ready`` are ``ctypes.c_size_t`` words shared with
    other threads (either None); A is read once ``ready`` covers all k depths,
    and ``done`` is raised to n once C is stored. Device tensors: ``done`` /
    ``ready`` are one-element int64 device tensors, raised and awaited by
    kernels (a producer on another stream stores ``ready``), and ``sync`` is a
    two-element int32 device tensor, zero before the first call (element 1
    becomes 1 when a wait of ``wait_us`` microseconds, 0 for 100 ms, expired).
    Returns False, with ``done`` not raised, when the kernel failed, as the
    reference does; the reason is in ``last_error()``.
    """
    ep = ep or Epilogue()
    n, k = w.n(), w.k()
    if _is_dev(a):
        if not _is_dev(c):
            raise ValueError("a is m*k and c is m*n, both device tensors")
        dev = w.device()
        _dev16(a, m * k, "a (m*k)", dev)
        _dev16(c, m * n, "c (m*n)", dev)
        ep.validate(m, n, dev)
        eptr, keep = _ep_ptr(ep, n)
        ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
        return lib().smg_q4_chained_dev(m, w._h, c.data_ptr(), a.data_ptr(), eptr, ptr(done), ptr(ready),
                                        ptr(sync), wait_us, _stream()) == 0
    a = _host16(a, m * k, "a")
    if not isinstance(c, np.ndarray) or c.dtype not in (np.uint16, np.float16) or c.size != m * n:
        raise ValueError("c is m*n (uint16/float16 numpy array)")
    ep.validate(m, n)
    eptr, keep = _ep_ptr(ep, n)
    ref = lambda x: None if x is None else C.addressof(x)  # noqa: E731
    return lib().gemm_gpu_f16f16_q4_chained(m, w._h, c.ctypes.data, a.ctypes.data, eptr, ref(done),
                                            ref(ready)) == 0


def last_error() -> str:
    """Text of the calling thread's last error in the library."""
    return lib().smg_last_error().decode()


def matmul_q4(a, w: Q4Weights, c, m: int):
    return matmul_q4_ep(a, w, c, m, Epilogue())


def matmul_q4_bf16_ep(a, w: Q4Weights, c, m: int, ep: Epilogue):
    """src/kernels/q4/matmul.rs:187."""
    return _run_host_or_dev("gemm_gpu_b16b16_q4", lambda *x: lib().smg_q4_matmul_dev(*x[:5], 1, x[5]),
                            a, w, c, m, ep)


def matmul_q4_bf16(a, w: Q4Weights, c, m: int):
    return matmul_q4_bf16_ep(a, w, c, m, Epilogue())


def matmul_q2_ep(a, w: Q2Weights, c, m: int, ep: Epilogue):
    """src/kernels/lowbit/matmul.rs:48."""
    return _run_host_or_dev("gemm_gpu_f16_q2", lib().smg_lowbit_matmul_dev, a, w, c, m, ep)


def matmul_q2(a, w: Q2Weights, c, m: int):
    return matmul_q2_ep(a, w, c, m, Epilogue())


def matmul_q1_ep(a, w: Q1Weights, c, m: int, ep: Epilogue):
    """src/kernels/lowbit/matmul.rs:79."""
    return _run_host_or_dev("gemm_gpu_f16_q1", lib().smg_lowbit_matmul_dev, a, w, c, m, ep)


def matmul_q1(a, w: Q1Weights, c, m: int):
    return matmul_q1_ep(a, w, c, m, Epilogue())


def matmul_q2_mopa_ep(a, w: Q2Weights, c, m: int, ep: Epilogue):
    """src/kernels/lowbit/matmul.rs:107."""
    return _run_host_or_dev("gemm_gpu_f16f16_q2", lib().smg_lowbit_mopa_dev, a, w, c, m, ep)


def matmul_q2_mopa(a, w: Q2Weights, c, m: int):
    return matmul_q2_mopa_ep(a, w, c, m, Epilogue())


def matmul_q1_mopa_ep(a, w: Q1Weights, c, m: int, ep: Epilogue):
    """src/kernels/lowbit/matmul.rs:131."""
    return _run_host_or_dev("gemm_gpu_f16f16_q1", lib().smg_lowbit_mopa_dev, a, w, c, m, ep)


def matmul_q1_mopa(a, w: Q1Weights, c, m: int):
    return matmul_q1_mopa_ep(a, w, c, m, Epilogue())


class Gemm:
    """Gemm::new(&a, &packed, m) builder (src/exec/builder.rs:220-814) over a
    device-resident Packed<f16>/<bf16>: row-major output, beta = 1 and no
    epilogue until configured."""

    def __init__(self, a, packed: Packed, m: int):
        self.a = a
        self.packed = packed
        self.m = m
        self._beta = 0x3F80 if packed.bf16 else 0x3C00
        self.ep = Epilogue(packed.bf16)
        self._col_major = False

    def col_major_output(self) -> "Gemm":
        self._col_major = True
        return self

    def beta(self, v) -> "Gemm":
        """Gemm::beta(v: T): a value (int or float, rounded to T), or T's bit
        pattern given explicitly as np.uint16."""
        self._beta = _bits16(v, self.packed.bf16)
        return self

    def __getattr__(self, name):
        # every Epilogue builder method, chained on this Gemm
        fn = getattr(self.ep, name)

        def chain(*args):
            fn(*args)
            return self
        return chain

    def run(self, c):
        m, n, k = self.m, self.packed.n(), self.packed.k()
        dst_cs, dst_rs = (m, 1) if self._col_major else (1, n)
        if _is_dev(self.a):
            dev = self.packed.device()
            _dev16(self.a, m * k, "a (m*k)", dev, self.packed.bf16)
            _dev16(c, m * n, "c (m*n)", dev, self.packed.bf16)
            self.ep.validate(m, n, dev)
            eptr, keep = _ep_ptr(self.ep, n)
            _check(lib().smg_packed_matmul_dev(m, self.packed._h, c.data_ptr(), dst_cs, dst_rs,
                                               self.a.data_ptr(), 1, k, self._beta, eptr,
                                               int(self.packed.bf16), _stream()),
                   "smg_packed_matmul_dev")
            return c
        a = _host16(self.a, m * k, "a")
        if c.size != m * n:
            raise ValueError("c is m*n")
        self.ep.validate(m, n)
        eptr, keep = _ep_ptr(self.ep, n)
        fn = lib().gemm_gpu_b16b16_run_packed if self.packed.bf16 else lib().gemm_gpu_f16f16_run_packed
        _check(fn(m, n, k, c.ctypes.data, dst_cs, dst_rs, 0, a.ctypes.data, 1, k, self.packed._h,
                  0, self._beta, eptr), "run_packed")
        return c


def matmul_f16_packed(a, packed: Packed, c, m: int):
    """src/kernels/f16.rs:255."""
    return Gemm(a, packed, m).run(c)


def matmul_bf16_packed(a, packed: Packed, c, m: int):
    return Gemm(a, packed, m).run(c)


class Accum:
    """Accum (src/element.rs:19-27): the accumulation the reference's SME
    kernels use. On this device every choice accumulates in f32, as the
    portable path those kernels fall back to (src/reference.rs:308-387)."""
    F32 = 0
    F16 = 1
    Bf16 = 2


def _check_strided(what, length, d0, rs, d1, cs):
    """check_strided (src/exec/guard.rs:49-60)."""
    if d0 == 0 or d1 == 0:
        return
    if min(rs, cs) < 0 or (d0 - 1) * rs + (d1 - 1) * cs >= length:
        raise ValueError(f"{what}: {d0}x{d1} view at strides {rs}/{cs} overflows the slice (len {length})")


def _bits16(v, bf16):
    """A scalar of T (f16 or bf16) as its bit pattern. Python ints and floats
    are values, rounded to T (alpha=0, beta=1 mean 0.0 and 1.0, as the
    reference's `alpha: T`); only an np.uint16 is taken as raw bits."""
    if isinstance(v, np.uint16):
        return int(v)
    if isinstance(v, bool) or not isinstance(v, (int, float, np.floating, np.integer)):
        raise TypeError(f"alpha/beta: a number or np.uint16 bits, got {type(v).__name__}")
    if bf16:
        return int(np.float32(_bf16_round(float(v))).view(np.uint32)) >> 16
    return int(np.float16(float(v)).view(np.uint16))


def _gemm_host16(v, bf16: bool, name: str) -> np.ndarray:
    """A host GEMM operand as its 16-bit patterns: uint16 bits, or float16
    values for an f16 GEMM. Any other dtype is refused rather than
    reinterpreted (a float32 array viewed as uint16 is twice as many
    meaningless halves)."""
    arr = np.asarray(v)
    if arr.dtype == np.uint16 or (arr.dtype == np.float16 and not bf16):
        return arr
    raise TypeError(f"{name}: expected {'uint16 bf16 bits' if bf16 else 'float16 or uint16 bits'}, got {arr.dtype}")


def _gemm_strided(bf16, m, n, k, c, c_rs, c_cs, a, a_rs, a_cs, b, b_rs, b_cs, alpha, beta, accum):
    if m == 0 or n == 0:
        return c
    ab, bb = _bits16(alpha, bf16), _bits16(beta, bf16)
    read_dst = int((ab & 0x7FFF) != 0)  # alpha != 0 (+0 and -0 are zero; NaN is not)
    if _is_dev(c):
        dev = c.device.index
        for t, name in ((c, "c"), (a, "a"), (b, "b")):
            if not _is_dev(t):
                raise TypeError(f"{name}: every operand on the device, or every one on the host")
            _dev16(t, None, name, dev, bf16)
        _check_strided("c", c.numel(), m, c_rs, n, c_cs)
        _check_strided("a", a.numel(), m, a_rs, k, a_cs)
        _check_strided("b", b.numel(), k, b_rs, n, b_cs)
        _check(lib().smg_gemm_run_dev(int(bf16), m, n, k, c.data_ptr(), c_cs, c_rs, read_dst, a.data_ptr(), a_cs,
                                      a_rs, b.data_ptr(), b_cs, b_rs, ab, bb, _stream()), "smg_gemm_run_dev")
        return c
    cc = _gemm_host16(c, bf16, "c")
    if not cc.flags.c_contiguous:
        raise TypeError("c: a contiguous array (updated in place)")
    av = np.ascontiguousarray(_gemm_host16(a, bf16, "a")).view(np.uint16).ravel()
    bv = np.ascontiguousarray(_gemm_host16(b, bf16, "b")).view(np.uint16).ravel()
    _check_strided("c", cc.size, m, c_rs, n, c_cs)
    _check_strided("a", av.size, m, a_rs, k, a_cs)
    _check_strided("b", bv.size, k, b_rs, n, b_cs)
    _require_device()
    if bf16:
        fn = lib().gemm_gpu_b16b16_run if accum == Accum.Bf16 else lib().gemm_gpu_bf16f32_run
    else:
        fn = lib().gemm_gpu_f16f16_run if accum == Accum.F16 else lib().gemm_gpu_f16f32_run
    _check(fn(m, n, k, cc.ctypes.data, c_cs, c_rs, read_dst, av.ctypes.data, a_cs, a_rs, bv.ctypes.data, b_cs,
              b_rs, ab, bb), "gemm run")
    return c


def gemm_f16(m, n, k, c, c_row_stride, c_col_stride, a, a_row_stride, a_col_stride, b, b_row_stride,
             b_col_stride, alpha, beta, accum=Accum.F32):
    """gemm_f16 (src/kernels/f16.rs:126-204): C = alpha*C + beta*(A @ B) over
    strided f16 views (host arrays, C updated in place; or device tensors);
    C is read only when alpha != 0."""
    return _gemm_strided(False, m, n, k, c, c_row_stride, c_col_stride, a, a_row_stride, a_col_stride, b,
                         b_row_stride, b_col_stride, alpha, beta, accum)


def gemm_bf16(m, n, k, c, c_row_stride, c_col_stride, a, a_row_stride, a_col_stride, b, b_row_stride,
              b_col_stride, alpha, beta, accum=Accum.F32):
    """gemm_bf16 (src/kernels/bf16.rs:140-200)."""
    return _gemm_strided(True, m, n, k, c, c_row_stride, c_col_stride, a, a_row_stride, a_col_stride, b,
                         b_row_stride, b_col_stride, alpha, beta, accum)


def matmul_f16(a, b, c, m, n, k, accum=Accum.F32):
    """matmul_f16 (src/kernels/f16.rs:89-111): row-major C = A @ B."""
    for t, sz, name in ((a, m * k, "a is m*k"), (b, k * n, "b is k*n"), (c, m * n, "c is m*n")):
        if (t.numel() if _is_dev(t) else np.asarray(t).size) != sz:
            raise ValueError(name)
    return gemm_f16(m, n, k, c, n, 1, a, k, 1, b, n, 1, 0.0, 1.0, accum)


def matmul_bf16(a, b, c, m, n, k, accum=Accum.F32):
    """matmul_bf16 (src/kernels/bf16.rs:101-137)."""
    for t, sz, name in ((a, m * k, "a is m*k"), (b, k * n, "b is k*n"), (c, m * n, "c is m*n")):
        if (t.numel() if _is_dev(t) else np.asarray(t).size) != sz:
            raise ValueError(name)
    return gemm_bf16(m, n, k, c, n, 1, a, k, 1, b, n, 1, 0.0, 1.0, accum)


# ---- the model-level parts: Linear, GatedLinear, Mlp, KvCache, SelfAttention,
# ---- Norm, Block and the nn passes (src/linear.rs, src/mlp.rs,
# ---- src/self_attention.rs, src/kernels/kv_attention.rs, src/nn.rs, src/block.rs)
#
# They run on device tensors (torch, on torch's current stream): residual
# streams float32, activations handed between parts float16, as the
# reference's f32 residual / f16 kernel inputs (src/linear.rs:14-29).

class Gate:
    """src/linear.rs:563-575: the activation an MLP applies (silu / tanh gelu)."""
    Silu = EP_ACT["silu"]
    Gelu = EP_ACT["gelu"]


def _take(w: _Handle) -> C.c_void_p:
    """Hands a weight handle over to a part that takes it over (the reference's
    constructors move their Linears): the Python object no longer owns it."""
    h = w._h
    if not h:
        raise ValueError("these weights were already handed to another part")
    w._h = None
    return h


def _f32dev(x, n, what, device):
    if x.dtype.itemsize != 4 or not x.is_floating_point():
        raise TypeError(f"{what}: expected a float32 tensor, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if device is not None and x.device.index != device:
        raise ValueError(f"{what} is on cuda:{x.device.index}, the weights on cuda:{device}")
    if n is not None and x.numel() != n:
        raise ValueError(f"{what} has {x.numel()} elements, expected {n}")
    return x


class Linear:
    """A 4-bit linear layer y = x @ W, n outputs by k inputs (src/linear.rs:139):
    Linear::from_q4 / quantize over resident Q4Weights."""

    def __init__(self, q4: Q4Weights):
        self.q4 = q4

    @classmethod
    def from_q4(cls, q4: Q4Weights) -> "Linear":
        return cls(q4)

    @classmethod
    def quantize(cls, w, layout: int, n: int, k: int, p: Q4Params | None = None) -> "Linear":
        """Linear::quantize / quantize_with (src/linear.rs:178-193)."""
        return cls(Q4Weights.quantize(w, layout, n, k, p))

    def n(self) -> int:
        return self.q4.n()

    def k(self) -> int:
        return self.q4.k()

    def forward(self, x, y, m: int):
        """Linear::forward (src/linear.rs:373): y = x @ W, f16."""
        return matmul_q4(x, self.q4, y, m)

    def forward_ep(self, x, y, m: int, ep: Epilogue):
        return matmul_q4_ep(x, self.q4, y, m, ep)

    def accumulate(self, x, y, m: int):
        """Linear::accumulate (src/linear.rs:425-432): y (f32) += f32(f16(x @ W)).
        Host arrays (x f16 or f32, y float32 numpy, updated in place) or
        device tensors (x f16, y float32)."""
        if not _same_side(x, y):
            xh = _host_x16(x, m * self.k(), "x (m*k)")
            _host_out(y, m * self.n(), (np.float32,), "y (m*n)")
            _check(lib().smg_q4_accumulate(m, self.q4._h, y.ctypes.data, xh.ctypes.data), "smg_q4_accumulate")
            return y
        dev = self.q4.device()
        _dev16(x, m * self.k(), "x (m*k)", dev, False)
        _f32dev(y, m * self.n(), "y (m*n)", dev)
        _check(lib().smg_q4_accumulate_dev(m, self.q4._h, y.data_ptr(), x.data_ptr(), _stream()),
               "smg_q4_accumulate_dev")
        return y


class GatedLinear:
    """act(x @ W_gate) * (x @ W_up) as one 2n-output Q4 Linear, gate and up
    interleaved 32 columns at a time (src/linear.rs:596-801)."""

    def __init__(self, inner: Linear, gate: int):
        if inner.n() % 2:
            raise ValueError("a gated layer has 2n outputs")
        self.inner = inner
        self._gate = gate

    @classmethod
    def quantize(cls, w_gate, w_up, layout: int, n: int, k: int, gate: int,
                 p: Q4Params | None = None) -> "GatedLinear":
        """GatedLinear::quantize / quantize_with (src/linear.rs:625-671)."""
        def inout(w):
            w = np.asarray(w, np.float32).reshape(-1)
            if w.size != n * k:
                raise ValueError("w holds n * k weights")
            return w.reshape(n, k).T if layout == WeightLayout.OutIn else w.reshape(k, n)
        g, u = inout(w_gate), inout(w_up)
        parts = []
        for c0 in range(0, n, 32):
            c1 = min(c0 + 32, n)
            parts += [g[:, c0:c1], u[:, c0:c1]]
        both = np.ascontiguousarray(np.concatenate(parts, axis=1))
        return cls(Linear.quantize(both, WeightLayout.InOut, 2 * n, k, p), gate)

    @classmethod
    def from_q4(cls, gate_w: Q4Weights, up_w: Q4Weights, gate: int) -> "GatedLinear":
        """The interleave of two Q4 weight sets, exactly (as
        GatedLinear::from_q1 does for 1-bit weights, src/linear.rs:697-704)."""
        import copy
        h = C.c_void_p()
        _check(lib().smg_q4_interleave(gate_w._h, up_w._h, C.byref(h)), "smg_q4_interleave")
        c = copy.copy(gate_w)
        c._h = h
        c._n = 2 * gate_w.n()
        return cls(Linear(c), gate)

    def n(self) -> int:
        return self.inner.n() // 2

    def k(self) -> int:
        return self.inner.k()

    def gate(self) -> int:
        return self._gate

    def forward(self, x, y, m: int):
        """GatedLinear::forward (src/linear.rs:779-791): the 2n-output GEMV, then glu."""
        import torch
        both = torch.empty(m * 2 * self.n(), dtype=torch.float16, device=x.device)
        self.inner.forward(x, both, m)
        return glu(both, m, self.n(), self._gate, y)


class Mlp:
    """y += down(act(up(x))) (Mlp::new) or y += down(act(x @ W_gate) * (x @ W_up))
    (Mlp::gated), src/mlp.rs:56-149: the up GEMV with its activation (or glu)
    at the store, then the down GEMV adding into y. Takes over its layers."""

    def __init__(self, up, act: int, down: Linear, gated: bool):
        if down.k() != (up.n()):
            raise ValueError("down takes up's outputs")
        self._k, self._n, self._hidden = up.k(), down.n(), up.n()
        upw = up.inner.q4 if gated else up.q4
        h = C.c_void_p()
        _check(lib().smg_mlp_create(upw._h, down.q4._h, act, int(gated), C.byref(h)), "smg_mlp_create")
        _take(upw)
        _take(down.q4)
        self._h = h
        self._device = torch_device_index()

    @classmethod
    def new(cls, up: Linear, act: int, down: Linear) -> "Mlp":
        return cls(up, act, down, False)

    @classmethod
    def gated(cls, up: GatedLinear, down: Linear) -> "Mlp":
        return cls(up, up.gate(), down, True)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.smg_mlp_destroy(h)
            self._h = None

    def k(self) -> int:
        return self._k

    def n(self) -> int:
        return self._n

    def hidden(self) -> int:
        return self._hidden

    def accumulate(self, x, y, m: int):
        """Mlp::accumulate (src/mlp.rs:113-149): y (f32 m x n) += ... for x f16
        (host arrays, where x may also be f32, or device tensors)."""
        if not _same_side(x, y):
            xh = _host_x16(x, m * self._k, "x (m*k)")
            _host_out(y, m * self._n, (np.float32,), "y (m*n)")
            _check(lib().smg_mlp_accumulate(self._h, xh.ctypes.data, y.ctypes.data, m), "Mlp::accumulate")
            return y
        _dev16(x, m * self._k, "x (m*k)", self._device, False)
        _f32dev(y, m * self._n, "y (m*n)", self._device)
        _check(lib().smg_mlp_accumulate_dev(self._h, x.data_ptr(), y.data_ptr(), m, _stream()),
               "smg_mlp_accumulate_dev")
        return y


def torch_device_index() -> int:
    import torch
    return torch.cuda.current_device()


class KvCache:
    """An f16 key/value cache for one attention layer on the device
    (src/kernels/kv_attention.rs:342-578)."""

    def __init__(self, heads: int, kv_heads: int, head_dim: int, capacity: int):
        h = C.c_void_p()
        _check(lib().smg_kv_cache_create(heads, kv_heads, head_dim, capacity, C.byref(h)),
               "KvCache::new")
        self._h = h
        self._heads, self._kv_heads, self._hd = heads, kv_heads, head_dim
        self._device = torch_device_index()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.smg_kv_cache_destroy(h)
            self._h = None

    def _info(self):
        ln, cap, sc = SZ(), SZ(), C.c_float()
        _check(lib().smg_kv_cache_info(self._h, C.byref(ln), C.byref(cap), C.byref(sc)), "smg_kv_cache_info")
        return ln.value, cap.value, sc.value

    def with_scale(self, scale: float) -> "KvCache":
        _check(lib().smg_kv_cache_set_scale(self._h, float(np.float32(scale))), "with_scale")
        return self

    def len(self) -> int:
        return self._info()[0]

    def is_empty(self) -> bool:
        return self.len() == 0

    def capacity(self) -> int:
        return self._info()[1]

    def scale(self) -> float:
        return self._info()[2]

    def heads(self) -> int:
        return self._heads

    def kv_heads(self) -> int:
        return self._kv_heads

    def head_dim(self) -> int:
        return self._hd

    def row_len(self) -> int:
        return self._kv_heads * self._hd

    def query_len(self) -> int:
        return self._heads * self._hd

    def clear(self):
        _check(lib().smg_kv_cache_truncate(self._h, 0), "clear")

    def truncate(self, length: int):
        _check(lib().smg_kv_cache_truncate(self._h, length), "truncate")

    def extend(self, k, v):
        """KvCache::extend (kv_attention.rs:499-519): whole rows of f16 keys and values."""
        row = self.row_len()
        if not _same_side(k, v):
            kh, vh = np.asarray(k), np.asarray(v)
            if kh.size != vh.size or kh.size % row or kh.size == 0:
                raise ValueError("k and v hold the same whole number of kv_heads * head_dim rows")
            kh = _host_x16(kh, kh.size, "k")
            vh = _host_x16(vh, vh.size, "v")
            _check(lib().smg_kv_cache_extend(self._h, kh.ctypes.data, vh.ctypes.data, kh.size // row),
                   "KvCache::extend")
            return
        if k.numel() != v.numel() or k.numel() % row or k.numel() == 0:
            raise ValueError("k and v hold the same whole number of kv_heads * head_dim rows")
        _dev16(k, None, "k", self._device, False)
        _dev16(v, None, "v", self._device, False)
        _check(lib().smg_kv_cache_extend_dev(self._h, k.data_ptr(), v.data_ptr(), k.numel() // row,
                                             _stream()), "KvCache::extend")

    push = extend

    def _rows(self, which: int):
        """The first len() rows of the keys (0) or values (1), copied into a
        new f16 device tensor (keys() / values(), kv_attention.rs:522-531)."""
        import torch
        n = self.len() * self.row_len()
        out = torch.empty(n, dtype=torch.float16, device=f"cuda:{self._device}")
        if n:
            k = out.data_ptr() if which == 0 else None
            v = out.data_ptr() if which == 1 else None
            _check(lib().smg_kv_cache_read_dev(self._h, k, v, _stream()), "smg_kv_cache_read_dev")
        return out

    def keys(self):
        return self._rows(0)

    def values(self):
        return self._rows(1)

    def keys_host(self) -> np.ndarray:
        """keys() copied into a new float16 numpy array."""
        return self._rows_host(0)

    def values_host(self) -> np.ndarray:
        """values() copied into a new float16 numpy array."""
        return self._rows_host(1)

    def _rows_host(self, which: int) -> np.ndarray:
        out = np.empty(self.len() * self.row_len(), np.float16)
        if out.size:
            p = out.ctypes.data
            _check(lib().smg_kv_cache_read(self._h, p if which == 0 else None, p if which == 1 else None),
                   "smg_kv_cache_read")
        return out

    def attend(self, q, out):
        """KvCache::attend (kv_attention.rs:537-552): q and out f32 heads*head_dim
        (host arrays or device tensors)."""
        if not _same_side(q, out):
            qh = _host_f32(q, self.query_len(), "q")
            _host_out(out, self.query_len(), (np.float32,), "out")
            _check(lib().smg_kv_cache_attend(self._h, qh.ctypes.data, out.ctypes.data), "attend")
            return out
        _f32dev(q, self.query_len(), "q", self._device)
        _f32dev(out, self.query_len(), "out", self._device)
        _check(lib().smg_kv_cache_attend_dev(self._h, q.data_ptr(), out.data_ptr(), _stream()), "attend")
        return out

    def attend_causal(self, q, rows: int, out):
        """KvCache::attend_causal (kv_attention.rs:560-578): `rows` query rows
        that are the last `rows` cached positions, each attending to itself and
        everything before it; q and out f32 rows * heads * head_dim."""
        if rows > self.len():
            raise ValueError(f"attend_causal: {rows} rows but {self.len()} cached")
        if not _same_side(q, out):
            qh = _host_f32(q, rows * self.query_len(), "q")
            _host_out(out, rows * self.query_len(), (np.float32,), "out")
            _check(lib().smg_kv_cache_attend_causal(self._h, qh.ctypes.data, rows, out.ctypes.data),
                   "attend_causal")
            return out
        _f32dev(q, rows * self.query_len(), "q", self._device)
        _f32dev(out, rows * self.query_len(), "out", self._device)
        _check(lib().smg_kv_cache_attend_causal_dev(self._h, q.data_ptr(), rows, out.data_ptr(), _stream()),
               "attend_causal")
        return out


class SelfAttention:
    """y += out(attention(qkv(x))) over a KvCache (src/self_attention.rs:69-240),
    for m rows (m > 1 attends causally). rope_theta > 0 adds the NeoX rotary
    embedding to q and k as
    examples/bonsai/model.rs:30-99 does (not part of the library's
    SelfAttention). Takes over its two layers."""

    def __init__(self, qkv: Linear, out: Linear, heads: int, kv_heads: int, head_dim: int,
                 rope_theta: float = 0.0):
        if kv_heads <= 0 or heads <= 0 or heads % kv_heads:
            raise ValueError("heads must be a positive multiple of kv_heads")
        if qkv.n() != (heads + 2 * kv_heads) * head_dim:
            raise ValueError("qkv has (heads + 2 kv_heads) * head_dim outputs")
        if out.k() != heads * head_dim:
            raise ValueError("out takes heads * head_dim inputs")
        self._width, self._out_width = qkv.k(), out.n()
        self._heads, self._kv_heads, self._hd = heads, kv_heads, head_dim
        h = C.c_void_p()
        _check(lib().smg_attn_create(qkv.q4._h, out.q4._h, heads, kv_heads, head_dim, float(rope_theta),
                                     C.byref(h)), "SelfAttention::new")
        _take(qkv.q4)
        _take(out.q4)
        self._h = h
        self._device = torch_device_index()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.smg_attn_destroy(h)
            self._h = None

    def width(self) -> int:
        return self._width

    def out_width(self) -> int:
        return self._out_width

    def cache(self, capacity: int) -> KvCache:
        return KvCache(self._heads, self._kv_heads, self._hd, capacity)

    def accumulate(self, x, cache: KvCache, y, m: int):
        """SelfAttention::accumulate (self_attention.rs:148-183): m rows at the
        cache's next m positions (attend_rows, :192-240, for m > 1). Host
        arrays (x f16 or f32, y float32, updated in place) or device tensors."""
        if not _same_side(x, y):
            xh = _host_x16(x, m * self._width, "x (m*width)")
            _host_out(y, m * self._out_width, (np.float32,), "y (m*out.n)")
            _check(lib().smg_attn_accumulate(self._h, xh.ctypes.data, cache._h, y.ctypes.data, m),
                   "SelfAttention::accumulate")
            return y
        _dev16(x, m * self._width, "x (m*width)", self._device, False)
        _f32dev(y, m * self._out_width, "y (m*out.n)", self._device)
        _check(lib().smg_attn_accumulate_dev(self._h, x.data_ptr(), cache._h, y.data_ptr(), m, _stream()),
               "SelfAttention::accumulate")
        return y


class Norm:
    """nn::Norm (src/nn.rs:164-235): Norm::layer (GPT-2's LayerNorm, optional
    bias) or Norm::rms (Llama's RMSNorm)."""

    def __init__(self, weight, eps: float, bias=None, rms: bool = True):
        w = np.ascontiguousarray(np.asarray(weight, np.float32).ravel())
        if w.size == 0:
            raise ValueError("a norm needs at least one feature")
        b = None
        if bias is not None:
            b = np.ascontiguousarray(np.asarray(bias, np.float32).ravel())
            if b.size != w.size:
                raise ValueError("bias holds weight.len() values")
        self.weight = w
        self.bias = b
        self.eps = float(np.float32(eps))
        self.rms_kind = rms
        self._dev = None

    @classmethod
    def rms(cls, weight, eps: float) -> "Norm":
        return cls(weight, eps)

    @classmethod
    def layer(cls, weight, bias, eps: float) -> "Norm":
        """Norm::layer(weight, bias, eps) (src/nn.rs:187-198); bias may be None."""
        return cls(weight, eps, bias, rms=False)

    def width(self) -> int:
        return self.weight.size

    def forward(self, x, y):
        """Norm::forward (src/nn.rs:227): f32 rows x to f16 y (host arrays or
        device tensors)."""
        if not _same_side(x, y):
            if self.rms_kind:
                return rms_norm(x, self.weight, self.eps, y)
            return layer_norm(x, self.weight, self.bias, self.eps, y)
        import torch
        if self._dev is None:
            self._dev = (torch.from_numpy(self.weight).cuda(),
                         None if self.bias is None else torch.from_numpy(self.bias).cuda())
        if self.rms_kind:
            return rms_norm(x, self._dev[0], self.eps, y)
        return layer_norm(x, self._dev[0], self._dev[1], self.eps, y)


class Block:
    """A pre-norm transformer layer over an f32 residual stream
    (src/block.rs:40-107): x += attn(norm1(x)), then x += mlp(norm2(x)).
    Takes over its attention and MLP."""

    def __init__(self, norm1: Norm, attn: SelfAttention, norm2: Norm, mlp: Mlp):
        d = attn.width()
        if not (norm1.width() == d and attn.out_width() == d and norm2.width() == d and mlp.k() == d
                and mlp.n() == d):
            raise ValueError("the norms, attention and MLP share the residual's width")
        h = C.c_void_p()
        bp = lambda nm: None if nm.bias is None else nm.bias.ctypes.data  # noqa: E731
        _check(lib().smg_block_create_norms(norm1.weight.ctypes.data, bp(norm1), norm1.eps, int(not norm1.rms_kind),
                                            norm2.weight.ctypes.data, bp(norm2), norm2.eps, int(not norm2.rms_kind),
                                            d, attn._h, mlp._h, C.byref(h)), "Block::new")
        attn._h = None
        mlp._h = None
        self._h = h
        self._d = d
        self._attn_shape = (attn._heads, attn._kv_heads, attn._hd)
        self._device = torch_device_index()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.smg_block_destroy(h)
            self._h = None

    def width(self) -> int:
        return self._d

    def cache(self, capacity: int) -> KvCache:
        return KvCache(*self._attn_shape, capacity)

    def accumulate(self, x, cache: KvCache, rows: int):
        """Block::accumulate (src/block.rs:90-106): rows rows of the f32
        residual at the cache's next rows positions (causal attention among
        them), which it appends. x a float32 numpy array (host) or device
        tensor, updated in place."""
        if not _is_dev(x):
            _host_out(x, rows * self._d, (np.float32,), "x (rows*width)")
            _check(lib().smg_block_accumulate(self._h, x.ctypes.data, cache._h, rows), "Block::accumulate")
            return x
        _f32dev(x, rows * self._d, "x (rows*width)", self._device)
        _check(lib().smg_block_accumulate_dev(self._h, x.data_ptr(), cache._h, rows, _stream()),
               "Block::accumulate")
        return x


def rms_norm(x, weight, eps: float, y):
    """nn::rms_norm (src/nn.rs:147-161): f32 rows of x to f16 y; weight f32.
    Host arrays (y a float16 / uint16 numpy array) or device tensors."""
    if not _same_side(x, weight, y):
        w = _host_f32(weight, None, "weight")
        xh = _host_f32(x, None, "x")
        if w.size == 0 or xh.size % w.size:
            raise ValueError("x holds whole rows of weight.len()")
        _host_out(y, xh.size, (np.float16, np.uint16), "y")
        _check(lib().smg_rms_norm_f16(xh.ctypes.data, w.ctypes.data, xh.size // w.size, w.size,
                                      float(np.float32(eps)), y.ctypes.data), "rms_norm")
        return y
    dim = weight.numel()
    if dim == 0 or x.numel() % dim:
        raise ValueError("x holds whole rows of weight.len()")
    dev = x.device.index
    _f32dev(x, None, "x", dev)
    _f32dev(weight, dim, "weight", dev)
    _dev16(y, x.numel(), "y", dev, False)
    _check(lib().smg_rms_norm_f16_dev(x.data_ptr(), weight.data_ptr(), x.numel() // dim, dim,
                                      float(np.float32(eps)), y.data_ptr(), _stream()), "rms_norm")
    return y


def layer_norm(x, weight, bias, eps: float, y):
    """nn::layer_norm (src/nn.rs:73-86): f32 rows of x to f16 y; weight (and
    bias, or None) f32. Host arrays (y a float16 / uint16 numpy array) or
    device tensors."""
    if not _same_side(x, weight, bias, y):
        w = _host_f32(weight, None, "weight")
        b = None if bias is None else _host_f32(bias, w.size, "bias")
        xh = _host_f32(x, None, "x")
        if w.size == 0 or xh.size % w.size:
            raise ValueError("x holds whole rows of weight.len()")
        _host_out(y, xh.size, (np.float16, np.uint16), "y")
        _check(lib().smg_layer_norm_f16(xh.ctypes.data, w.ctypes.data, None if b is None else b.ctypes.data,
                                        xh.size // w.size, w.size, float(np.float32(eps)), y.ctypes.data),
               "layer_norm")
        return y
    dim = weight.numel()
    if dim == 0 or x.numel() % dim:
        raise ValueError("x holds whole rows of weight.len()")
    dev = x.device.index
    _f32dev(x, None, "x", dev)
    _f32dev(weight, dim, "weight", dev)
    if bias is not None:
        _f32dev(bias, dim, "bias", dev)
    _dev16(y, x.numel(), "y", dev, False)
    _check(lib().smg_layer_norm_f16_dev(x.data_ptr(), weight.data_ptr(), None if bias is None else bias.data_ptr(),
                                        x.numel() // dim, dim, float(np.float32(eps)), y.data_ptr(), _stream()),
           "layer_norm")
    return y


def attention_kv_causal_f16(q, k, v, start: int, rows: int, heads: int, kv_heads: int, head_dim: int,
                            scale: float, out):
    """attention_kv_causal_f16 (src/kernels/kv_attention.rs:140-240) on device
    tensors or host arrays: query row i attends to keys 0 .. start + i."""
    if rows == 0:
        raise ValueError("attention_kv_causal_f16 needs at least one query row")
    if head_dim % 8 or not 8 <= head_dim <= 256:
        raise ValueError("head_dim must be a multiple of 8 in 8..=256")
    if kv_heads <= 0 or heads <= 0 or heads % kv_heads:
        raise ValueError("heads must be a positive multiple of kv_heads")
    ld = kv_heads * head_dim
    if not _same_side(q, k, v, out):
        n_kv = (start + rows) * ld
        qh = _host_f32(q, rows * heads * head_dim, "q")
        kh = _host_x16(np.asarray(k).ravel()[:n_kv], n_kv, "k")
        vh = _host_x16(np.asarray(v).ravel()[:n_kv], n_kv, "v")
        _host_out(out, rows * heads * head_dim, (np.float32,), "out")
        _check(lib().smg_attention_kv_causal_f16(qh.ctypes.data, kh.ctypes.data, vh.ctypes.data, start, rows,
                                                 heads, kv_heads, head_dim, float(np.float32(scale)),
                                                 out.ctypes.data), "attention_kv_causal_f16")
        return out
    dev = q.device.index
    _f32dev(q, rows * heads * head_dim, "q", dev)
    _f32dev(out, rows * heads * head_dim, "out", dev)
    for t, name in ((k, "k"), (v, "v")):
        _dev16(t, None, name, dev, False)
        if t.numel() < (start + rows) * ld:
            raise ValueError(f"{name} holds (start + rows) * kv_heads * head_dim")
    _check(lib().smg_attention_kv_causal_f16_dev(q.data_ptr(), k.data_ptr(), v.data_ptr(), start, rows, heads,
                                                 kv_heads, head_dim, float(np.float32(scale)), out.data_ptr(),
                                                 _stream()), "attention_kv_causal_f16")
    return out


def glu(both, m: int, n: int, gate: int, y):
    """GatedLinear's glu (src/linear.rs:804-826) over m rows of 2n interleaved f16."""
    dev = both.device.index
    _dev16(both, m * 2 * n, "both", dev, False)
    _dev16(y, m * n, "y", dev, False)
    _check(lib().smg_glu_f16_dev(both.data_ptr(), m, n, gate, y.data_ptr(), _stream()), "glu")
    return y


def attention_kv_f16(q, k, v, length: int, heads: int, kv_heads: int, head_dim: int, scale: float, out):
    """attention_kv_f16 (src/kernels/kv_attention.rs:29-78) on device tensors
    or host arrays."""
    if length == 0:
        raise ValueError("attention_kv_f16 needs at least one cached key")
    if head_dim % 8 or not 8 <= head_dim <= 256:
        raise ValueError("head_dim must be a multiple of 8 in 8..=256")
    if kv_heads <= 0 or heads <= 0 or heads % kv_heads:
        raise ValueError("heads must be a positive multiple of kv_heads")
    ld = kv_heads * head_dim
    if not _same_side(q, k, v, out):
        n_kv = length * ld
        qh = _host_f32(q, heads * head_dim, "q")
        kh = _host_x16(np.asarray(k).ravel()[:n_kv], n_kv, "k")
        vh = _host_x16(np.asarray(v).ravel()[:n_kv], n_kv, "v")
        _host_out(out, heads * head_dim, (np.float32,), "out")
        _check(lib().smg_attention_kv_f16(qh.ctypes.data, kh.ctypes.data, vh.ctypes.data, length, heads, kv_heads,
                                          head_dim, float(np.float32(scale)), out.ctypes.data), "attention_kv_f16")
        return out
    dev = q.device.index
    _f32dev(q, heads * head_dim, "q", dev)
    _f32dev(out, heads * head_dim, "out", dev)
    for t, name in ((k, "k"), (v, "v")):
        _dev16(t, None, name, dev, False)
        if t.numel() < length * ld:
            raise ValueError(f"{name} holds len * kv_heads * head_dim")
    _check(lib().smg_attention_kv_f16_dev(q.data_ptr(), k.data_ptr(), v.data_ptr(), length, heads, kv_heads,
                                          head_dim, float(np.float32(scale)), out.data_ptr(), _stream()),
           "attention_kv_f16")
    return out
