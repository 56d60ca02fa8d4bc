"""GGUF import of ``Q4_0`` / ``Q1_0`` weight tensors into the library's weight
handles.

The reader follows the reference example's loader
(examples/bonsai/gguf.rs:110-170): GGUF version 3 only, metadata values of
every GGUF type, tensor data at ``general.alignment`` (default 32) past the
header, and only types whose blocks it knows: F32, F16 and ``Q1_0`` as there
(gguf.rs:29-37), plus ``Q4_0``, the GGUF type ``Q4Weights`` holds in its scale
form (src/kernels/q4/mod.rs:33-38); anything else is an error. The file is
memory-mapped, so a tensor is a view into it until it is converted.

Block formats (ggml; dims[0] is the row length K, dims[1] the rows N, so a
weight tensor is ``OutIn``):

* ``Q4_0`` (type 2): 32 values per block, an f16 scale ``d`` then 16 bytes;
  byte i holds value i in its low nibble and value i + 16 in its high nibble,
  each an unsigned code u with value ``d * (u - 8)``. The import keeps ``d``
  and the code ``u - 8`` exactly: the handle's input arrays are the reference's
  (``Q4Weights::new``: row-major K x N two's-complement nibbles, low nibble
  first, and scales ``[j * nbk + block]``, src/kernels/q4/mod.rs:206-214).
* ``Q1_0`` (type 41): 128 values per block, an f16 scale then 16 bytes of sign
  bits; the blocks' sign bytes in file order are the ``OutIn`` sign array and
  their scales the scale array, as examples/bonsai/model.rs:132-160 builds its
  ``Q1Weights`` (rows of several tensors stacked in the order named).
"""
from __future__ import annotations

import mmap
import struct

import numpy as np

F32, F16, Q4_0, Q1_0 = 0, 1, 2, 41
# (values per block, bytes per block)
_BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q1_0: (128, 18)}

# metadata value types: struct code and size of the scalar ones
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
           11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9


class GgufError(ValueError):
    pass


class Tensor:
    def __init__(self, name: str, dims: list[int], ty: int, begin: int, end: int):
        self.name, self.dims, self.ty, self.begin, self.end = name, dims, ty, begin, end

    def __repr__(self):
        return f"Tensor({self.name!r}, dims={self.dims}, ty={self.ty})"


class _Reader:
    def __init__(self, buf):
        self.b, self.at = buf, 0

    def take(self, n: int) -> bytes:
        if self.at + n > len(self.b):
            raise GgufError("truncated GGUF header")
        out = self.b[self.at:self.at + n]
        self.at += n
        return bytes(out)

    def scalar(self, code: str):
        return struct.unpack(code, self.take(struct.calcsize(code)))[0]

    def string(self) -> str:
        return self.take(self.scalar("<Q")).decode("utf-8")

    def value(self, ty: int):
        if ty in _SCALAR:
            return self.scalar(_SCALAR[ty])
        if ty == _STRING:
            return self.string()
        if ty == _ARRAY:
            ety, count = self.scalar("<I"), self.scalar("<Q")
            return [self.value(ety) for _ in range(count)]
        raise GgufError(f"unknown GGUF value type {ty}")


class Gguf:
    """A GGUF file: ``meta`` (key -> value) and ``tensors`` (name -> Tensor)."""

    def __init__(self, path: str):
        with open(path, "rb") as f:
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self._data = np.frombuffer(self._map, dtype=np.uint8)
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    def _parse(self) -> None:
        r = _Reader(self._map)
        if r.take(4) != b"GGUF":
            raise GgufError("not a GGUF file")
        version = r.scalar("<I")
        if version != 3:
            raise GgufError(f"GGUF version {version}, expected 3")
        n_tensors, n_kv = r.scalar("<Q"), r.scalar("<Q")
        self.meta = {}
        for _ in range(n_kv):
            key = r.string()
            self.meta[key] = r.value(r.scalar("<I"))
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            dims = [r.scalar("<Q") for _ in range(r.scalar("<I"))]
            infos.append((name, dims, r.scalar("<I"), r.scalar("<Q")))
        align = self.meta.get("general.alignment", 32)
        if not isinstance(align, int) or isinstance(align, bool) or align <= 0:
            raise GgufError("bad alignment")
        start = -(-r.at // align) * align
        self.tensors = {}
        for name, dims, ty, offset in infos:
            if ty not in _BLOCK:
                raise GgufError(f"{name}: unsupported ggml type {ty}")
            per, nbytes = _BLOCK[ty]
            elems = int(np.prod(dims, dtype=np.int64)) if dims else 1
            if elems % per:
                raise GgufError(f"{name}: {elems} values is not whole blocks")
            begin = start + offset
            end = begin + elems // per * nbytes
            if end > len(self._data):
                raise GgufError(f"{name}: data past the end of the file")
            self.tensors[name] = Tensor(name, dims, ty, begin, end)

    def tensor(self, name: str) -> tuple[Tensor, np.ndarray]:
        t = self.tensors.get(name)
        if t is None:
            raise GgufError(f"no tensor {name}")
        return t, self._data[t.begin:t.end]

    def close(self) -> None:
        """Unmaps the file, or leaves that to the last tensor view still held."""
        self._data = None
        try:
            self._map.close()
        except BufferError:
            pass


def _matrix(g: Gguf, name: str, ty: int, type_name: str):
    t, raw = g.tensor(name)
    if t.ty != ty or len(t.dims) != 2:
        raise GgufError(f"{name}: expected a 2-D {type_name} tensor")
    k, n = t.dims
    return raw.reshape(n, k // _BLOCK[ty][0], 18), n, k


def q4_0_arrays(blocks: np.ndarray, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """``Q4_0`` blocks of an N x K ``OutIn`` tensor (N rows of K/32 blocks) ->
    (quants, scales), the input arrays of ``Q4Weights(quants, scales, n, k)``."""
    b = np.asarray(blocks, np.uint8).reshape(n, k // 32, 18)
    scales = np.ascontiguousarray(b[:, :, 0:2]).view("<u2").reshape(n * (k // 32)).astype(np.uint16)
    qs = b[:, :, 2:18]
    u = np.concatenate([qs & 0x0F, qs >> 4], axis=2).reshape(n, k)  # values 0..31 of each block
    code = (u.astype(np.int16) - 8).astype(np.uint8) & 0x0F          # two's-complement nibble
    nib = np.ascontiguousarray(code.T).reshape(-1)                   # K x N row-major
    if nib.size % 2:
        nib = np.append(nib, np.uint8(0))
    quants = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    return quants, scales


def q1_0_arrays(blocks: np.ndarray, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """``Q1_0`` blocks of an N x K ``OutIn`` tensor -> (signs, scales), the input
    arrays of ``Q1Weights(signs, scales, WeightLayout.OutIn, n, k, 128)``."""
    b = np.asarray(blocks, np.uint8).reshape(n * (k // 128), 18)
    scales = np.ascontiguousarray(b[:, 0:2]).view("<u2").reshape(-1).astype(np.uint16)
    signs = np.ascontiguousarray(b[:, 2:18]).reshape(-1)
    return signs, scales


def load_q4_0(g: Gguf, names, smg=None):
    """The named ``Q4_0`` tensors' rows stacked (rows in order) as one
    ``Q4Weights`` handle (block 32, scale form)."""
    smg = smg or _smegemm()
    names = [names] if isinstance(names, str) else list(names)
    parts, k = [], None
    for name in names:
        b, n, kk = _matrix(g, name, Q4_0, "Q4_0")
        if k is None:
            k = kk
        elif kk != k:
            raise GgufError(f"{name}: input width differs")
        parts.append(b)
    if not parts:
        raise GgufError("no tensors named")
    rows = np.concatenate(parts, axis=0)
    quants, scales = q4_0_arrays(rows, rows.shape[0], k)
    return smg.Q4Weights(quants, scales, rows.shape[0], k)


def load_q1_0(g: Gguf, names, smg=None):
    """examples/bonsai/model.rs:132-160: the named ``Q1_0`` tensors' rows
    stacked (``OutIn``, rows in order) as one ``Q1Weights`` handle, block 128."""
    smg = smg or _smegemm()
    names = [names] if isinstance(names, str) else list(names)
    parts, k, n = [], None, 0
    for name in names:
        b, nn, kk = _matrix(g, name, Q1_0, "Q1_0")
        if k is None:
            k = kk
        elif kk != k:
            raise GgufError(f"{name}: input width differs")
        parts.append(b)
        n += nn
    if not parts:
        raise GgufError("no tensors named")
    signs, scales = q1_0_arrays(np.concatenate(parts, axis=0), n, k)
    return smg.Q1Weights(signs, scales, smg.WeightLayout.OutIn, n, k, 128)


def _smegemm():
    import smegemm
    return smegemm
