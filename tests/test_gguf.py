"""GGUF import (sme-gemm_amd/smegemm_gguf.py): the reader against files written here
by an independent writer, and the Q4_0 / Q1_0 block conversions against the
ggml block formulas (value i of a Q4_0 block is d*(u-8) with u the low nibble
of byte i for i < 16 and the high nibble of byte i-16 after; a Q1_0 block is
128 sign bits, bit i of byte i/8 set for +d) and the reference's input-array
rules (src/kernels/q4/mod.rs:206-214; src/kernels/lowbit/q1.rs:35-41).

The GPU tests run imported weights through the kernels and compare with the
CPU oracle, on the same arrays and, for Q4_0, with an f64 product of the ggml
values rounded per weight to f16.
"""
import struct

import numpy as np
import pytest

from conftest import f16_tol, max_rel

GGUF_TYPES = {"u8": (0, "<B"), "i8": (1, "<b"), "u16": (2, "<H"), "i16": (3, "<h"), "u32": (4, "<I"),
              "i32": (5, "<i"), "f32": (6, "<f"), "bool": (7, "<?"), "u64": (10, "<Q"),
              "i64": (11, "<q"), "f64": (12, "<d")}


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind, v) -> bytes:
    if kind == "str":
        return struct.pack("<I", 8) + _s(v)
    if isinstance(kind, tuple):  # ("arr", element kind)
        ek = kind[1]
        et = 8 if ek == "str" else GGUF_TYPES[ek][0]
        body = b"".join(_s(x) if ek == "str" else struct.pack(GGUF_TYPES[ek][1], x) for x in v)
        return struct.pack("<I", 9) + struct.pack("<IQ", et, len(v)) + body
    t, code = GGUF_TYPES[kind]
    return struct.pack("<I", t) + struct.pack(code, v)


def write_gguf(path, meta, tensors, align=32, version=3, magic=b"GGUF"):
    """meta: [(key, kind, value)]; tensors: [(name, dims, ggml type, raw bytes)]."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, kind, v in meta:
        head += _s(key) + _value(kind, v)
    off, datas = 0, []
    for name, dims, ty, raw in tensors:
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, off)
        datas.append((off, raw))
        off = -(-(off + len(raw)) // align) * align
    start = -(-len(head) // align) * align
    out = bytearray(head + b"\0" * (start - len(head)))
    for o, raw in datas:
        need = start + o
        out += b"\0" * (need - len(out))
        out += raw
    with open(path, "wb") as f:
        f.write(bytes(out))


def q4_0_blocks(rng, n, k):
    """Random Q4_0 rows: f16 scales in [0.002, 0.05), random code bytes."""
    d = rng.uniform(0.002, 0.05, (n, k // 32)).astype(np.float16).view(np.uint16)
    qs = rng.integers(0, 256, (n, k // 32, 16), dtype=np.uint8)
    b = np.concatenate([d.reshape(n, k // 32, 1).view(np.uint8), qs], axis=2)
    return np.ascontiguousarray(b).reshape(-1)


def ggml_q4_0_values(blocks, n, k):
    """value[j][i] of the N x K tensor as (d as f64, integer code) per ggml."""
    b = blocks.reshape(n, k // 32, 18)
    d = b[..., 0].astype(np.uint16) | (b[..., 1].astype(np.uint16) << 8)
    code = np.empty((n, k // 32, 32), np.int64)
    for i in range(16):
        code[..., i] = (b[..., 2 + i] & 0x0F).astype(np.int64) - 8
        code[..., 16 + i] = (b[..., 2 + i] >> 4).astype(np.int64) - 8
    dd = d.view(np.float16).astype(np.float64)
    return np.repeat(dd, 32, axis=1).reshape(n, k), code.reshape(n, k)


def decode_q4_input(quants, scales, n, k):
    """The reference's reading of Q4Weights::new's arrays (mod.rs:206-214):
    weight (d, j) is nibble idx%2 of byte idx/2, idx = d*n + j, two's complement;
    its scale scales[j*nbk + d/32]."""
    idx = np.arange(k * n)
    nib = (quants[idx // 2] >> (4 * (idx % 2))) & 0x0F
    code = np.where(nib < 8, nib.astype(np.int64), nib.astype(np.int64) - 16).reshape(k, n).T
    nbk = -(-k // 32)
    sc = scales.view(np.float16).astype(np.float64).reshape(n, nbk)
    return np.repeat(sc, 32, axis=1)[:, :k], code


@pytest.fixture
def gg():
    import smegemm_gguf
    return smegemm_gguf


def test_reader_metadata_and_tensors(tmp_path, gg):
    meta = [("general.name", "str", "tiny"), ("a.u8", "u8", 200), ("a.i8", "i8", -5),
            ("a.u16", "u16", 60000), ("a.i16", "i16", -3000), ("a.u32", "u32", 4_000_000_000),
            ("a.i32", "i32", -7), ("a.f32", "f32", 0.5), ("a.bool", "bool", True),
            ("a.u64", "u64", 1 << 40), ("a.i64", "i64", -(1 << 40)), ("a.f64", "f64", 1e-300),
            ("tok.tokens", ("arr", "str"), ["a", "bb", "ccc"]), ("a.ints", ("arr", "i32"), [1, -2, 3])]
    f32 = np.arange(6, dtype=np.float32).tobytes()
    rng = np.random.default_rng(1)
    q4 = q4_0_blocks(rng, 3, 64).tobytes()
    path = tmp_path / "t.gguf"
    write_gguf(path, meta, [("w.f32", [3, 2], 0, f32), ("w.q4", [64, 3], 2, q4)])
    g = gg.Gguf(str(path))
    for key, kind, v in meta:
        got = g.meta[key]
        assert (got == pytest.approx(v) if kind == "f32" else got == v), key
    t, raw = g.tensor("w.f32")
    assert t.dims == [3, 2] and t.ty == 0 and raw.tobytes() == f32
    t, raw = g.tensor("w.q4")
    assert t.dims == [64, 3] and t.ty == 2 and raw.tobytes() == q4
    g.close()


def test_reader_alignment_key(tmp_path, gg):
    raw = bytes(range(18)) * 2
    path = tmp_path / "a.gguf"
    write_gguf(path, [("general.alignment", "u32", 64)], [("x", [32, 2], 2, raw), ("y", [32, 2], 2, raw)],
               align=64)
    g = gg.Gguf(str(path))
    assert g.tensor("y")[1].tobytes() == raw
    assert g.tensors["y"].begin % 64 == 0


@pytest.mark.parametrize("case,msg", [("magic", "not a GGUF"), ("version", "version 2"),
                                      ("type", "unsupported ggml type 8"), ("blocks", "not whole blocks"),
                                      ("short", "past the end"), ("truncated", "truncated")])
def test_reader_errors(tmp_path, gg, case, msg):
    """gguf.rs:110-170's error cases."""
    path = tmp_path / "e.gguf"
    raw = bytes(18)
    if case == "magic":
        write_gguf(path, [], [], magic=b"GGML")
    elif case == "version":
        write_gguf(path, [], [], version=2)
    elif case == "type":
        write_gguf(path, [], [("x", [32], 8, bytes(34))])
    elif case == "blocks":
        write_gguf(path, [], [("x", [33], 2, raw * 2)])
    elif case == "short":
        write_gguf(path, [], [("x", [64], 2, raw)])
    else:
        write_gguf(path, [("k", "str", "value")], [])
        path.write_bytes(path.read_bytes()[:30])
    with pytest.raises(gg.GgufError, match=msg):
        gg.Gguf(str(path))


def test_q4_0_known_block(gg):
    """One block by hand: d = 1.0, byte i = i | (15 - i) << 4, so value i is
    i - 8 and value 16 + i is 7 - i."""
    blk = np.array([0x00, 0x3C] + [i | ((15 - i) << 4) for i in range(16)], np.uint8)
    quants, scales = gg.q4_0_arrays(blk, 1, 32)
    sc, code = decode_q4_input(quants, scales, 1, 32)
    assert scales.tolist() == [0x3C00]
    assert code[0].tolist() == [i - 8 for i in range(16)] + [7 - i for i in range(16)]


@pytest.mark.parametrize("n,k", [(1, 32), (3, 64), (7, 96), (64, 256)])
def test_q4_0_conversion_keeps_every_value(gg, n, k):
    """Every weight's scale and integer code survive the conversion exactly."""
    rng = np.random.default_rng(n * 100 + k)
    blocks = q4_0_blocks(rng, n, k)
    quants, scales = gg.q4_0_arrays(blocks, n, k)
    assert quants.size == -(-(k * n) // 2) and scales.size == n * (k // 32)
    d_want, c_want = ggml_q4_0_values(blocks, n, k)
    d_got, c_got = decode_q4_input(quants, scales, n, k)
    assert np.array_equal(c_got, c_want)
    assert np.array_equal(d_got, d_want)


@pytest.mark.parametrize("n,k", [(1, 128), (5, 256), (33, 512)])
def test_q1_0_conversion_keeps_every_sign(gg, n, k):
    """q1.rs:35-41 on the converted arrays (OutIn: bit idx%8 of byte idx/8,
    idx = j*k + d) gives the ggml block's bit i of byte i/8 and its scale."""
    rng = np.random.default_rng(n + k)
    d = rng.uniform(0.01, 0.1, n * k // 128).astype(np.float16).view(np.uint16)
    sb = rng.integers(0, 256, (n * k // 128, 16), dtype=np.uint8)
    blocks = np.concatenate([d.reshape(-1, 1).view(np.uint8), sb], axis=1).reshape(-1)
    signs, scales = gg.q1_0_arrays(blocks, n, k)
    assert np.array_equal(scales, d)
    idx = np.arange(n * k)
    got = (signs[idx // 8] >> (idx % 8)) & 1
    blk, i = idx // 128, idx % 128
    want = (sb[blk, i // 8] >> (i % 8)) & 1
    assert np.array_equal(got, want)


@pytest.mark.gpu
def test_imported_q4_0_matmul(tmp_path, gg, smg, orc):
    """Q4_0 tensors imported (one, and two stacked as one weight set) multiply
    as the oracle does on the converted arrays, and within the f16 bar of an
    f64 product of the ggml values, each rounded once to f16."""
    k, n1, n2 = 512, 96, 160
    rng = np.random.default_rng(7)
    b1, b2 = q4_0_blocks(rng, n1, k), q4_0_blocks(rng, n2, k)
    path = tmp_path / "q4.gguf"
    write_gguf(path, [("general.name", "str", "q4")], [("w1", [k, n1], 2, b1.tobytes()),
                                                      ("w2", [k, n2], 2, b2.tobytes())])
    g = gg.Gguf(str(path))
    for names, blocks, n in ((["w1"], b1, n1), (["w1", "w2"], np.concatenate([b1, b2]), n1 + n2)):
        w = gg.load_q4_0(g, names, smg)
        quants, scales = gg.q4_0_arrays(blocks, n, k)
        for m in (1, 40):
            a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
            c = np.zeros(m * n, np.uint16)
            smg.matmul_q4(a, w, c, m)
            assert max_rel(c, orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32)) <= f16_tol(k)
            d, code = ggml_q4_0_values(blocks, n, k)
            wt = (d * code).astype(np.float16).astype(np.float64)  # N x K
            ref = orc.f16_to_f32(a).astype(np.float64).reshape(m, k) @ wt.T
            assert max_rel(c, orc.f32_to_f16(ref.astype(np.float32))) <= f16_tol(k)


@pytest.mark.gpu
def test_imported_q1_0_matmul_bit_exact(tmp_path, gg, smg, orc):
    """Q1_0 tensors stacked as model.rs:132-160 does (q, k, v rows in order),
    then matmul_q1 on the device: bit-exact with the oracle on those arrays."""
    k, ns = 512, (64, 32, 32)
    rng = np.random.default_rng(8)
    tensors, raw_all = [], []
    for i, n in enumerate(ns):
        d = rng.uniform(0.01, 0.1, n * k // 128).astype(np.float16).view(np.uint16)
        sb = rng.integers(0, 256, (n * k // 128, 16), dtype=np.uint8)
        raw = np.concatenate([d.reshape(-1, 1).view(np.uint8), sb], axis=1).reshape(-1)
        tensors.append((f"attn_{'qkv'[i]}", [k, n], 41, raw.tobytes()))
        raw_all.append(raw)
    path = tmp_path / "q1.gguf"
    write_gguf(path, [], tensors)
    g = gg.Gguf(str(path))
    w = gg.load_q1_0(g, ["attn_q", "attn_k", "attn_v"], smg)
    n = sum(ns)
    signs, scales = gg.q1_0_arrays(np.concatenate(raw_all), n, k)
    for m in (1, 3):
        a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
        c = np.zeros(m * n, np.uint16)
        smg.matmul_q1(a, w, c, m)
        want = orc.matmul_lowbit_ep(1, a, signs, scales, m, n, k, 128)
        assert np.array_equal(c, want)
