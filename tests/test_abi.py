"""The C ABI on any host: the library loads, exports every function
include/smegemm_gpu.h declares, keeps the reference's EpNode layout, and the
host-side mirror validates arguments as the Rust API panics. No GPU calls."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "smegemm_gpu.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b((?:smg|gemm_gpu)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    import smegemm
    path = os.path.join(ROOT, "sme-gemm_amd", "libsmegemm_gpu.so")
    if not os.path.exists(path):
        smegemm.build()
    return C.CDLL(path)


def test_header_declares_the_drop_ins():
    names = _declared_functions()
    for must in ("gemm_gpu_f16f16_q4", "gemm_gpu_b16b16_q4", "gemm_gpu_f16_q2", "gemm_gpu_f16_q1",
                 "gemm_gpu_f16f16_q2", "gemm_gpu_f16f16_q1", "gemm_gpu_f16f16_run_packed",
                 "gemm_gpu_b16b16_run_packed", "gemm_gpu_f16f16_q4_single", "gemm_gpu_f16f16_q4_chained",
                 "smg_q4_create",
                 "smg_q4_create_band", "smg_q2_create", "smg_q1_create", "smg_f16_prepack"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_epnode_layout_matches_reference():
    """csrc/epilogue.h:224-229: 32 bytes, op@0 aux@4 scalar@8 ptr@16 ld@24."""
    import smegemm
    E = smegemm.EpNode
    assert C.sizeof(E) == 32
    assert (E.op.offset, E.aux.offset, E.scalar.offset, E.ptr.offset, E.ld.offset) == \
        (0, 4, 8, 16, 24)


def test_enum_values_match_reference():
    """ep_op / ep_act numbering (csrc/epilogue.h:136-199)."""
    import smegemm
    text = open(HEADER).read()
    for name, val in smegemm.EP_OP.items():
        if name == "act":
            continue
        assert re.search(rf"EP_OP_{name.upper()} = {val}\b", text), name
    for name, val in smegemm.EP_ACT.items():
        assert re.search(rf"EP_ACT_{name.upper()} = {val}\b", text), name


def test_q4_gemv_single_cut(lib):
    lib.gemm_gpu_f16f16_q4_single.argtypes = [C.c_size_t] * 3
    assert lib.gemm_gpu_f16f16_q4_single(1, 4096, 4096) == 1
    assert lib.gemm_gpu_f16f16_q4_single(8, 4096, 4096) == 1
    assert lib.gemm_gpu_f16f16_q4_single(9, 4096, 4096) == 0


def test_chained_link_refuses_a_null_handle_without_raising_done(lib):
    """A failed chained call returns non-zero and leaves `done` where it was
    (src/kernels/q4/matmul.rs:105-115: `false` with nothing done); checked
    before any device work, so it runs without a GPU."""
    P = C.c_void_p
    lib.gemm_gpu_f16f16_q4_chained.argtypes = [C.c_size_t, P, P, P, P, P, P]
    lib.smg_q4_chained_dev.argtypes = [C.c_size_t, P, P, P, P, P, P, P, C.c_uint, P]
    done, ready = C.c_size_t(7), C.c_size_t(0)
    c = np.zeros(4, np.uint16)
    a = np.zeros(4, np.uint16)
    rc = lib.gemm_gpu_f16f16_q4_chained(1, None, c.ctypes.data, a.ctypes.data, None,
                                        C.addressof(done), C.addressof(ready))
    assert rc != 0 and done.value == 7
    assert lib.smg_q4_chained_dev(1, None, None, None, None, None, None, None, 0, None) != 0


def test_params_validation_mirrors_reference_panics():
    import smegemm as smg
    with pytest.raises(ValueError):
        smg.Q4Params(24)  # q4/mod.rs:76-79
    with pytest.raises(ValueError):
        smg.Q2Params(8)   # lowbit/mod.rs:65-68
    with pytest.raises(ValueError):
        smg.Q2Params(1 << 17)
    assert smg.Q2Params().block() == 256 and smg.Q2Params().codebook() == (-1, 0, 1, 0)
    assert smg.Q4Params().block() == 32 and not smg.Q4Params().is_affine()
    assert smg.Q4Params(64).affine().is_affine()


def test_epilogue_resolve_nodes():
    """resolve_nodes (src/exec/scalar.rs:28-53): tensor ld 0 -> n and the
    trailing activation appended last with alpha 0."""
    import smegemm as smg
    col = np.zeros(10, np.uint16)
    ten = np.zeros(30, np.uint16)
    ep = smg.Epilogue().add_col(col).silu().add_tensor(ten).leaky_relu(0.5).mul_scalar(2.0)
    d, keep = ep.desc(10)
    nodes = [d.nodes[i] for i in range(d.n_nodes)]
    assert [nd.op for nd in nodes] == [4, 6, 8, 1, 8]
    assert nodes[1].ld == 10
    assert (nodes[2].aux, nodes[2].scalar) == (6, 0.5)
    assert nodes[3].scalar == 2.0
    assert (nodes[4].aux, nodes[4].scalar) == (3, 0.0)
    assert smg.Epilogue().desc(10)[0] is None


def test_epilogue_validate_lengths():
    """validate_ep (src/exec/guard.rs:112-147)."""
    import smegemm as smg
    with pytest.raises(ValueError):
        smg.Epilogue().add_col(np.zeros(5, np.uint16)).validate(3, 6)
    with pytest.raises(ValueError):
        smg.Epilogue().add_row(np.zeros(5, np.uint16)).validate(3, 6)
    with pytest.raises(ValueError):
        smg.Epilogue().add_tensor(np.zeros(17, np.uint16)).validate(3, 6)
    smg.Epilogue().add_tensor(np.zeros(20, np.uint16), 7).validate(3, 6)
    with pytest.raises(ValueError):
        smg.Epilogue().add_tensor(np.zeros(40, np.uint16), 5).validate(3, 6)


def test_c_boundary_refuses_operand_nodes_without_a_pointer(lib):
    """A ROW / COL / TENSOR node with a NULL operand (which a kernel would read
    at address 0) or a tensor stride below n is refused with SMG_EINVAL at the
    C boundary, before any device work; scalar and activation nodes need no
    pointer."""
    import smegemm as smg
    lib.smg_ep_check.argtypes = [C.c_void_p, C.c_size_t]
    lib.smg_last_error.restype = C.c_char_p
    buf = np.zeros(64, np.uint16)

    def check(nodes, n=8):
        arr = (smg.EpNode * len(nodes))(*nodes)
        d = smg.EpDesc16(len(nodes), C.cast(arr, C.POINTER(smg.EpNode)))
        return lib.smg_ep_check(C.addressof(d), n)

    for op in (2, 4, 6, 12, 13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 24, 3, 5, 7):
        assert check([smg.EpNode(op, 0, 0.0, None, 0)]) == -1, op
        assert b"null operand" in lib.smg_last_error()
        assert check([smg.EpNode(op, 0, 0.0, buf.ctypes.data, 0)]) == 0, op
    assert check([smg.EpNode(6, 0, 0.0, buf.ctypes.data, 7)]) == -1  # ld 7 < n 8
    assert check([smg.EpNode(6, 0, 0.0, buf.ctypes.data, 9)]) == 0
    assert check([smg.EpNode(0, 0, 1.0, None, 0), smg.EpNode(8, 3, 0.0, None, 0)]) == 0
    assert check([smg.EpNode(25, 0, 0.0, None, 0)]) == -1       # unknown op
    assert check([smg.EpNode(8, 25, 0.0, None, 0)]) == -1       # unknown activation
    # past the store's 16 nodes a graph runs as a pass over C, up to 64 nodes,
    # each node checked alike
    assert check([smg.EpNode(0, 0, 1.0, None, 0)] * 17) == 0
    assert check([smg.EpNode(0, 0, 1.0, None, 0)] * 64) == 0
    assert check([smg.EpNode(0, 0, 1.0, None, 0)] * 65) == -1   # too many nodes
    assert check([smg.EpNode(0, 0, 1.0, None, 0)] * 40 + [smg.EpNode(4, 0, 0.0, None, 0)]) == -1
    assert b"null operand" in lib.smg_last_error()
    assert check([smg.EpNode(0, 0, 1.0, None, 0)] * 30 + [smg.EpNode(6, 0, 0.0, buf.ctypes.data, 7)]) == -1
    assert lib.smg_ep_check(None, 8) == 0                       # no epilogue
    d = smg.EpDesc16(1, None)
    assert lib.smg_ep_check(C.addressof(d), 8) == -1            # n_nodes without nodes


def test_host_operands_must_be_16_bit_patterns():
    """A host operand of another dtype is refused, not cast by value (a float32
    bias cast to uint16 would hold the wrong bits)."""
    import smegemm as smg
    with pytest.raises(TypeError):
        smg.Epilogue().add_col(np.linspace(-1, 1, 6, dtype=np.float32)).desc(6)
    with pytest.raises(TypeError):
        smg.Epilogue().add_col(np.zeros(6, np.int32)).validate(1, 6)
    with pytest.raises(TypeError):  # f16 values into a bf16 graph
        smg.Epilogue(bf16=True).add_col(np.zeros(6, np.float16)).desc(6)
    d, keep = smg.Epilogue().add_col(np.full(6, 0.5, np.float16)).desc(6)
    assert np.frombuffer((C.c_uint16 * 6).from_address(d.nodes[0].ptr), np.uint16)[0] == 0x3800


def test_band_constructors_check_lengths_before_reading():
    """from_band reads exactly the band-size formulas' lengths from the host
    arrays (q4/weights.rs:89-113, q2.rs:148-161, q1.rs:186-201); shorter (or
    longer) arrays are refused before the library is asked to read them."""
    import smegemm as smg
    n, k = 200, 96
    nib, sc = smg.q4_band_sizes(n, k, 32)
    assert (nib, sc) == (2 * 96 * 64, 2 * 3 * 128)
    with pytest.raises(ValueError):
        smg.Q4Weights.from_band(np.zeros(nib - 1, np.uint8), np.zeros(sc, np.uint16), None, n, k,
                                smg.Q4Params())
    with pytest.raises(ValueError):
        smg.Q4Weights.from_band(np.zeros(nib, np.uint8), np.zeros(sc - 1, np.uint16), None, n, k,
                                smg.Q4Params())
    with pytest.raises(ValueError):
        smg.Q4Weights.from_band(np.zeros(nib, np.uint8), np.zeros(sc, np.uint16),
                                np.zeros(sc - 2, np.uint16), n, k, smg.Q4Params().affine())
    c2, s2 = smg.lowbit_band_sizes(2, n, k, 32)
    assert (c2, s2) == (4 * 96 * 16, 4 * 3 * 64)
    with pytest.raises(ValueError):
        smg.Q2Weights.from_band(np.zeros(c2 - 16, np.uint8), np.zeros(s2, np.uint16), n, k,
                                smg.Q2Params(32))
    c1, s1 = smg.lowbit_band_sizes(1, n, 100, 32)
    assert (c1, s1) == (4 * 112 * 8, 4 * 4 * 64)
    with pytest.raises(ValueError):
        smg.Q1Weights.from_band(np.zeros(c1, np.uint8), np.zeros(s1 - 64, np.uint16), n, 100, 32)


def test_band_sizes_match_the_oracle():
    import oracle
    import smegemm as smg
    for n, k, block in ((1, 1, 16), (200, 96, 32), (129, 4097, 64), (64, 16, 16)):
        assert smg.q4_band_sizes(n, k, block) == oracle.q4_band_sizes(n, k, block)
        for kind in (1, 2):
            assert smg.lowbit_band_sizes(kind, n, k, block) == oracle.lowbit_band_sizes(kind, n, k, block)


def test_q2_codebook_is_four_int8_values():
    """Q2Params::with_codebook takes an [i8; 4] (src/kernels/lowbit/mod.rs:74-81)."""
    import smegemm as smg
    assert smg.Q2Params().with_codebook([-2, -1, 1, 2]).codebook() == (-2, -1, 1, 2)
    for bad in ([-1, 0, 1], [-1, 0, 1, 0, 2], [0, 0, 0, 128], [-129, 0, 0, 0]):
        with pytest.raises(ValueError):
            smg.Q2Params().with_codebook(bad)


def test_scalar_operands_round_through_the_element_type():
    """Scalars are stored as T::ep_to_f32 (graph.rs:86-96)."""
    import smegemm as smg
    e = smg.Epilogue().add_scalar(0.1)
    assert e.nodes[0][2] == float(np.float16(0.1))
    e = smg.Epilogue(bf16=True).add_scalar(0.1)
    assert e.nodes[0][2] == float(np.float32(0.10009765625))


def test_alpha_beta_and_scalars_are_values_not_bits():
    """alpha, beta and scalar operands are values of T (`alpha: T` in
    src/kernels/f16.rs:126, `Gemm::beta(v: T)`, `EpOp::*Scalar(T)`): the
    Python ints 0 and 1 mean 0.0 and 1.0, as the floats do; only an np.uint16
    is taken as raw bits."""
    import smegemm as smg
    for bf16, one in ((False, 0x3C00), (True, 0x3F80)):
        assert smg._bits16(1, bf16) == smg._bits16(1.0, bf16) == one
        assert smg._bits16(0, bf16) == smg._bits16(0.0, bf16) == 0
        assert smg._bits16(2, bf16) == smg._bits16(2.0, bf16)
        assert smg._bits16(np.uint16(one), bf16) == one
        assert smg._scalar_to_f32(1, bf16) == smg._scalar_to_f32(1.0, bf16) == 1.0
        assert smg._scalar_to_f32(np.uint16(one), bf16) == 1.0
        with pytest.raises(TypeError):
            smg._bits16("1", bf16)
        with pytest.raises(TypeError):
            smg._bits16(True, bf16)
    assert smg.Epilogue().add_scalar(3).nodes[0][2] == 3.0
    assert smg.Epilogue().mul_scalar(np.uint16(0x4000)).nodes[0][2] == 2.0


def test_strided_gemm_host_operands_must_be_16_bit(monkeypatch):
    """The host strided GEMM takes uint16 bits (or float16 values for f16);
    a float32 A or B is refused, not viewed as twice as many halves, and an
    f16 C is refused for a bf16 GEMM. The checks run before any library
    call (the device check is stubbed so no call can reach a GPU)."""
    import smegemm as smg
    monkeypatch.setattr(smg, "_require_device", lambda: (_ for _ in ()).throw(AssertionError("reached")))
    m = n = k = 2
    c16, a16, b16 = np.zeros(4, np.float16), np.zeros(4, np.float16), np.zeros(4, np.float16)
    for bad_a, bad_b in ((np.zeros(4, np.float32), b16), (a16, np.zeros(4, np.float32)),
                         (np.zeros(4, np.float64), b16), (a16, np.zeros(4, np.int32))):
        with pytest.raises(TypeError):
            smg.gemm_f16(m, n, k, c16, n, 1, bad_a, k, 1, bad_b, n, 1, 0.0, 1.0)
    with pytest.raises(TypeError):  # f16 C for a bf16 GEMM
        smg.gemm_bf16(m, n, k, c16, n, 1, np.zeros(4, np.uint16), k, 1, np.zeros(4, np.uint16), n, 1, 0.0, 1.0)
    with pytest.raises(TypeError):  # f16 A for a bf16 GEMM
        smg.gemm_bf16(m, n, k, np.zeros(4, np.uint16), n, 1, a16, k, 1, np.zeros(4, np.uint16), n, 1, 0.0, 1.0)
    with pytest.raises(AssertionError, match="reached"):  # well-typed operands pass every check
        smg.gemm_f16(m, n, k, c16, n, 1, a16, k, 1, np.zeros(4, np.uint16), n, 1, 0, 1)


def test_strided_gemm_refuses_bad_views(lib):
    """gemm_gpu_*_run check strides before touching a device: C's cells must
    be distinct (a zero or overlapping stride would race), no stride is
    negative (SMG_EINVAL, -1); an empty output returns at once. The mirror raises ValueError
    for a view past its slice, as check_strided panics (guard.rs:49-60)."""
    import smegemm as smg
    SZ = C.c_size_t
    for name in ("gemm_gpu_f16f16_run", "gemm_gpu_f16f32_run", "gemm_gpu_b16b16_run", "gemm_gpu_bf16f32_run"):
        fn = getattr(lib, name)
        fn.argtypes = [SZ, SZ, SZ, C.c_void_p, C.c_long, C.c_long, C.c_int, C.c_void_p, C.c_long, C.c_long,
                       C.c_void_p, C.c_long, C.c_long, C.c_uint16, C.c_uint16]
        buf = np.zeros(64, np.uint16)
        p = buf.ctypes.data
        assert fn(0, 4, 4, p, 1, 4, 0, p, 1, 4, p, 1, 4, 0, 0x3C00) == 0
        # C rows overlapping (row stride 2 for 4 columns), a zero column stride, a negative stride
        for dcs, drs in ((1, 2), (0, 4), (-1, 4)):
            assert fn(3, 4, 2, p, dcs, drs, 0, p, 1, 2, p, 1, 4, 0, 0x3C00) == -1, (name, dcs, drs)
        assert fn(3, 4, 2, p, 1, 4, 0, p, -1, 2, p, 1, 4, 0, 0x3C00) == -1  # SMG_EINVAL
    with pytest.raises(ValueError, match="overflows"):
        smg.gemm_f16(3, 4, 2, np.zeros(12, np.uint16), 4, 1, np.zeros(5, np.uint16), 2, 1,
                     np.zeros(8, np.uint16), 4, 1, 0.0, 1.0)


def test_host_slice_forms_check_before_any_device_call(lib):
    """The host-slice model entries refuse null handles and bad shapes, and
    return at once for empty work, before touching a device (SMG_EINVAL, -1)."""
    SZ, P = C.c_size_t, C.c_void_p
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    lib.smg_q4_accumulate.argtypes = [SZ, P, P, P]
    lib.smg_block_accumulate.argtypes = [P, P, P, SZ]
    lib.smg_attn_accumulate.argtypes = [P, P, P, P, SZ]
    lib.smg_mlp_accumulate.argtypes = [P, P, P, SZ]
    lib.smg_kv_cache_read.argtypes = [P, P, P]
    lib.smg_kv_cache_extend.argtypes = [P, P, P, SZ]
    lib.smg_attention_kv_f16.argtypes = [P, P, P, SZ, SZ, SZ, SZ, C.c_float, P]
    lib.smg_rms_norm_f16.argtypes = [P, P, SZ, SZ, C.c_float, P]
    assert lib.smg_q4_accumulate(1, None, p, p) == -1
    assert lib.smg_block_accumulate(None, p, None, 1) == -1
    assert lib.smg_attn_accumulate(None, p, None, p, 1) == -1
    assert lib.smg_mlp_accumulate(None, p, p, 1) == -1
    assert lib.smg_kv_cache_read(None, p, p) == -1
    assert lib.smg_kv_cache_extend(None, p, p, 1) == -1
    assert lib.smg_attention_kv_f16(p, p, p, 4, 3, 2, 64, 1.0, p) == -1   # heads not a multiple of kv_heads
    assert lib.smg_attention_kv_f16(p, p, p, 4, 2, 2, 12, 1.0, p) == -1   # head_dim not a multiple of 8
    assert lib.smg_rms_norm_f16(p, p, 2, 0, 1e-5, p) == -1
    assert lib.smg_rms_norm_f16(p, p, 0, 8, 1e-5, p) == 0                 # no rows: nothing to do


def test_host_slice_arrays_in_the_mirror():
    """The mirror's host-array rules: f32 inputs round to f16 to nearest even
    (ModelFloat::as_f16, src/linear.rs:61-66), outputs written in place must
    be contiguous, writable and of the output's type, and host arrays and
    device tensors do not mix in one call."""
    import smegemm as smg
    x = np.array([1.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65520.0, -0.0], np.float32)
    got = smg._host_x16(x, 5, "x")
    assert got.dtype == np.uint16
    assert list(got) == [0x3C00, 0x3C00, 0x3C02, 0x7C00, 0x8000]
    with np.errstate(over="ignore"):
        x16 = x.astype(np.float16)
    assert np.array_equal(smg._host_x16(x16, 5, "x"), got)
    with pytest.raises(TypeError):
        smg._host_x16(np.zeros(5, np.float64), 5, "x")
    with pytest.raises(ValueError, match="elements"):
        smg._host_x16(x, 4, "x")
    y = np.zeros(8, np.float32)
    assert smg._host_out(y, 8, (np.float32,), "y") is y
    with pytest.raises(TypeError):
        smg._host_out(np.zeros(8, np.float64), 8, (np.float32,), "y")
    with pytest.raises(TypeError):
        smg._host_out([0.0] * 8, 8, (np.float32,), "y")
    with pytest.raises(ValueError, match="contiguous"):
        smg._host_out(np.zeros(16, np.float32)[::2], 8, (np.float32,), "y")
    ro = np.zeros(8, np.float32)
    ro.flags.writeable = False
    with pytest.raises(ValueError, match="writable"):
        smg._host_out(ro, 8, (np.float32,), "y")
    with pytest.raises(ValueError, match="elements"):
        smg._host_out(y, 9, (np.float32,), "y")

    class FakeDev:
        is_cuda = True
    assert smg._same_side(y, None, y) is False
    assert smg._same_side(FakeDev(), FakeDev()) is True
    with pytest.raises(ValueError, match="host arrays or all device tensors"):
        smg._same_side(y, FakeDev())
