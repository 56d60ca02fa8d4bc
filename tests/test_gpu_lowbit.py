"""2-bit / 1-bit int8 path on the GPU vs the oracle, bit for bit.

Mirrors src/kernels/lowbit/matmul.rs:457 (kernels_match_reference_bits: 12
shapes x 4 blocks x 3 codebooks, both Q1 layouts, the reference's own LCG
data), tests/correctness/q2.rs:83 (fused epilogue == plain then applied) and
the headline configs 2 and 3 (the benchmark shapes). Integer quantization and i32 block
sums are exact, so outputs must be identical bits.
"""
import numpy as np
import pytest

from conftest import f16_tol, max_rel, ulp_dist

pytestmark = pytest.mark.gpu

SHAPES = [(1, 64, 256), (1, 65, 37), (1, 1, 1), (2, 200, 300), (3, 64, 16), (5, 130, 513),
          (6, 192, 256), (7, 100, 64), (12, 70, 200), (1, 2048, 1024), (4, 1536, 512),
          (9, 1024, 384)]
BOOKS = [(-1, 0, 1, 0), (-2, -1, 1, 2), (-128, 127, 3, -7)]


def _data(orc, seed, length):
    return orc.lcg_bytes(seed, length)


@pytest.mark.parametrize("si", range(len(SHAPES)))
@pytest.mark.parametrize("bi,block", list(enumerate([16, 64, 128, 4096])))
def test_kernels_match_reference_bits(smg, orc, si, bi, block):
    """matmul.rs:457-500, with the same generators and parameters."""
    m, n, k = SHAPES[si]
    nbk = -(-k // block)
    sbytes = _data(orc, si + 7, n * nbk)
    scales = orc.f32_to_f16(sbytes.astype(np.float32) * np.float32(1e-3) - np.float32(0.1))
    abytes = _data(orc, si + 99, m * k)
    a = orc.f32_to_f16((abytes.astype(np.float32) - np.float32(128.0)) / np.float32(37.0))
    book = BOOKS[(si + bi) % len(BOOKS)]
    p = smg.Q2Params(block).with_codebook(book)
    codes = _data(orc, si * 31 + bi, (k * n + 3) // 4)
    q2 = smg.Q2Weights(codes, scales, n, k, p)
    got = np.full(m * n, 0x4880, np.uint16)  # f16 9.0, as the reference pre-fills
    smg.matmul_q2(a, q2, got, m)
    want = orc.lowbit_reference(2, a, codes, scales, m, n, k, block, book)
    assert np.array_equal(got, want), f"q2 {m}x{n}x{k} {block} {book}"
    signs = _data(orc, si * 17 + bi, (k * n + 7) // 8)
    for layout in (smg.WeightLayout.OutIn, smg.WeightLayout.InOut):
        q1 = smg.Q1Weights(signs, scales, layout, n, k, block)
        got = np.full(m * n, 0x4880, np.uint16)
        smg.matmul_q1(a, q1, got, m)
        want = orc.lowbit_reference(1, a, signs, scales, m, n, k, block,
                                    inout=(layout == smg.WeightLayout.InOut))
        assert np.array_equal(got, want), f"q1 {m}x{n}x{k} {block} layout {layout}"


@pytest.mark.parametrize("block", [32, 256, 512, 1024, 2048])
@pytest.mark.parametrize("m,n,k", [(1, 300, 9000), (3, 129, 4096), (8, 64, 5000), (2, 40, 700),
                                   (1, 20000, 512), (1, 300, 8000)])
def test_single_launch_blocks_and_segments(smg, orc, block, m, n, k):
    """The streaming path and its limits: blocks within a wave's K range and
    blocks spanning waves (amax and sum(q) combined through LDS, block sums
    through integer atomics), A quantized over several passes, more tiles per
    workgroup than the ring holds (N = 20000), the widest K ranges per lane,
    partial last blocks, and shapes past its limits (the two-kernel path)."""
    nbk = -(-k // block)
    rng = np.random.default_rng(block * 7 + m)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * nbk).astype(np.float32))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    q2 = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block))
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q2(a, q2, got, m)
    assert np.array_equal(got, orc.lowbit_reference(2, a, codes, scales, m, n, k, block, (-1, 0, 1, 0)))
    signs = rng.integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
    q1 = smg.Q1Weights(signs, scales, smg.WeightLayout.InOut, n, k, block)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q1(a, q1, got, m)
    assert np.array_equal(got, orc.lowbit_reference(1, a, signs, scales, m, n, k, block, inout=True))


@pytest.mark.parametrize("m", [1, 2, 8])
def test_config2_q2_ternary(smg, orc, m):
    """Headline config 2: K=4096, N=11008, block 128, ternary; bitwise."""
    import workloads
    n, k = 11008, 4096
    a, codes, scales = workloads.q2_inputs(m, n, k, seed=0)
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(128))
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q2(a, w, got, m)
    want = orc.lowbit_reference(2, a, codes, scales, m, n, k, 128)
    assert np.array_equal(got, want)


def test_config3_q1_add_col_silu(smg, orc):
    """Headline config 3: Q1 + add_col(bias) + silu, K=4096, N=14336; bitwise."""
    import workloads
    m, n, k = 1, 14336, 4096
    a, signs, scales, bias = workloads.q1_inputs(m, n, k, seed=0)
    w = smg.Q1Weights(signs, scales, smg.WeightLayout.OutIn, n, k, 128)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q1_ep(a, w, got, m, smg.Epilogue().add_col(bias).silu())
    want = orc.matmul_lowbit_ep(1, a, signs, scales, m, n, k, 128, [(4, 0, 0.0, bias, 0)], 3)
    assert np.array_equal(got, want)


ACT_METHODS = {1: ("relu", ()), 2: ("gelu", ()), 3: ("silu", ()), 4: ("tanh", ()), 5: ("sigmoid", ()),
               6: ("leaky_relu", (0.2,)), 7: ("relu6", ()), 8: ("hardsigmoid", ()),
               9: ("hardswish", ()), 10: ("abs", ()), 11: ("neg", ()), 12: ("square", ()),
               13: ("sign", ()), 14: ("sqrt", ()), 15: ("softsign", ()), 16: ("recip", ()),
               17: ("rsqrt", ()), 18: ("exp", ()), 19: ("log", ()), 20: ("elu", (0.7,)),
               21: ("selu", ()), 22: ("softplus", ()), 23: ("mish", ()), 24: ("gelu_exact", ())}


@pytest.mark.parametrize("kind", range(1, 25))
def test_every_activation_bitwise(smg, orc, kind):
    """Each of the 24 activation kinds on the int8 path, bit for bit with the
    oracle: the named five as the trailing act (alone after add_col, then
    after a mul_scalar node), the rest as in-order nodes, last in the graph and
    then followed by mul_scalar 2. Pre-activation
    values span -8..8 so every branch of the piecewise kinds is taken."""
    m, n, k = 2, 512, 256
    rng = np.random.default_rng(500 + kind)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * (k // 128)).astype(np.float32))
    bias = orc.f32_to_f16(rng.uniform(-8.0, 8.0, n).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(128))
    name, args = ACT_METHODS[kind]
    alpha = float(np.float32(args[0])) if args else 0.0
    for inner in (False, True):
        ep, nodes, act = smg.Epilogue().add_col(bias), [(4, 0, 0.0, bias, 0)], None
        if kind <= 5:  # a trailing act stays last (graph.rs:193-223); a node precedes it
            if inner:
                ep, nodes = ep.mul_scalar(2.0), nodes + [(1, 0, 2.0, None, 0)]
            ep, act = getattr(ep, name)(*args), kind
        else:
            ep, nodes = getattr(ep, name)(*args), nodes + [(8, kind, alpha, None, 0)]
            if inner:
                ep, nodes = ep.mul_scalar(2.0), nodes + [(1, 0, 2.0, None, 0)]
        got = np.zeros(m * n, np.uint16)
        smg.matmul_q2_ep(a, w, got, m, ep)
        want = orc.matmul_lowbit_ep(2, a, codes, scales, m, n, k, 128, nodes, act)
        # a NaN's sign and payload are the platform's (log of a negative: glibc
        # gives -NaN, the device +NaN): NaN must meet NaN, every other value its bits
        nan_g, nan_w = (got & 0x7C00 == 0x7C00) & (got & 0x3FF != 0), (want & 0x7C00 == 0x7C00) & (want & 0x3FF != 0)
        assert np.array_equal(nan_g, nan_w), f"{name} inner={inner}: NaN positions"
        assert np.array_equal(got[~nan_g], want[~nan_w]), f"{name} inner={inner}"


@pytest.mark.parametrize("act", ["silu", "sigmoid"])
def test_logistic_epilogue_bitwise_wide_range(smg, orc, act):
    """A trailing silu / sigmoid over 32768 outputs whose pre-activation values
    span -30..30 (bias added first): bit-identical to the reference's f64
    formula rounded to f32 then f16, including where the stores take their
    fast f32 path."""
    m, n, k = 8, 4096, 256
    rng = np.random.default_rng(99 + len(act))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * (k // 128)).astype(np.float32))
    bias = orc.f32_to_f16(rng.uniform(-30.0, 30.0, n).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(128))
    got = np.zeros(m * n, np.uint16)
    ep = smg.Epilogue().add_col(bias)
    ep = ep.silu() if act == "silu" else ep.sigmoid()
    smg.matmul_q2_ep(a, w, got, m, ep)
    want = orc.matmul_lowbit_ep(2, a, codes, scales, m, n, k, 128, [(4, 0, 0.0, bias, 0)],
                                3 if act == "silu" else 5)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("m,n,k", [(1, 200, 300), (4, 1536, 512), (13, 70, 64)])
def test_fused_epilogue_is_plain_then_applied(smg, orc, m, n, k):
    """q2.rs:83-108: bias, row scale and trailing gelu == plain product then the
    scalar graph (bitwise here: both sides are the reference's arithmetic)."""
    rng = np.random.default_rng(m * 131 + n * 17 + k)
    a, codes, scales = (orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32) * 0.5),
                        rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8),
                        orc.f32_to_f16(rng.uniform(0.005, 0.03, n * -(-k // 256))
                                       .astype(np.float32)))
    bias = orc.f32_to_f16(rng.uniform(-0.5, 0.5, n).astype(np.float32))
    rows = orc.f32_to_f16(rng.uniform(-0.5, 0.5, m).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k)
    plain = np.zeros(m * n, np.uint16)
    smg.matmul_q2(a, w, plain, m)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q2_ep(a, w, got, m, smg.Epilogue().add_col(bias).mul_row(rows).gelu())
    want = orc.apply_ep(plain, m, n, [(4, 0, 0.0, bias, 0), (3, 0, 0.0, rows, 0)], 2)
    assert np.array_equal(got, want)


def test_m_independence_and_row_groups(smg, orc):
    """Results depend only on the row and column (ARCHITECTURE.md:511-514):
    row i of an m=20 call (three row groups) equals the m=1 call on row i."""
    m, n, k = 20, 300, 700
    rng = np.random.default_rng(3)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * -(-k // 64)).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(64))
    full = np.zeros(m * n, np.uint16)
    smg.matmul_q2(a, w, full, m)
    for i in (0, 7, 8, 19):
        one = np.zeros(n, np.uint16)
        smg.matmul_q2(a[i * k:(i + 1) * k], w, one, 1)
        assert np.array_equal(one, full[i * n:(i + 1) * n])


@pytest.mark.parametrize("block,k,m", [(8192, 20000, 1), (65536, 70000, 2), (16384, 16384, 9)])
def test_long_blocks_prequantized(smg, orc, block, k, m):
    """Blocks longer than one in-kernel pass (quantized by the stand-alone
    kernel first), including the maximum block 65536 and a partial last block."""
    n = 96
    rng = np.random.default_rng(block + k)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    nbk = -(-k // block)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * nbk).astype(np.float32))
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block))
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q2(a, w, got, m)
    assert np.array_equal(got, orc.lowbit_reference(2, a, codes, scales, m, n, k, block))
    signs = rng.integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
    w1 = smg.Q1Weights(signs, scales, smg.WeightLayout.OutIn, n, k, block)
    got1 = np.zeros(m * n, np.uint16)
    smg.matmul_q1(a, w1, got1, m)
    assert np.array_equal(got1, orc.lowbit_reference(1, a, signs, scales, m, n, k, block))


def test_nan_and_inf_activations(smg, orc):
    """A NaN in a block makes its amax NaN (matmul.rs:356-363) and an inf gives
    inv = 0; both propagate exactly as the reference's fold does."""
    m, n, k = 2, 64, 256
    rng = np.random.default_rng(1)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    a[5] = 0x7E00      # NaN in row 0, block 0
    a[k + 200] = 0x7C00  # +inf in row 1, block 1 (block 128)
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * 2).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(128))
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q2(a, w, got, m)
    want = orc.lowbit_reference(2, a, codes, scales, m, n, k, 128)
    gnan = (got & 0x7C00) == 0x7C00
    wnan = (want & 0x7C00) == 0x7C00
    assert np.array_equal(gnan & ((got & 0x3FF) != 0), wnan & ((want & 0x3FF) != 0))
    fin = ~wnan
    assert np.array_equal(got[fin], want[fin])


def test_band_major_upload_matches_row_major(smg, orc):
    n, k, block = 130, 300, 64
    rng = np.random.default_rng(2)
    a = orc.f32_to_f16(rng.standard_normal(3 * k).astype(np.float32))
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    nbk = -(-k // block)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * nbk).astype(np.float32))
    p = smg.Q2Params(block).with_codebook((-2, -1, 1, 2))
    packed, sc = orc.lowbit_pack_band(2, codes, scales, n, k, block)
    c1 = np.zeros(3 * n, np.uint16)
    c2 = np.zeros(3 * n, np.uint16)
    smg.matmul_q2(a, smg.Q2Weights(codes, scales, n, k, p), c1, 3)
    smg.matmul_q2(a, smg.Q2Weights.from_band(packed, sc, n, k, p), c2, 3)
    assert np.array_equal(c1, c2)
    signs = rng.integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
    packed1, sc1 = orc.lowbit_pack_band(1, signs, scales, n, k, block, inout=True)
    d1 = np.zeros(3 * n, np.uint16)
    d2 = np.zeros(3 * n, np.uint16)
    smg.matmul_q1(a, smg.Q1Weights(signs, scales, smg.WeightLayout.InOut, n, k, block), d1, 3)
    smg.matmul_q1(a, smg.Q1Weights.from_band(packed1, sc1, n, k, block), d2, 3)
    assert np.array_equal(d1, d2)


MOPA_SHAPES = [(8, 64, 256), (1, 65, 37), (3, 200, 301), (33, 130, 514), (40, 4200, 1030),
               (200, 1000, 2048)]


@pytest.mark.parametrize("si", range(len(MOPA_SHAPES)))
@pytest.mark.parametrize("bi,block", list(enumerate([16, 128, 4096])))
def test_mopa_matches_eager_dequant(smg, orc, si, bi, block):
    """matmul.rs:527-567: the MOPA route against eager dequant + dense GEMM
    (f32 accumulation here and in the oracle; tolerance on the sum order)."""
    m, n, k = MOPA_SHAPES[si]
    nbk = -(-k // block)
    scales = orc.f32_to_f16(_data(orc, si + 3, n * nbk).astype(np.float32) * np.float32(1e-3)
                            - np.float32(0.1))
    a = orc.f32_to_f16((_data(orc, si + 77, m * k).astype(np.float32) - np.float32(128.0))
                       / np.float32(61.0))
    book = BOOKS[(si + bi) % len(BOOKS)]
    codes = _data(orc, si * 13 + bi, (k * n + 3) // 4)
    signs = _data(orc, si * 19 + bi, (k * n + 7) // 8)
    bias = orc.f32_to_f16(np.arange(n, dtype=np.float32) * np.float32(0.01) - np.float32(1.0))
    q2 = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block).with_codebook(book))
    q1 = smg.Q1Weights(signs, scales, smg.WeightLayout.OutIn, n, k, block)
    # plain product within tolerance of the oracle; the fused epilogue equals
    # the scalar op-graph applied to the GPU's own plain product (as q2.rs:83
    # checks it) to one f16 ulp -- the GEMM store evaluates the activation in
    # f32 -- so a 1-ulp flip of the rounded sum is not amplified by add_col
    # cancellation into a tolerance failure
    ep = smg.Epilogue().add_col(bias).silu()
    nodes, act = [(4, 0, 0.0, bias, 0)], 3
    for kind, w, codes_ in ((2, q2, codes), (1, q1, signs)):
        plain = np.zeros(m * n, np.uint16)
        fused = np.zeros(m * n, np.uint16)
        if kind == 2:
            smg.matmul_q2_mopa(a, w, plain, m)
            smg.matmul_q2_mopa_ep(a, w, fused, m, ep)
            want = orc.matmul_lowbit_mopa_ep(2, a, codes_, scales, m, n, k, block, (), None, book)
        else:
            smg.matmul_q1_mopa(a, w, plain, m)
            smg.matmul_q1_mopa_ep(a, w, fused, m, ep)
            want = orc.matmul_lowbit_mopa_ep(1, a, codes_, scales, m, n, k, block)
        assert max_rel(plain, want) <= f16_tol(k), f"q{kind} mopa plain"
        assert ulp_dist(fused, orc.apply_ep(plain, m, n, nodes, act)) <= 1, f"q{kind} mopa ep"


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("m,n,k,block", [(1, 96, 512, 64), (5, 70, 300, 64), (40, 33, 1000, 128)])
def test_quantize_then_matmul(smg, orc, layout, m, n, k, block):
    """Q2Weights::quantize / Q1Weights::quantize from f32 weights in either
    layout, uploaded and multiplied on the device: bit-exact with the reference
    path over the oracle's quantized arrays."""
    rng = np.random.default_rng(m * 7 + n + k + layout)
    w = rng.standard_normal(n * k).astype(np.float32)
    x = w if layout == 0 else np.ascontiguousarray(w.reshape(n, k).T).ravel()
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    book = (-2, -1, 1, 2)
    q2 = smg.Q2Weights.quantize(x, layout, n, k, smg.Q2Params(block).with_codebook(book))
    codes, scales = orc.q2_quantize(x, layout, n, k, block, book)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q2(a, q2, got, m)
    assert np.array_equal(got, orc.lowbit_reference(2, a, codes, scales, m, n, k, block, book))
    q1 = smg.Q1Weights.quantize(x, layout, n, k, block)
    signs, scales = orc.q1_quantize(x, layout, n, k, block)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q1(a, q1, got, m)
    assert np.array_equal(got, orc.lowbit_reference(1, a, signs, scales, m, n, k, block))


@pytest.mark.parametrize("n,k,block", [(70, 300, 64), (64, 512, 128), (33, 1000, 32), (5, 64, 16)])
def test_q1_interleave(smg, orc, n, k, block):
    """Q1Weights::interleave (q1.rs:149-185, test :279-320): 2n columns, each
    32-column chunk of gate then the same chunk of up; every column is exactly
    the source column, so outputs match the oracle over the interleaved arrays
    and the separate gate / up products, bitwise."""
    rng = np.random.default_rng(n + k)
    wg = rng.standard_normal(n * k).astype(np.float32)
    wu = -wg * np.float32(0.5) + rng.standard_normal(n * k).astype(np.float32) * np.float32(0.1)
    gate = smg.Q1Weights.quantize(wg, 0, n, k, block)
    up = smg.Q1Weights.quantize(wu, 0, n, k, block)
    both = smg.Q1Weights.interleave(gate, up)
    assert both.n() == 2 * n and both.k() == k
    order = [(src, j) for c0 in range(0, n, 32) for src in (0, 1)
             for j in range(c0, min(c0 + 32, n))]
    arrays = [orc.q1_quantize(wg, 0, n, k, block), orc.q1_quantize(wu, 0, n, k, block)]
    bits = [np.unpackbits(s, bitorder="little")[: n * k].reshape(n, k) for s, _ in arrays]
    nbk = -(-k // block)
    isig = np.packbits(np.stack([bits[s][j] for s, j in order]).ravel(), bitorder="little")
    isc = np.concatenate([arrays[s][1][j * nbk:(j + 1) * nbk] for s, j in order])
    for m in (1, 3, 9):
        a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
        got = np.zeros(m * 2 * n, np.uint16)
        smg.matmul_q1(a, both, got, m)
        assert np.array_equal(got, orc.lowbit_reference(1, a, isig, isc, m, 2 * n, k, block)), m
        g = np.zeros(m * n, np.uint16)
        u = np.zeros(m * n, np.uint16)
        smg.matmul_q1(a, gate, g, m)
        smg.matmul_q1(a, up, u, m)
        parts = [g.reshape(m, n), u.reshape(m, n)]
        want = np.stack([parts[s][:, j] for s, j in order], 1).ravel()
        assert np.array_equal(got, want), m


def test_q1_interleave_rejects_mismatch(smg):
    w = np.ones(64 * 32, np.float32)
    a = smg.Q1Weights.quantize(w, 0, 32, 64, 32)
    b = smg.Q1Weights.quantize(w, 0, 32, 64, 64)
    with pytest.raises(smg.SmeGemmError, match="same shape"):
        smg.Q1Weights.interleave(a, b)


def test_multi_row_calls_in_a_replayed_graph(smg, orc):
    """Multi-row calls (A quantized once per call into the thread's staging
    buffer, then the tile launch): three calls captured in a HIP graph after
    eager warm-up, the graph replayed three times with eager calls between
    replays, every replay bit-identical to the eager results and to the
    reference."""
    import torch
    n, k, block = 2048, 1024, 128
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * (k // block)).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block))
    to_dev = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
    cases = []
    for m in (8, 4, 2):
        a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
        want = orc.matmul_lowbit_ep(2, a, codes, scales, m, n, k, block)
        cases.append((m, to_dev(a), torch.zeros(m * n, dtype=torch.int16, device="cuda"), want))
    for m, ad, cd, want in cases:  # eager (also sizes the staging buffer before capture)
        smg.matmul_q2(ad, w, cd, m)
    torch.cuda.synchronize()
    for m, ad, cd, want in cases:
        assert np.array_equal(cd.cpu().numpy().view(np.uint16), want), f"eager m={m}"
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for m, ad, cd, want in cases:  # warm the capture stream too
            smg.matmul_q2(ad, w, cd, m)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=side):
            for m, ad, cd, want in cases:
                smg.matmul_q2(ad, w, cd, m)
    torch.cuda.synchronize()
    for rep in range(3):
        for m, ad, cd, want in cases:
            cd.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for m, ad, cd, want in cases:
            assert np.array_equal(cd.cpu().numpy().view(np.uint16), want), f"replay {rep} m={m}"
        for m, ad, cd, want in cases:  # eager work between replays
            smg.matmul_q2(ad, w, cd, m)
        torch.cuda.synchronize()


# Shapes of the persistent kernel (lowbit_row: m <= 8, blocks of 128, the
# compiled stores): 1-4 tiles a compute unit on a 256-CU device (N up to 53248
# with 64-column tiles), K short of a block, ragged, over one pass (8192), and
# grids of fewer tiles than compute units.
ROW_CASES = [(1, 16, 128), (2, 48, 640), (3, 2064, 4096), (5, 4112, 1000), (8, 12304, 4096),
             (1, 14336, 8192), (7, 20496, 384), (4, 53248, 128), (1, 53264, 256), (6, 33, 4100)]


@pytest.mark.parametrize("graph", ["none", "add_silu", "mul_add_relu"])
@pytest.mark.parametrize("case", range(len(ROW_CASES)))
@pytest.mark.parametrize("kind", [2, 1])
def test_persistent_row_kernel_shapes(smg, orc, kind, case, graph):
    """Bit for bit against the oracle's portable path, every compiled store."""
    m, n, k = ROW_CASES[case]
    rng = np.random.default_rng(1000 * kind + 10 * case + len(graph))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    nbk = -(-k // 128)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * nbk).astype(np.float32))
    if kind == 2:
        codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
        w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(128))
    else:
        codes = rng.integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
        w = smg.Q1Weights(codes, scales, smg.WeightLayout.OutIn, n, k, 128)
    colv = orc.f32_to_f16(rng.uniform(0.5, 1.5, n).astype(np.float32))
    bias = orc.f32_to_f16(rng.normal(0, 0.1, n).astype(np.float32))
    ep, nodes, act = None, [], 0
    if graph == "add_silu":
        ep, nodes, act = smg.Epilogue().add_col(bias).silu(), [(4, 0, 0.0, bias, 0)], 3
    elif graph == "mul_add_relu":
        ep = smg.Epilogue().mul_col(colv).add_col(bias).relu()
        nodes, act = [(5, 0, 0.0, colv, 0), (4, 0, 0.0, bias, 0)], 1
    got = np.full(m * n, 0x1234, np.uint16)
    if kind == 2:
        (smg.matmul_q2_ep(a, w, got, m, ep) if ep else smg.matmul_q2(a, w, got, m))
    else:
        (smg.matmul_q1_ep(a, w, got, m, ep) if ep else smg.matmul_q1(a, w, got, m))
    want = orc.matmul_lowbit_ep(kind, a, codes, scales, m, n, k, 128, nodes, act)
    assert np.array_equal(got, want), (kind, m, n, k, graph)
