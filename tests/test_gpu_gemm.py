"""Prefill-shaped MFMA GEMM on the GPU: the dense Gemm builder path and the Q4
GEMM of headline config 4.

Mirrors tests/correctness/epilogue_half.rs:383 (opgraph_f16_mulcol_addcol_silu),
gemv.rs (matmul_f16_packed over ragged shapes) and the strided builder options
(beta, col_major_output). The oracle is the portable path's f32-accumulating
reference GEMM + scalar op-graph; tolerance 2e-3*sqrt(K)/64 on max rel.
"""
import numpy as np
import pytest

from conftest import bf16_tol, f16_tol, max_rel

pytestmark = pytest.mark.gpu


def _rand16(orc, rng, size, scale=1.0, bf16=False):
    x = (rng.standard_normal(size) * scale).astype(np.float32)
    return orc.f32_to_bf16(x) if bf16 else orc.f32_to_f16(x)


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 5, 3), (33, 17, 9), (64, 96, 48),
                                   (128, 64, 80), (65, 257, 257), (97, 300, 131),
                                   (130, 200, 1000), (256, 384, 512)])
@pytest.mark.parametrize("bf16", [False, True])
def test_packed_gemm_plain(smg, orc, m, n, k, bf16):
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = _rand16(orc, rng, m * k, 0.5, bf16)
    b = _rand16(orc, rng, k * n, 0.5, bf16)
    packed = smg.prepack_bf16(b, n, k) if bf16 else smg.prepack_f16(b, n, k)
    c = np.zeros(m * n, np.uint16)
    smg.Gemm(a, packed, m).run(c)
    want = orc.packed_ep(a, b, m, n, k, bf16=bf16)
    tol = bf16_tol(k) if bf16 else f16_tol(k)
    assert max_rel(c, want, bf16) <= tol


@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_builder_all_ops(smg, orc, bf16):
    """Every op-graph node kind and activation in one graph, plus beta and
    column-major output (src/exec/builder.rs:428-814)."""
    m, n, k = 70, 90, 128
    rng = np.random.default_rng(42)
    a = _rand16(orc, rng, m * k, 0.3, bf16)
    b = _rand16(orc, rng, k * n, 0.3, bf16)
    cv = orc.f32_to_bf16 if bf16 else orc.f32_to_f16
    col = cv(rng.uniform(0.5, 1.5, n).astype(np.float32))
    row = cv(rng.uniform(0.5, 1.5, m).astype(np.float32))
    ten = cv(rng.uniform(-0.5, 0.5, m * (n + 3)).astype(np.float32))
    packed = smg.prepack_bf16(b, n, k) if bf16 else smg.prepack_f16(b, n, k)
    for col_major in (False, True):
        g = smg.Gemm(a, packed, m).beta(0.75)
        g = g.mul_col(col).add_row(row).sub_scalar(0.125).div_col(col).add_tensor(ten, n + 3)
        g = g.max(-1.0).min(2.0).mul_row(row).leaky_relu(0.1).hardswish().softplus().gelu()
        if col_major:
            g = g.col_major_output()
        c = np.zeros(m * n, np.uint16)
        g.run(c)
        beta_bits = int(cv(np.float32(0.75))[0])
        s = lambda v: float(orc.f16_to_f32(orc.f32_to_f16(np.float32(v)))[0])  # noqa: E731
        nodes = [(5, 0, 0.0, col, 0), (2, 0, 0.0, row, 0), (11, 0, s(0.125), None, 0),
                 (17, 0, 0.0, col, 0), (6, 0, 0.0, ten, n + 3), (9, 0, s(-1.0), None, 0),
                 (10, 0, s(2.0), None, 0), (3, 0, 0.0, row, 0),
                 (8, 6, float(np.float32(0.1)), None, 0), (8, 9, 0.0, None, 0),
                 (8, 22, 0.0, None, 0)]
        want = orc.packed_ep(a, b, m, n, k, nodes, 2, beta_bits, col_major, bf16)
        tol = bf16_tol(k) if bf16 else f16_tol(k)
        assert max_rel(c, want, bf16) <= tol, f"col_major={col_major}"


def test_gemm_every_activation(smg, orc):
    """All 24 activation kinds as in-order nodes, each vs the f64 scalar path."""
    m, n, k = 16, 64, 64
    rng = np.random.default_rng(8)
    a = _rand16(orc, rng, m * k, 0.4)
    b = _rand16(orc, rng, k * n, 0.4)
    packed = smg.prepack_f16(b, n, k)
    names = ["relu", "gelu", "silu", "tanh", "sigmoid"]
    for kind in range(1, 25):
        g = smg.Gemm(a, packed, m)
        if kind <= 5:
            g = getattr(g, names[kind - 1])()
            nodes, act = [], kind
        else:
            meth = {6: ("leaky_relu", (0.2,)), 7: ("relu6", ()), 8: ("hardsigmoid", ()),
                    9: ("hardswish", ()), 10: ("abs", ()), 11: ("neg", ()), 12: ("square", ()),
                    13: ("sign", ()), 14: ("sqrt", ()), 15: ("softsign", ()), 16: ("recip", ()),
                    17: ("rsqrt", ()), 18: ("exp", ()), 19: ("log", ()), 20: ("elu", (0.7,)),
                    21: ("selu", ()), 22: ("softplus", ()), 23: ("mish", ()),
                    24: ("gelu_exact", ())}[kind]
            g = getattr(g, meth[0])(*meth[1])
            alpha = float(np.float32(meth[1][0])) if meth[1] else 0.0
            nodes, act = [(8, kind, alpha, None, 0)], None
        c = np.zeros(m * n, np.uint16)
        g.run(c)
        want = orc.packed_ep(a, b, m, n, k, nodes, act)
        assert max_rel(c, want) <= f16_tol(k), f"activation {kind}"


@pytest.mark.parametrize("m,n,k", [(64, 1024, 4096), (512, 512, 4096), (300, 700, 1000)])
def test_q4_gemm_config4_epilogue_slices(smg, orc, m, n, k):
    """Config 4's arithmetic (Q4 block 32, mul_col, add_col, silu) on slices the
    oracle finishes in seconds."""
    import workloads
    a, quants, scales, _ = workloads.q4_inputs(m, n, k, seed=4)
    s, b = workloads.q4_gemm_epilogue_inputs(n)
    w = smg.Q4Weights(quants, scales, n, k)
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a, w, c, m, smg.Epilogue().mul_col(s).add_col(b).silu())
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32,
                            [(5, 0, 0.0, s, 0), (4, 0, 0.0, b, 0)], 3)
    assert max_rel(c, want) <= f16_tol(k)


def test_q4_gemm_config4_full_size_vs_torch(smg, orc):
    """Full config 4 (m=512, K=4096, N=14336) against a torch fp32 GEMM over the
    oracle's dequantized weights (the kernel is floating point: f32 accumulate)."""
    import torch
    import workloads
    m, n, k = 512, 14336, 4096
    a, quants, scales, _ = workloads.q4_inputs(m, n, k, seed=0)
    s, b = workloads.q4_gemm_epilogue_inputs(n)
    w = smg.Q4Weights(quants, scales, n, k)
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a, w, c, m, smg.Epilogue().mul_col(s).add_col(b).silu())
    wdq = orc.q4_dequant(quants, scales, None, n, k, 32)
    A = torch.from_numpy(a.view(np.float16).astype(np.float32)).reshape(m, k).cuda()
    B = torch.from_numpy(wdq.view(np.float16).astype(np.float32)).reshape(k, n).cuda()
    acc = (A @ B).cpu().numpy().astype(np.float32)
    x = acc.astype(np.float16).astype(np.float32)
    x = x * s.view(np.float16).astype(np.float32)[None, :]
    x = x + b.view(np.float16).astype(np.float32)[None, :]
    x64 = x.astype(np.float64)
    want = (x64 / (1.0 + np.exp(-x64))).astype(np.float32).astype(np.float16).view(np.uint16)
    assert max_rel(c, want.ravel()) <= f16_tol(k)


def test_q4_dequant_eager_matches_oracle_bits(smg, orc):
    """dequant_q4 / dequant_q4_with / dequant_q4_bf16 on the device give the
    portable dequant's weights: a GEMM with A = identity rows returns them."""
    n, k = 96, 64
    rng = np.random.default_rng(12)
    for affine in (False, True):
        for bf16 in (False, True):
            nbk = k // 32
            quants = rng.integers(0, 256, k * n // 2, dtype=np.uint8)
            scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * nbk).astype(np.float32))
            mins = orc.f32_to_f16(rng.uniform(-0.1, 0.1, n * nbk).astype(np.float32)) \
                if affine else None
            p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
            fn = smg.dequant_q4_bf16_with if bf16 else smg.dequant_q4_with
            packed = fn(quants, scales, mins, n, k, p)
            one = 0x3F80 if bf16 else 0x3C00
            eye = np.zeros(k * k, np.uint16)
            eye[:: k + 1] = one
            c = np.zeros(k * n, np.uint16)
            smg.Gemm(eye, packed, k).run(c)
            want = orc.q4_dequant(quants, scales, mins, n, k, 32, bf16)
            assert np.array_equal(c, want), f"affine={affine} bf16={bf16}"


@pytest.mark.parametrize("m,n,k,block,affine", [
    (9, 256, 64, 32, False), (40, 300, 128, 64, True), (129, 520, 320, 32, False),
    (200, 1000, 512, 128, True), (256, 768, 1024, 32, False), (17, 129, 192, 64, False),
    (512, 512, 4096, 32, False), (130, 384, 256, 256, True),
    # 128-240 tiles (about one per CU) with short K
    (512, 8192, 256, 32, False), (640, 8192, 512, 64, True), (136, 30720, 128, 32, False)])
def test_q4_register_weight_gemm(smg, orc, m, n, k, block, affine):
    """The Q4 f16 prefill kernel that dequantizes weights in registers (K a
    multiple of 64, block >= 32; two waves split each 64-depth step and add
    their f32 partial tiles): within tolerance of the oracle and of the dense
    GEMM over the eagerly dequantized weights."""
    rng = np.random.default_rng(m + n + k + block)
    nbk = -(-k // block)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.002, 0.02, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.05, 0.05, n * nbk).astype(np.float32)) if affine else None
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w, c, m)
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, block)
    assert max_rel(c, want) <= f16_tol(k)
    packed = smg.dequant_q4_with(quants, scales, mins, n, k, p)
    d = np.zeros(m * n, np.uint16)
    smg.Gemm(a, packed, m).run(d)
    assert max_rel(c, d) <= f16_tol(k)


def test_q4_register_weight_gemm_epilogue_repeat(smg, orc):
    """The prefill configuration's op-graph (mul_col, add_col, silu) on a grid
    of about one tile per CU, twice in a row into fresh outputs, within
    tolerance of the oracle both times."""
    m, n, k = 512, 8192, 256
    rng = np.random.default_rng(7)
    quants = rng.integers(0, 256, k * n // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.002, 0.02, n * (k // 32)).astype(np.float32))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    sc = orc.f32_to_f16(rng.uniform(0.5, 1.5, n).astype(np.float32))
    bias = orc.f32_to_f16((0.1 * rng.standard_normal(n)).astype(np.float32))
    w = smg.Q4Weights.with_params(quants, scales, None, n, k, smg.Q4Params(32))
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32,
                            [(5, 0, 0.0, sc, 0), (4, 0, 0.0, bias, 0)], 3)
    for _ in range(2):
        c = np.zeros(m * n, np.uint16)
        smg.matmul_q4_ep(a, w, c, m, smg.Epilogue().mul_col(sc).add_col(bias).silu())
        assert max_rel(c, want) <= f16_tol(k)


@pytest.mark.parametrize("graph", ["none", "add_col", "add_col_relu", "mul_add_silu", "mul_add_gelu",
                                   "mul_add_sigmoid", "add_col_tanh"])
@pytest.mark.parametrize("m,n,k,affine", [(200, 1000, 512, False), (512, 2056, 1024, True), (130, 300, 256, False)])
def test_q4_gemm_compiled_store_equals_interpreted(smg, orc, graph, m, n, k, affine):
    """The prefill GEMM compiles its store for the common op-graphs (none,
    [add_col] + act, [mul_col, add_col] + act). The same graph with an extra
    mul_scalar(1.0) node (x * 1 is exact in f32) takes the interpreted store:
    the two give the same bits, and both are within tolerance of the oracle."""
    rng = np.random.default_rng(m + n + k)
    nbk = k // 32
    quants = rng.integers(0, 256, k * n // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.002, 0.02, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.05, 0.05, n * nbk).astype(np.float32)) if affine else None
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    sc = orc.f32_to_f16(rng.uniform(0.5, 1.5, n).astype(np.float32))
    bias = orc.f32_to_f16((0.1 * rng.standard_normal(n)).astype(np.float32))
    p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)

    def build(extra):
        e = smg.Epilogue()
        nodes, act = [], None
        if graph.startswith("mul_add"):
            e = e.mul_col(sc).add_col(bias)
            nodes = [(5, 0, 0.0, sc, 0), (4, 0, 0.0, bias, 0)]
        elif graph.startswith("add_col"):
            e = e.add_col(bias)
            nodes = [(4, 0, 0.0, bias, 0)]
        if extra:
            e = e.mul_scalar(1.0)
            nodes = nodes + [(1, 0, 1.0, None, 0)]
        for name, kind in (("relu", 1), ("gelu", 2), ("silu", 3), ("tanh", 4), ("sigmoid", 5)):
            if graph.endswith(name):
                e = getattr(e, name)()
                act = kind
        return e, nodes, act

    e0, nodes0, act0 = build(False)
    e1, _, _ = build(True)
    c0 = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a, w, c0, m, e0)
    c1 = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a, w, c1, m, e1)
    assert np.array_equal(c0, c1), graph
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, 32, nodes0, act0)
    assert max_rel(c0, want) <= f16_tol(k)
