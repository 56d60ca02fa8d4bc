"""Op-graphs longer than the 16 nodes a product kernel's store applies, up to
SMG_MAX_EP_NODES (64): the product is stored without a graph, then one pass
over C applies the whole graph -- the reference's own order, GEMM to T then
apply_ep_scalar (src/exec/macros.rs:188-206).

Bar: bit for bit against the same call with no graph, followed by the oracle's
apply_ep (src/exec/scalar.rs:125-140) on that output. Cases: the Q4 GEMV and
GEMM (f16, bf16), the low-bit GEMV and MOPA, the packed GEMM (row- and
column-major C, and read_dst's alpha * old C added after the graph), each in
its host and device form; 17 and 64 nodes alike; 65 nodes, or 17 on the chained
GEMV, refused.
"""
import numpy as np
import pytest

import workloads as WL
from conftest import ulp_dist

pytestmark = pytest.mark.gpu


def _dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.int16)).cuda()


def _bits(t):
    return t.cpu().numpy().view(np.uint16).ravel()


def _steps(orc, seed, length, m, n, bf16):
    """length - 1 in-order nodes drawn from every node family that stays
    finite, then a trailing silu: (builder method, args) pairs."""
    rng = np.random.default_rng(seed)
    cv = orc.f32_to_bf16 if bf16 else orc.f32_to_f16
    u = lambda lo, hi, size: cv(rng.uniform(lo, hi, size).astype(np.float32))  # noqa: E731
    ld = n + 3
    row, rowp, col, colp = u(-0.5, 0.5, m), u(0.75, 1.25, m), u(-0.5, 0.5, n), u(0.75, 1.25, n)
    ten, tenp = u(-0.5, 0.5, m * ld), u(0.75, 1.25, m * ld)
    menu = [("add_scalar", (0.25,)), ("mul_scalar", (1.125,)), ("sub_scalar", (0.0625,)), ("div_scalar", (2.0,)),
            ("max", (-3.0,)), ("min", (4.0,)), ("add_row", (row,)), ("mul_row", (rowp,)), ("sub_row", (row,)),
            ("max_row", (row,)), ("min_row", (rowp,)), ("add_col", (col,)), ("mul_col", (colp,)),
            ("sub_col", (col,)), ("max_col", (col,)), ("min_col", (colp,)), ("add_tensor", (ten, ld)),
            ("mul_tensor", (tenp, ld)), ("sub_tensor", (ten, 0)), ("leaky_relu", (0.1,)), ("relu6", ()),
            ("hardsigmoid", ()), ("hardswish", ()), ("abs", ()), ("neg", ()), ("softsign", ()), ("selu", ()),
            ("softplus", ()), ("elu", (1.0,))]
    pick = rng.integers(0, len(menu), length - 1)
    return [menu[i] for i in pick]


def _graph(smg, steps, bf16, device=False):
    ep = smg.Epilogue(bf16)
    for name, args in steps:
        args = tuple(_dev(a) if device and isinstance(a, np.ndarray) else a for a in args)
        getattr(ep, name)(*args)
    return ep.silu()


def _expected(orc, plain, m, n, steps, smg, bf16, col_major=False):
    host = _graph(smg, steps, bf16)
    nodes = [(op, aux, scalar, v, ld) for op, aux, scalar, v, ld in host.nodes]
    return orc.apply_ep(plain, m, n, nodes, 3, bf16, col_major)


@pytest.mark.parametrize("m,n,k,bf16,length", [(1, 256, 512, False, 17), (1, 256, 512, False, 64),
                                                (3, 200, 256, False, 40), (100, 300, 256, False, 33),
                                                (1, 256, 512, True, 20), (80, 256, 256, True, 40)])
def test_q4_long_graph(smg, orc, m, n, k, bf16, length):
    import torch
    a, quants, scales, _ = WL.q4_inputs(m, n, k, seed=m + length)
    if bf16:
        a = orc.f32_to_bf16(orc.f16_to_f32(a))
    w = smg.Q4Weights(quants, scales, n, k)
    fn = smg.matmul_q4_bf16_ep if bf16 else smg.matmul_q4_ep
    steps = _steps(orc, length, length, m, n, bf16)
    plain = np.zeros(m * n, np.uint16)
    fn(a, w, plain, m, smg.Epilogue(bf16))
    want = _expected(orc, plain, m, n, steps, smg, bf16)
    got = np.zeros(m * n, np.uint16)
    fn(a, w, got, m, _graph(smg, steps, bf16))
    assert np.array_equal(got, want)
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    fn(_dev(a), w, cd, m, _graph(smg, steps, bf16, device=True))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(cd), want)


@pytest.mark.parametrize("kind,m,mopa,length", [(2, 1, False, 17), (1, 1, False, 48), (2, 8, False, 30),
                                                 (2, 20, True, 25)])
def test_lowbit_long_graph(smg, orc, kind, m, mopa, length):
    import torch
    n, k = 384, 1024
    if kind == 2:
        a, codes, sc = WL.q2_inputs(m, n, k, seed=m + length)
        w = smg.Q2Weights(codes, sc, n, k, smg.Q2Params(128))
        fn = smg.matmul_q2_mopa_ep if mopa else smg.matmul_q2_ep
    else:
        a, signs, sc, _ = WL.q1_inputs(m, n, k, seed=m + length)
        w = smg.Q1Weights(signs, sc, smg.WeightLayout.OutIn, n, k, 128)
        fn = smg.matmul_q1_ep
    steps = _steps(orc, 100 + length, length, m, n, False)
    plain = np.zeros(m * n, np.uint16)
    fn(a, w, plain, m, smg.Epilogue())
    want = _expected(orc, plain, m, n, steps, smg, False)
    got = np.zeros(m * n, np.uint16)
    fn(a, w, got, m, _graph(smg, steps, False))
    assert np.array_equal(got, want)
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    fn(_dev(a), w, cd, m, _graph(smg, steps, False, device=True))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(cd), want)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("col_major", [False, True])
def test_packed_long_graph(smg, orc, bf16, col_major):
    import torch
    m, n, k, length = 70, 90, 128, 37
    rng = np.random.default_rng(7)
    cv = orc.f32_to_bf16 if bf16 else orc.f32_to_f16
    a = cv((rng.standard_normal(m * k) * 0.3).astype(np.float32))
    b = cv((rng.standard_normal(k * n) * 0.3).astype(np.float32))
    packed = smg.prepack_bf16(b, n, k) if bf16 else smg.prepack_f16(b, n, k)
    steps = _steps(orc, 200 + int(bf16), length, m, n, bf16)

    def run(c, ep, a_in):
        g = smg.Gemm(a_in, packed, m).beta(0.75)
        g.ep = ep
        if col_major:
            g = g.col_major_output()
        return g.run(c)
    plain = run(np.zeros(m * n, np.uint16), smg.Epilogue(bf16), a)
    want = _expected(orc, plain, m, n, steps, smg, bf16, col_major)
    got = run(np.zeros(m * n, np.uint16), _graph(smg, steps, bf16), a)
    assert np.array_equal(got, want)
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    run(cd, _graph(smg, steps, bf16, device=True), _dev(a))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(cd), want)


@pytest.mark.parametrize("length", [12, 40])
def test_packed_long_graph_adds_old_c_after_the_graph(smg, orc, length):
    """read_dst with a graph: C = T(T(graph(T(beta * A @ B))) + alpha * old C),
    the store's add_dst step, for a graph the store applies itself (12 nodes)
    and one past it (40): the product then goes to scratch, the old C stays,
    and the graph's pass adds it."""
    m, n, k = 40, 72, 96
    rng = np.random.default_rng(length)
    a = orc.f32_to_f16((rng.standard_normal(m * k) * 0.3).astype(np.float32))
    b = orc.f32_to_f16((rng.standard_normal(k * n) * 0.3).astype(np.float32))
    old = orc.f32_to_f16(rng.uniform(-2, 2, m * n).astype(np.float32))
    packed = smg.prepack_f16(b, n, k)
    steps = _steps(orc, 300 + length, length, m, n, False)
    lib = smg.lib()
    alpha_bits = int(orc.f32_to_f16(np.array([0.5], np.float32))[0])
    beta_bits = int(orc.f32_to_f16(np.array([0.75], np.float32))[0])

    def call(c, ep, read_dst):
        eptr, keep = smg._ep_ptr(ep, n)
        rc = lib.gemm_gpu_f16f16_run_packed(m, n, k, c.ctypes.data, 1, n, int(read_dst), a.ctypes.data, 1, k,
                                            packed._h, alpha_bits if read_dst else 0, beta_bits, eptr)
        assert rc == 0, smg.last_error()
        return c
    plain = call(np.zeros(m * n, np.uint16), smg.Epilogue(), False)
    graphed = _expected(orc, plain, m, n, steps, smg, False)
    x = orc.f16_to_f32(graphed).astype(np.float32) + np.float32(0.5) * orc.f16_to_f32(old).astype(np.float32)
    want = orc.f32_to_f16(x.astype(np.float32))
    got = call(old.copy(), _graph(smg, steps, False), True)
    if length > 16:
        assert np.array_equal(got, want)
    else:
        # the store's own graph computes a trailing activation in f32 (the
        # fast form the GEMM stores use), the oracle rounds it once from f64
        assert ulp_dist(got, want) <= 1


def test_graph_length_limits(smg, orc):
    """65 nodes are refused on every call; the chained GEMV's device form takes
    at most 16 (its kernel raises done once C is stored)."""
    import torch
    m, n, k = 1, 256, 512
    a, quants, scales, _ = WL.q4_inputs(m, n, k, seed=5)
    w = smg.Q4Weights(quants, scales, n, k)
    ep = smg.Epilogue()
    for _ in range(65):
        ep.add_scalar(0.0)
    with pytest.raises(smg.SmeGemmError, match="too many nodes"):
        smg.matmul_q4_ep(a, w, np.zeros(n, np.uint16), m, ep)
    long_ep = smg.Epilogue()
    for _ in range(17):
        long_ep.mul_scalar(1.0)
    cd = torch.zeros(n, dtype=torch.int16, device="cuda")
    assert not smg.q4_chained(_dev(a), w, cd, long_ep)
    assert "at most SMG_FUSED_EP_NODES" in smg.last_error()
    # the host chained form runs the host GEMV, whose graph pass ends before done
    c = np.zeros(n, np.uint16)
    assert smg.q4_chained(a, w, c, long_ep)
    plain = np.zeros(n, np.uint16)
    smg.matmul_q4(a, w, plain, m)
    assert np.array_equal(c, plain)
