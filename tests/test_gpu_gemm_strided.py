"""Strided unpacked dense GEMM on the GPU: gemm_f16 / gemm_bf16 / matmul_f16 /
matmul_bf16 (src/kernels/f16.rs:89-204, src/kernels/bf16.rs:101-200) through
gemm_gpu_*_run (host arrays) and smg_gemm_run_dev (device tensors), against
the oracle's reference::gemm_f16 / gemm_bf16 restatement (src/reference.rs:
308-387) on the same operands.

Bar: rel = |g - w| / (1 + |w|) <= f16_tol(K) (bf16: 8x, one bf16 ulp being 8
f16 ulps), the sums running in another order; cells of C outside the view
keep their bytes; alpha = 0 never reads C; k = 0 leaves T(alpha * C)
bit for bit (an empty sum)."""
import numpy as np
import pytest

from conftest import f16_tol, max_rel

pytestmark = pytest.mark.gpu

NAN16 = 0x7E00


def _layout(x, rows, cols, layout):
    """(buffer, row stride, col stride) of a row-major rows x cols uint16 x."""
    x = np.asarray(x, np.uint16).reshape(rows, cols)
    if layout == "row":
        return x.ravel().copy(), cols, 1
    if layout == "col":
        return x.T.ravel().copy(), 1, rows
    ld = cols + 5
    buf = np.full(rows * ld, NAN16, np.uint16)
    buf.reshape(rows, ld)[:, :cols] = x
    return buf, ld, 1


def _cells(buf, rs, cs, m, n):
    return np.array([buf[i * rs + j * cs] for i in range(m) for j in range(n)], np.uint16)


def _operands(orc, m, n, k, bf16, seed):
    rng = np.random.default_rng(seed)
    cv = orc.f32_to_bf16 if bf16 else orc.f32_to_f16
    a = cv(rng.standard_normal(m * k).astype(np.float32))
    b = cv((rng.standard_normal(k * n) * 0.5).astype(np.float32))
    c = cv(rng.standard_normal(m * n).astype(np.float32))
    return a, b, c, cv


def _tol(k, bf16):
    return f16_tol(max(k, 1)) * (8 if bf16 else 1)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 33, 65), (130, 97, 129), (200, 300, 64)])
@pytest.mark.parametrize("la,lb,lc", [("row", "row", "row"), ("col", "col", "col"), ("pad", "row", "pad"),
                                      ("row", "col", "col")])
def test_gemm_strided_host(smg, orc, bf16, m, n, k, la, lb, lc):
    a, b, c0, cv = _operands(orc, m, n, k, bf16, m * 1000 + n * 10 + k)
    ab, rs_a, cs_a = _layout(a, m, k, la)
    bb, rs_b, cs_b = _layout(b, k, n, lb)
    gemm = smg.gemm_bf16 if bf16 else smg.gemm_f16
    for alpha, beta in ((0.0, 1.0), (0.5, -2.0)):
        cin = c0 if alpha else np.full(m * n, NAN16, np.uint16)  # alpha = 0: C never read
        cb, rs_c, cs_c = _layout(cin, m, n, lc)
        want_buf = orc.gemm_strided(cb, rs_c, cs_c, ab, rs_a, cs_a, bb, rs_b, cs_b, m, n, k,
                                    int(cv(np.float32(alpha))[0]), int(cv(np.float32(beta))[0]), bf16)
        got_buf = cb.copy()
        gemm(m, n, k, got_buf, rs_c, cs_c, ab, rs_a, cs_a, bb, rs_b, cs_b, alpha, beta)
        got, want = _cells(got_buf, rs_c, cs_c, m, n), _cells(want_buf, rs_c, cs_c, m, n)
        assert max_rel(got, want, bf16) <= _tol(k, bf16), (alpha, beta)
        if lc == "pad":  # cells outside the view untouched
            assert np.array_equal(got_buf.reshape(m, rs_c)[:, n:], cb.reshape(m, rs_c)[:, n:])


@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_strided_device(smg, orc, bf16):
    """The device form on torch tensors: a column-major C with alpha, a
    transposed A and a padded B."""
    import torch
    m, n, k = 96, 80, 200
    a, b, c0, cv = _operands(orc, m, n, k, bf16, 77)
    ab, rs_a, cs_a = _layout(a, m, k, "col")
    bb, rs_b, cs_b = _layout(b, k, n, "pad")
    cb, rs_c, cs_c = _layout(c0, m, n, "col")
    dt = torch.bfloat16 if bf16 else torch.float16
    dev = lambda x: torch.from_numpy(x.view(np.int16)).cuda().view(dt)  # noqa: E731
    cd = dev(cb)
    gemm = smg.gemm_bf16 if bf16 else smg.gemm_f16
    gemm(m, n, k, cd, rs_c, cs_c, dev(ab), rs_a, cs_a, dev(bb), rs_b, cs_b, 1.0, 0.5)
    torch.cuda.synchronize()
    want = orc.gemm_strided(cb, rs_c, cs_c, ab, rs_a, cs_a, bb, rs_b, cs_b, m, n, k,
                            int(cv(np.float32(1.0))[0]), int(cv(np.float32(0.5))[0]), bf16)
    got = cd.view(torch.int16).cpu().numpy().view(np.uint16)
    assert max_rel(_cells(got, rs_c, cs_c, m, n), _cells(want, rs_c, cs_c, m, n), bf16) <= _tol(k, bf16)


def test_gemm_strided_k0_and_broadcast(smg, orc):
    """k = 0: C = T(alpha * C) bit for bit; a zero row stride of A (every row
    the same) gives identical rows."""
    m, n = 5, 9
    _, _, c0, cv = _operands(orc, m, n, 1, False, 3)
    c = c0.copy()
    smg.gemm_f16(m, n, 0, c, n, 1, np.zeros(0, np.uint16), 0, 1, np.zeros(0, np.uint16), n, 1, 0.5, 1.0)
    assert np.array_equal(c, orc.f32_to_f16(np.float32(0.5) * orc.f16_to_f32(c0)))
    k = 40
    a1, b, _, _ = _operands(orc, 1, n, k, False, 4)
    c = np.zeros(m * n, np.uint16)
    smg.gemm_f16(m, n, k, c, n, 1, a1, 0, 1, b, n, 1, 0.0, 1.0)
    rows = c.reshape(m, n)
    assert all(np.array_equal(rows[0], rows[i]) for i in range(m))
    want = orc.gemm_strided(np.zeros(n, np.uint16), n, 1, a1, k, 1, b, n, 1, 1, n, k, 0, 0x3C00)
    assert max_rel(rows[0], want) <= f16_tol(k)


@pytest.mark.parametrize("bf16", [False, True])
def test_matmul_row_major(smg, orc, bf16):
    m, n, k = 33, 65, 257
    a, b, _, _ = _operands(orc, m, n, k, bf16, 5)
    c = np.zeros(m * n, np.uint16)
    (smg.matmul_bf16 if bf16 else smg.matmul_f16)(a, b, c, m, n, k)
    want = orc.gemm16(a, b, m, n, k, bf16=bf16)
    assert max_rel(c, want, bf16) <= _tol(k, bf16)


def test_run_packed_read_dst(smg, orc):
    """gemm_gpu_f16f16_run_packed with read_dst: with no op-graph
    T(alpha * C + beta * acc) (one rounding, as gemm_strided); with a graph,
    T(graph(T(beta * acc)) + alpha * C)."""
    import ctypes as C
    m, n, k = 40, 72, 96
    a, b, c0, cv = _operands(orc, m, n, k, False, 6)
    packed = smg.prepack_f16(b, n, k)
    half = int(cv(np.float32(0.5))[0])
    c = c0.copy()
    L = smg.lib()
    rc = L.gemm_gpu_f16f16_run_packed(m, n, k, c.ctypes.data, 1, n, 1, a.ctypes.data, 1, k, packed._h,
                                      half, 0x3C00, None)
    assert rc == 0
    want = orc.gemm_strided(c0, n, 1, a, k, 1, b, n, 1, m, n, k, half, 0x3C00)
    assert max_rel(c, want) <= f16_tol(k)
    ep = smg.Epilogue().add_scalar(1.0)
    eptr, keep = smg._ep_ptr(ep, n)
    c = c0.copy()
    rc = L.gemm_gpu_f16f16_run_packed(m, n, k, c.ctypes.data, 1, n, 1, a.ctypes.data, 1, k, packed._h,
                                      half, 0x3C00, eptr)
    assert rc == 0
    base = orc.f16_to_f32(orc.gemm16(a, b, m, n, k)) + np.float32(1.0)
    want = orc.f32_to_f16(orc.f16_to_f32(orc.f32_to_f16(base)) + np.float32(0.5) * orc.f16_to_f32(c0))
    assert max_rel(c, want) <= f16_tol(k)
    del keep
