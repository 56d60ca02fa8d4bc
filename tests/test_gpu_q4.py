"""Q4 path on the GPU vs the CPU oracle (the reference's portable path).

Mirrors tests/correctness/q4.rs (q4_resident :66, q4_blocks_and_affine :127,
q4_fused_epilogue_matches_oracle :417), gemv.rs:229 (gemv_q4) and the
headline configs 1 and 4 (the benchmark shapes). Float outputs: max |g-w|/(1+|w|) against
the oracle's rounded output within 2e-3*sqrt(K)/64 (f16) or 8x that (bf16);
the empty epilogue is pinned bitwise to the plain call (q4.rs:508-513).
"""
import threading

import numpy as np
import pytest

from conftest import bf16_tol, f16_tol, max_rel

pytestmark = pytest.mark.gpu

# (m, n, k): the reference's SIZES (tests/correctness/main.rs:80-91) + tails
SIZES = [(1, 1, 1), (7, 5, 3), (31, 31, 31), (32, 32, 32), (33, 17, 9), (64, 96, 48),
         (128, 64, 80), (40, 8, 7), (7, 50, 200), (96, 96, 256)]
TAIL_SIZES = [(65, 257, 257), (33, 512, 257), (97, 300, 131), (7, 400, 800), (33, 161, 401)]


def _lcg_q4(orc, seed, m, n, k, block):
    """q4.rs:74-82 data: fill() activations, LCG bytes, scales 0.01+0.001*(i%5)."""
    a, s = orc.lcg_fill(seed, m * k)
    quants = orc.lcg_bytes(s, (k * n + 1) // 2)
    nbk = -(-k // block)
    scales = orc.f32_to_f16(np.float32(0.01) + np.float32(0.001) * (np.arange(n * nbk) % 5)
                            .astype(np.float32))
    return a, quants, scales


@pytest.mark.parametrize("m,n,k", SIZES + TAIL_SIZES)
def test_q4_resident_sizes(smg, orc, m, n, k):
    seed = 0x4444_9999_DEAD_0001 ^ (m * 131 + n * 17 + k)
    a, quants, scales = _lcg_q4(orc, seed, m, n, k, 32)
    w = smg.Q4Weights(quants, scales, n, k)
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w, c, m)
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32)
    assert max_rel(c, want) <= f16_tol(k), f"{m}x{n}x{k}"


GEMV_CASES = [(1, 33, 256), (1, 389, 1027), (1, 1100, 2051), (2, 100, 70), (3, 129, 1027),
              (4, 4109, 4099), (5, 70, 513), (7, 1030, 2050)]


@pytest.mark.parametrize("m,n,k", GEMV_CASES)
@pytest.mark.parametrize("block", [16, 32, 64])
@pytest.mark.parametrize("affine", [False, True])
def test_gemv_q4_blocks_affine(smg, orc, m, n, k, block, affine):
    """gemv.rs:229-300: ragged N and K, partial last block, both forms."""
    rng = np.random.default_rng(n * 17 + k + block)
    nbk = -(-k // block)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(np.float32(0.01) + np.float32(0.001) * (np.arange(n * nbk) % 7))
    mins = orc.f32_to_f16(np.float32(0.05) * (np.arange(n * nbk) % 5) - np.float32(0.1)) \
        if affine else None
    a = orc.f32_to_f16((np.arange(m * k) % 13).astype(np.float32) * np.float32(0.05)
                       - np.float32(0.3))
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w, c, m)
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, block)
    assert max_rel(c, want) <= f16_tol(k)


@pytest.mark.parametrize("block", [1, 2, 16, 32, 64, 128])
@pytest.mark.parametrize("m", [1, 6, 40])
def test_q4_block_sizes_gemv_and_gemm(smg, orc, block, m):
    """q4.rs:127: every power-of-two block (GEMV for m <= 8, MFMA above)."""
    n, k = 70, 200
    rng = np.random.default_rng(block * 100 + m)
    nbk = -(-k // block)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * nbk).astype(np.float32))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    w = smg.Q4Weights.with_params(quants, scales, None, n, k, smg.Q4Params(block))
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w, c, m)
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, block)
    assert max_rel(c, want) <= f16_tol(k)


def test_config1_q4_gemv(smg, orc):
    """Headline config 1: m=1, K=N=4096, block 32, seed 0."""
    import workloads
    m, n, k = 1, 4096, 4096
    a, quants, scales, _ = workloads.q4_inputs(m, n, k, seed=0)
    w = smg.Q4Weights(quants, scales, n, k)
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w, c, m)
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32)
    assert max_rel(c, want) <= f16_tol(k)
    # most outputs agree bit for bit (differences are f32 summation order only)
    assert np.mean(c == want) > 0.99


@pytest.mark.parametrize("m,n,k", [(64, 96, 128), (65, 33, 256), (200, 520, 512), (1, 96, 128),
                                   (5, 33, 256)])
@pytest.mark.parametrize("affine", [False, True])
def test_q4_fused_epilogue_matches_oracle(smg, orc, m, n, k, affine):
    """q4.rs:417-515 cases 0..3; the empty graph equals matmul_q4 bitwise."""
    nbk = -(-k // 32)
    rng = np.random.default_rng(m * 131 + n * 17 + k)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(np.float32(0.01) + np.float32(0.001) * (np.arange(n * nbk) % 7))
    mins = orc.f32_to_f16(np.float32(0.05) * (np.arange(n * nbk) % 5) - np.float32(0.1)) \
        if affine else None
    a = orc.f32_to_f16((np.arange(m * k) % 13) * np.float32(0.05) - np.float32(0.3))
    col = orc.f32_to_f16(np.float32(0.02) * np.arange(n, dtype=np.float32) - np.float32(0.4))
    row = orc.f32_to_f16(np.float32(0.01) * np.arange(m, dtype=np.float32) - np.float32(0.2))
    p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    for case in range(4):
        ep = smg.Epilogue()
        nodes, act = [], None
        if case >= 1:
            ep = ep.add_col(col) if case < 3 else ep.add_row(row).add_col(col)
            nodes = [(4, 0, 0.0, col, 0)] if case < 3 else [(2, 0, 0.0, row, 0), (4, 0, 0.0, col, 0)]
        if case == 2:
            ep = ep.relu()
            act = 1
        if case == 3:
            ep = ep.gelu()
            act = 2
        got = np.zeros(m * n, np.uint16)
        smg.matmul_q4_ep(a, w, got, m, ep)
        want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, 32, nodes, act)
        assert max_rel(got, want) <= f16_tol(k), f"case {case}"
        if case == 0:
            plain = np.zeros(m * n, np.uint16)
            smg.matmul_q4(a, w, plain, m)
            assert np.array_equal(plain, got)


@pytest.mark.parametrize("m,n,k", [(1, 96, 128), (3, 200, 300), (64, 96, 128), (33, 70, 257)])
@pytest.mark.parametrize("affine", [False, True])
def test_q4_bf16(smg, orc, m, n, k, affine):
    """matmul_q4_bf16(_ep) vs the bf16 portable path (q4/matmul.rs:258-270)."""
    nbk = -(-k // 32)
    rng = np.random.default_rng(7 * m + n + k)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.1, 0.1, n * nbk).astype(np.float32)) if affine else None
    a = orc.f32_to_bf16(rng.standard_normal(m * k).astype(np.float32))
    bias = orc.f32_to_bf16(rng.normal(0, 0.1, n).astype(np.float32))
    p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q4_bf16_ep(a, w, got, m, smg.Epilogue().add_col(bias).silu())
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, 32, [(4, 0, 0.0, bias, 0)], 3,
                            bf16=True)
    assert max_rel(got, want, bf16=True) <= bf16_tol(k)


@pytest.mark.parametrize("m,n,k", [(48, 1536, 1024), (100, 4096, 512), (128, 700, 1088)])
@pytest.mark.parametrize("affine", [False, True])
def test_q4_bf16_rows_on_gemv_launches(smg, orc, m, n, k, affine):
    """bf16 calls of 33 to 128 rows: the register-dequant GEMM with K split
    over the compute units (ROW and TENSOR operands through the reduction's
    store), and -- with A one element off 16-byte alignment, which the GEMM's
    DMA cannot read -- 16-row GEMV launches with ROW and TENSOR operands
    offset per launch; both against the bf16 portable path."""
    nbk = k // 32
    rng = np.random.default_rng(3 * m + n + k + affine)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.1, 0.1, n * nbk).astype(np.float32)) if affine else None
    a = orc.f32_to_bf16(rng.standard_normal(m * k).astype(np.float32))
    row = orc.f32_to_bf16(rng.normal(0, 0.1, m).astype(np.float32))
    ten = orc.f32_to_bf16(rng.normal(1, 0.1, m * n).astype(np.float32))
    col = orc.f32_to_bf16(rng.normal(0, 0.1, n).astype(np.float32))
    p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q4_bf16_ep(a, w, got, m, smg.Epilogue().add_row(row).mul_tensor(ten).add_col(col).silu())
    nodes = [(2, 0, 0.0, row, 0), (7, 0, 0.0, ten, 0), (4, 0, 0.0, col, 0)]
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, 32, nodes, 3, bf16=True)
    assert max_rel(got, want, bf16=True) <= bf16_tol(k)
    import torch
    dev = lambda x: torch.from_numpy(x.view(np.int16)).cuda()  # noqa: E731
    buf = torch.zeros(m * k + 1, dtype=torch.int16, device="cuda")
    buf[1:] = dev(a)
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    smg.matmul_q4_bf16_ep(buf[1:].view(torch.bfloat16), w, cd.view(torch.bfloat16), m,
                          smg.Epilogue(bf16=True).add_row(dev(row)).mul_tensor(dev(ten)).add_col(dev(col)).silu())
    torch.cuda.synchronize()
    assert max_rel(cd.cpu().numpy().view(np.uint16), want, bf16=True) <= bf16_tol(k)


@pytest.mark.parametrize("m,n,k,affine", [(512, 8192, 256, False), (512, 8192, 256, True), (256, 2048, 1024, False),
                                          (200, 1000, 4096, True), (64, 4096, 4096, False)])
def test_q4_bf16_prefill_gemm(smg, orc, m, n, k, affine):
    """matmul_q4_bf16 prefill on the register-dequant MFMA GEMM (bf16
    activations and weights, v_mfma_f32_16x16x32_bf16): unsplit grids (at least
    half the compute units of tiles) with the compiled [mul_col, add_col] +
    silu store and the interpreted store (the same graph with an exact
    mul_scalar(1.0): the same bits), and K-split grids; against the bf16
    portable path (q4/matmul.rs:258-270) at the bf16 bound."""
    nbk = k // 32
    rng = np.random.default_rng(m + n + k + affine)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.1, 0.1, n * nbk).astype(np.float32)) if affine else None
    a = orc.f32_to_bf16(rng.standard_normal(m * k).astype(np.float32))
    sc = orc.f32_to_bf16(rng.uniform(0.5, 1.5, n).astype(np.float32))
    bias = orc.f32_to_bf16(rng.normal(0, 0.1, n).astype(np.float32))
    p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q4_bf16_ep(a, w, got, m, smg.Epilogue(bf16=True).mul_col(sc).add_col(bias).silu())
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, 32,
                            [(5, 0, 0.0, sc, 0), (4, 0, 0.0, bias, 0)], 3, bf16=True)
    assert max_rel(got, want, bf16=True) <= bf16_tol(k)
    interp = np.zeros(m * n, np.uint16)
    smg.matmul_q4_bf16_ep(a, w, interp, m, smg.Epilogue(bf16=True).mul_col(sc).add_col(bias).mul_scalar(1.0).silu())
    assert np.array_equal(interp, got)
    plain = np.zeros(m * n, np.uint16)
    smg.matmul_q4_bf16(a, w, plain, m)
    assert max_rel(plain, orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, 32, bf16=True), bf16=True) \
        <= bf16_tol(k)


@pytest.mark.parametrize("m", [8, 16])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("block", [32, 64])
def test_gemv_weights_bitwise(smg, orc, m, bf16, affine, block):
    """Every weight the GEMV multiplies, read back exactly: row r of A is one
    at depth d_r and zero elsewhere, so C[r][j] is the weight (d_r, j) times
    one plus exact zeros -- it must equal the portable dequant's weight bit
    for bit (f16: RNE(scale*code [+ min]) once; bf16: through f32,
    src/kernels/q4/mod.rs:193-257), for the first and last depths of a block,
    the last depth of K, and the ragged last column."""
    n, k = 200, 300
    nbk = -(-k // block)
    rng = np.random.default_rng(block + 2 * affine + bf16 + m)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(-0.05, 0.05, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.1, 0.1, n * nbk).astype(np.float32)) if affine else None
    depths = [0, 1, block - 1, block, 2 * block + 5, k - 33, k - 2, k - 1,
              2, 31, 32, 63, 64, 100, 200, 255][:m]
    one = 0x3F80 if bf16 else 0x3C00
    a = np.zeros((m, k), np.uint16)
    for r, d in enumerate(depths):
        a[r, d] = one
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    got = np.zeros(m * n, np.uint16)
    (smg.matmul_q4_bf16 if bf16 else smg.matmul_q4)(a.ravel(), w, got, m)
    deq = orc.q4_dequant(quants, scales, mins, n, k, block, bf16).reshape(k, n)
    want = deq[depths]
    # a weight of -0 times one plus +0 terms sums to +0
    want = np.where(want == 0x8000, np.uint16(0), want)
    assert np.array_equal(got.reshape(m, n), want)


@pytest.mark.parametrize("m", [1, 5, 16, 40])
@pytest.mark.parametrize("bf16", [False, True])
def test_affine_zero_mins_equals_scale_bitwise(smg, orc, m, bf16):
    """Q4Form::Scale is exactly Affine with all-zero mins
    (src/kernels/q4/weights.rs:356-380, positive scales as there): the same
    call through the affine kernels gives the same bits."""
    n, k, block = 200, 320, 32
    nbk = -(-k // block)
    rng = np.random.default_rng(m + 10 * bf16)
    cv = orc.f32_to_bf16 if bf16 else orc.f32_to_f16
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.03, n * nbk).astype(np.float32))
    zeros = np.zeros(n * nbk, np.uint16)
    a = cv(rng.standard_normal(m * k).astype(np.float32))
    plain = smg.Q4Weights.with_params(quants, scales, None, n, k, smg.Q4Params(block))
    aff = smg.Q4Weights.with_params(quants, scales, zeros, n, k, smg.Q4Params(block).affine())
    fn = smg.matmul_q4_bf16 if bf16 else smg.matmul_q4
    c0, c1 = np.zeros(m * n, np.uint16), np.zeros(m * n, np.uint16)
    fn(a, plain, c0, m)
    fn(a, aff, c1, m)
    assert np.array_equal(c0, c1)


@pytest.mark.parametrize("m", [9, 12, 16, 24, 32])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("n,k", [(200, 300), (1030, 4099), (4096, 4096)])
def test_q4_wide_gemv_rows(smg, orc, m, bf16, affine, n, k):
    """9-16 rows with a scale per chunk run the matrix-core GEMV with all 16
    B-operand rows (half segments of 2048 depths staged), 17-32 rows as one
    such launch per 16 rows: against the portable path, with an op-graph
    whose ROW and (padded) TENSOR operands must follow each launch's rows."""
    block = 32
    nbk = -(-k // block)
    rng = np.random.default_rng(m * 7 + n + k + bf16 + 2 * affine)
    cv = orc.f32_to_bf16 if bf16 else orc.f32_to_f16
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.002, 0.01, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.02, 0.02, n * nbk).astype(np.float32)) if affine else None
    a = cv(rng.uniform(-0.5, 0.5, m * k).astype(np.float32))
    row = cv(rng.uniform(-0.5, 0.5, m).astype(np.float32))
    ld = n + 3
    ten = cv(rng.uniform(-0.5, 0.5, m * ld).astype(np.float32))
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    got = np.zeros(m * n, np.uint16)
    fn = smg.matmul_q4_bf16_ep if bf16 else smg.matmul_q4_ep
    fn(a, w, got, m, smg.Epilogue(bf16=bf16).add_row(row).add_tensor(ten, ld).relu())
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, block,
                            [(2, 0, 0.0, row, 0), (6, 0, 0.0, ten, ld)], 1, bf16)
    assert max_rel(got, want, bf16) <= (bf16_tol(k) if bf16 else f16_tol(k))


@pytest.mark.parametrize("m", [1, 4, 20])
@pytest.mark.parametrize("affine", [False, True])
def test_q4_band_major_upload_matches_row_major(smg, orc, m, affine):
    """The reference's band-major resident arrays (what src/ffi.rs passes) give
    the same device weights as the public row-major input."""
    n, k, block = 300, 160, 32
    rng = np.random.default_rng(11)
    nbk = -(-k // block)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.1, 0.1, n * nbk).astype(np.float32)) if affine else None
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    nib, sc, mn = orc.q4_pack_band(quants, scales, mins, n, k, block)
    w1 = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    w2 = smg.Q4Weights.from_band(nib, sc, mn, n, k, p)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    c1 = np.zeros(m * n, np.uint16)
    c2 = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w1, c1, m)
    smg.matmul_q4(a, w2, c2, m)
    assert np.array_equal(c1, c2)


def test_q4_empty_shapes_leave_c_untouched(smg):
    """m == 0 or n == 0 returns at once (q4/matmul.rs:43-44)."""
    w = smg.Q4Weights(np.zeros(0, np.uint8), np.zeros(0, np.uint16), 0, 64)
    c = np.zeros(0, np.uint16)
    smg.matmul_q4(np.zeros(0, np.uint16), w, c, 0)
    w2 = smg.Q4Weights(np.zeros(64 * 8 // 2, np.uint8), np.full(16, 0x3C00, np.uint16), 8, 64)
    c2 = np.zeros(0, np.uint16)
    smg.matmul_q4(np.zeros(0, np.uint16), w2, c2, 0)


def test_q4_k_zero_gives_epilogue_of_zero(smg, orc):
    """k == 0: the product is the empty sum (+0), then the op-graph."""
    n = 40
    w = smg.Q4Weights(np.zeros(0, np.uint8), np.zeros(0, np.uint16), n, 0)
    bias = orc.f32_to_f16(np.linspace(-1, 1, n).astype(np.float32))
    c = np.full(2 * n, 0x7777, np.uint16)
    smg.matmul_q4_ep(np.zeros(0, np.uint16), w, c, 2, smg.Epilogue().add_col(bias))
    assert np.array_equal(c, np.concatenate([bias, bias]))


def test_q4_concurrent_callers_bit_identical(smg, orc):
    """tests/concurrency.rs:130: concurrent callers get identical bits."""
    m, n, k = 3, 1000, 1024
    rng = np.random.default_rng(5)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    w = smg.Q4Weights(quants, scales, n, k)
    ref = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w, ref, m)
    outs = [np.zeros(m * n, np.uint16) for _ in range(8)]
    errs = []

    def run(i):
        try:
            for _ in range(5):
                smg.matmul_q4(a, w, outs[i], m)
        except Exception as e:  # noqa: BLE001
            errs.append(e)

    ts = [threading.Thread(target=run, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs
    for o in outs:
        assert np.array_equal(o, ref)


# Prefill shapes whose 128 x 256 GEMM tiles fill fewer than half of the 256
# compute units, so K is split into slices (8 slices of 8 steps at 48 x 4096 x
# 4096; 8 at 130 x 1000 x 1024 with two row tiles; 8 uneven slices of 2 or 3
# steps at 200 x 1500 x 1472, N not a multiple of 8; 4 of 2 steps at 33 x 520
# x 512) and a second kernel adds them.
SPLIT_CASES = [(48, 4096, 4096), (130, 1000, 1024), (200, 1500, 1472), (256, 2304, 2048), (33, 520, 512)]


@pytest.mark.parametrize("m,n,k", SPLIT_CASES)
@pytest.mark.parametrize("affine", [False, True])
def test_q4_split_k_prefill(smg, orc, m, n, k, affine):
    """The split-K GEMM against the oracle with an op-graph of every operand
    class (ROW, COL, TENSOR, activation), bit-identical over repeated calls
    (the slices are added in a fixed order), and the device-pointer entry
    (its partials in the stream's pool) bit-identical to the host entry
    (its partials in the call's staging)."""
    import torch
    rng = np.random.default_rng(m * 7 + n + k + affine)
    nbk = k // 32
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.1, 0.0, n * nbk).astype(np.float32)) if affine else None
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    row = orc.f32_to_f16(rng.normal(0, 0.1, m).astype(np.float32))
    col = orc.f32_to_f16(rng.normal(0, 0.1, n).astype(np.float32))
    ten = orc.f32_to_f16(rng.normal(1, 0.1, m * n).astype(np.float32))
    p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    ep = smg.Epilogue().add_row(row).mul_tensor(ten).add_col(col).silu()
    got = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a, w, got, m, ep)
    nodes = [(2, 0, 0.0, row, 0), (7, 0, 0.0, ten, 0), (4, 0, 0.0, col, 0)]
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, 32, nodes, 3)
    assert max_rel(got, want) <= f16_tol(k), f"{m}x{n}x{k}"
    again = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a, w, again, m, ep)
    assert np.array_equal(again, got)
    dev = lambda x: torch.from_numpy(x.view(np.int16)).cuda()  # noqa: E731
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    smg.matmul_q4_ep(dev(a), w, cd, m, smg.Epilogue().add_row(dev(row)).mul_tensor(dev(ten))
                     .add_col(dev(col)).silu())
    torch.cuda.synchronize()
    assert np.array_equal(cd.cpu().numpy().view(np.uint16), got)


@pytest.mark.parametrize("m", [40, 100])
def test_q4_device_a_gemm_q4r_cannot_read(smg, orc, m):
    """An f16 device A that is not 16-byte aligned (a view one element into
    its buffer) cannot be read by the split-K GEMM's DMA, so the call runs on
    the 16-row GEMV launches or gemm_kernel -- and allocates no split-K
    partials for it -- with the same result as the aligned A, within the f16
    bar of the oracle."""
    import torch
    n, k = 1024, 4096
    rng = np.random.default_rng(m)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    w = smg.Q4Weights(quants, scales, n, k)
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32)
    buf = torch.zeros(m * k + 1, dtype=torch.int16, device="cuda")
    buf[1:] = torch.from_numpy(a.view(np.int16)).cuda()
    ad = buf[1:]
    assert ad.data_ptr() % 16 == 2
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    smg.matmul_q4(ad, w, cd, m)
    torch.cuda.synchronize()
    got = cd.cpu().numpy().view(np.uint16)
    assert max_rel(got, want) <= f16_tol(k)
    aligned = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    smg.matmul_q4(torch.from_numpy(a.view(np.int16)).cuda(), w, aligned, m)
    torch.cuda.synchronize()
    assert max_rel(aligned.cpu().numpy().view(np.uint16), want) <= f16_tol(k)


def test_q4_device_pointer_path_matches_host(smg, orc):
    """smg_q4_matmul_dev (torch tensors on the current stream) == host path."""
    import torch
    m, n, k = 2, 512, 1024
    rng = np.random.default_rng(9)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    bias = orc.f32_to_f16(rng.normal(0, 0.1, n).astype(np.float32))
    w = smg.Q4Weights(quants, scales, n, k)
    host = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a, w, host, m, smg.Epilogue().add_col(bias).silu())
    ad = torch.from_numpy(a.view(np.int16)).cuda()
    bd = torch.from_numpy(bias.view(np.int16)).cuda()
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    smg.matmul_q4_ep(ad, w, cd, m, smg.Epilogue().add_col(bd).silu())
    torch.cuda.synchronize()
    assert np.array_equal(cd.cpu().numpy().view(np.uint16), host)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("m,n,k,block", [(1, 96, 512, 32), (3, 70, 300, 64), (40, 33, 1000, 32)])
def test_quantize_then_matmul(smg, orc, layout, affine, m, n, k, block):
    """Q4Weights::quantize from f32 weights in either layout, uploaded and
    multiplied on the device, against the oracle over its own quantized arrays."""
    rng = np.random.default_rng(m * 7 + n + k + layout + 2 * affine)
    w = rng.standard_normal(n * k).astype(np.float32)
    x = w if layout == 0 else np.ascontiguousarray(w.reshape(n, k).T).ravel()
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    q = smg.Q4Weights.quantize(x, layout, n, k, p)
    quants, scales, mins = orc.q4_quantize(x, layout, n, k, block, affine)
    c = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, q, c, m)
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, block)
    assert max_rel(c, want) <= f16_tol(k)


@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("m", [1, 5, 40])
def test_q4_permute_columns(smg, orc, m, affine):
    """Q4Weights::permute_columns (weights.rs:125-163): output column j is
    column perm[j]; the permuted handle gives the permuted output of the
    original, bitwise, and matches the oracle over permuted arrays."""
    n, k, block = 300, 200, 32
    rng = np.random.default_rng(m + 2 * affine)
    w = rng.standard_normal(n * k).astype(np.float32)
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    q = smg.Q4Weights.quantize(w, 0, n, k, p)
    perm = rng.permutation(n)
    qp = q.permute_columns(perm)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    c = np.zeros(m * n, np.uint16)
    cp = np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, q, c, m)
    smg.matmul_q4(a, qp, cp, m)
    assert np.array_equal(cp.reshape(m, n), c.reshape(m, n)[:, perm])
    quants, scales, mins = orc.q4_quantize(w, 0, n, k, block, affine)
    nib = np.stack([quants & 15, quants >> 4], 1).ravel()[: n * k].reshape(k, n)[:, perm].ravel()
    pq = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    nbk = -(-k // block)
    ps = scales.reshape(n, nbk)[perm].ravel()
    pm = mins.reshape(n, nbk)[perm].ravel() if affine else None
    want = orc.matmul_q4_ep(a, pq, ps, pm, m, n, k, block)
    assert max_rel(cp, want) <= f16_tol(k)


def test_q4_permute_columns_rejects_bad_perm(smg):
    q = smg.Q4Weights.quantize(np.ones(64 * 8, np.float32), 0, 8, 64)
    with pytest.raises(smg.SmeGemmError, match="out of range"):
        q.permute_columns([0, 1, 2, 3, 4, 5, 6, 8])
    with pytest.raises(ValueError):
        q.permute_columns([0, 1])
