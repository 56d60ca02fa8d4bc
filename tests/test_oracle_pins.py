"""Pins for the CPU oracle (oracle/oracle.c): each restated function is
checked against something other than itself -- numpy / torch IEEE conversions,
closed forms, brute force with exact rational arithmetic, and the reference's
own known-answer invariants. CPU only."""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O


# ---- f16 / bf16 conversions (the `half` crate: IEEE RNE) ---------------------

def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _f16_midpoints():
    """Every midpoint between adjacent finite f16 values (exact in f32), and
    one f32 ulp either side."""
    pos = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (pos[:-1] + pos[1:]) / 2
    mids = np.concatenate([mids, -mids]).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(-np.inf))
    return np.concatenate([mids, up, dn])


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 1 << 21, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), _f16_midpoints(),
                        np.array([65504, 65519.99, 65520, 1e-8, 2.0**-25, 2.0**-24 * 1.5,
                                  np.inf, -np.inf], np.float32)])
    got = O.f32_to_f16(x)
    with np.errstate(over="ignore"):  # values past f16's range round to inf, as tested
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_f64_to_f16_is_one_direct_rounding():
    """half::f16::from_f64 rounds once: a value just above a midpoint must go
    up even when its nearest f32 is the midpoint itself."""
    mids = _f16_midpoints()[: (len(_f16_midpoints()) // 3)].astype(np.float64)
    eps = np.abs(mids) * 2.0**-40
    x = np.concatenate([mids + eps, mids - eps, mids])
    rng = np.random.default_rng(1)
    x = np.concatenate([x, rng.standard_normal(1 << 18) * 10.0 ** rng.integers(-9, 6, 1 << 18)])
    got = O.f64_to_f16(x)
    with np.errstate(over="ignore"):  # values past f16's range round to inf, as tested
        want = x.astype(np.float16).view(np.uint16)
        # the double-rounded (via f32) result differs on the +-eps cases
        via32 = x.astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert np.any(via32 != want)


def test_f32_to_bf16_matches_torch_rne():
    import torch
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2**16, 4096, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    x = np.concatenate([bits, ties]).view(np.float32)
    got = O.f32_to_bf16(x)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7F80) == 0x7F80)


# ---- Q4 dequant: closed form over every nibble -----------------------------

def test_q4_dequant_closed_form_all_nibbles():
    """w = RNE16(f64(scale) * code [+ f64(min)]), code = nib<8 ? nib : nib-16
    (q4/mod.rs:211-222), for all 16 nibbles and a sweep of scales (subnormal
    to large), both forms, f16 and bf16 (through f32: mod.rs:250-256)."""
    scales_f = np.concatenate([np.array([0.0, 6e-8, 3e-5, 6.1e-5], np.float64),
                               np.geomspace(1e-4, 4000, 200)])
    sc = scales_f.astype(np.float16).view(np.uint16)
    n, k = 16, len(sc)
    # row-major k x n: row d uses scale sc[d]; column j holds nibble j
    nib = np.tile(np.arange(16, dtype=np.uint8), k)
    quants = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    # scales[j*nbk + d/block] with block 1 -> scale index j*k + d
    scales = np.tile(sc, n)
    mins_f = np.linspace(-3, 3, n * k)
    mins = mins_f.astype(np.float16).view(np.uint16)
    code = np.where(np.arange(16) < 8, np.arange(16), np.arange(16) - 16).astype(np.float64)
    s64 = sc.view(np.float16).astype(np.float64)
    for mv in (None, mins):
        w = s64[:, None] * code[None, :]
        if mv is not None:
            w = w + mv.view(np.float16).astype(np.float64).reshape(n, k).T
        got = O.q4_dequant(quants, scales, mv, n, k, 1)
        assert np.array_equal(got, w.astype(np.float16).view(np.uint16).ravel())
        got_bf = O.q4_dequant(quants, scales, mv, n, k, 1, bf16=True)
        assert np.array_equal(got_bf, O.f32_to_bf16(w.astype(np.float32).ravel()))


def _band_q4_reader(nib, sc, n, k, block):
    """Independent reader of the reference's band-major Q4 layout
    (q4/weights.rs:89-113)."""
    nbk = -(-k // block)
    codes = np.zeros((k, n), np.int64)
    scales = np.zeros((n, nbk), np.uint16)
    for j in range(n):
        b, c = divmod(j, 128)
        for d in range(k):
            byte = nib[b * k * 64 + d * 64 + c // 2]
            codes[d, j] = (byte >> (4 * (c % 2))) & 15
        for blk in range(nbk):
            scales[j, blk] = sc[b * nbk * 128 + blk * 128 + c]
    return codes, scales


@pytest.mark.parametrize("n,k,block", [(33, 96, 16), (64, 64, 32), (17, 130, 64), (130, 32, 128)])
def test_q4_band_pack_round_trip(n, k, block):
    """weights.rs:315: the band-major pack keeps every nibble and scale."""
    rng = np.random.default_rng(n + k)
    nbk = -(-k // block)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = rng.integers(0, 0x7C00, n * nbk).astype(np.uint16)
    nib, sc, _ = O.q4_pack_band(quants, scales, None, n, k, block)
    codes, sback = _band_q4_reader(nib, sc, n, k, block)
    flat = np.stack([quants & 15, quants >> 4], 1).ravel()[: k * n].reshape(k, n)
    assert np.array_equal(codes, flat)
    assert np.array_equal(sback.ravel(), scales)


def test_q4_affine_zero_mins_equals_scale():
    """weights.rs:359: Affine with all-zero mins == Scale, bitwise."""
    rng = np.random.default_rng(3)
    n, k = 40, 96
    quants = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
    scales = rng.uniform(0.001, 0.1, n * 3).astype(np.float16).view(np.uint16)
    a = O.q4_dequant(quants, scales, None, n, k, 32)
    b = O.q4_dequant(quants, scales, np.zeros(n * 3, np.uint16), n, k, 32)
    assert np.array_equal(a, b)


# ---- reference GEMM -------------------------------------------------------------

def _numpy_gemm16(a, b, m, n, k, bf16=False, beta=1.0):
    """Independent restatement of reference::gemm_f16: per row, a float32
    accumulator updated in K order (numpy float32 ops are IEEE, no fusion)."""
    to32 = O.bf16_to_f32 if bf16 else (lambda h: np.asarray(h, np.uint16).view(np.float16)
                                       .astype(np.float32))
    A = to32(a).reshape(m, k)
    B = to32(b).reshape(k, n)
    out = np.zeros((m, n), np.float32)
    for i in range(m):
        acc = np.zeros(n, np.float32)
        for l in range(k):
            acc = acc + A[i, l] * B[l]
        out[i] = np.float32(0.0) + np.float32(beta) * acc
    return O.f32_to_bf16(out.ravel()) if bf16 else out.ravel().astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 5, 3), (31, 31, 31), (33, 17, 9), (5, 40, 130)])
@pytest.mark.parametrize("bf16", [False, True])
def test_gemm16_brute_force(m, n, k, bf16):
    rng = np.random.default_rng(m * 100 + n + k)
    cv = O.f32_to_bf16 if bf16 else O.f32_to_f16
    a = cv(rng.standard_normal(m * k).astype(np.float32))
    b = cv(rng.standard_normal(k * n).astype(np.float32))
    assert np.array_equal(O.gemm16(a, b, m, n, k, bf16=bf16), _numpy_gemm16(a, b, m, n, k, bf16))
    beta_bits = int(cv(np.float32(0.75))[0])
    assert np.array_equal(O.gemm16(a, b, m, n, k, beta_bits, bf16=bf16),
                          _numpy_gemm16(a, b, m, n, k, bf16, 0.75))


def test_gemm16_closed_forms():
    """All-ones A gives exact column sums of small-integer B; k = 0 gives +0;
    col_major output is the transpose of row-major."""
    m, n, k = 3, 20, 50
    rng = np.random.default_rng(4)
    bi = rng.integers(-5, 6, k * n)
    b = bi.astype(np.float16).view(np.uint16)
    a = np.full(m * k, 0x3C00, np.uint16)
    got = O.gemm16(a, b, m, n, k).view(np.float16).astype(np.int64).reshape(m, n)
    assert np.array_equal(got, np.tile(bi.reshape(k, n).sum(0), (m, 1)))
    assert np.array_equal(O.gemm16(np.zeros(0, np.uint16), np.zeros(0, np.uint16), 2, 5, 0),
                          np.zeros(10, np.uint16))
    a2 = rng.standard_normal(m * k).astype(np.float16).view(np.uint16)
    rm = O.gemm16(a2, b, m, n, k).reshape(m, n)
    cm = O.gemm16(a2, b, m, n, k, col_major=True).reshape(n, m)
    assert np.array_equal(rm, cm.T)


def _strided_layout(x, rows, cols, layout, rng):
    """x (rows x cols, row-major uint16) laid out row-major, column-major or
    row-major with padded rows: (buffer, row stride, col stride). Padding
    cells hold NaN bits so a read of one shows in the result."""
    x = np.asarray(x, np.uint16).reshape(rows, cols)
    if layout == "row":
        return x.ravel().copy(), cols, 1
    if layout == "col":
        return x.T.ravel().copy(), 1, rows
    ld = cols + 3
    buf = np.full(rows * ld, 0x7E00, np.uint16)
    buf.reshape(rows, ld)[:, :cols] = x
    return buf, ld, 1


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("la,lb,lc", [("row", "row", "row"), ("col", "col", "col"), ("pad", "col", "pad"),
                                      ("row", "pad", "col")])
def test_gemm_strided_pins(bf16, la, lb, lc):
    """or_gemm_strided against an independent numpy restatement on
    materialized row-major operands (f32 K-order accumulator, then
    alpha * C + beta * acc rounded once): layout-independent, alpha = 0 never
    reads C (NaN there does not show), C's padding cells are left alone."""
    m, n, k = 6, 9, 13
    rng = np.random.default_rng(hash((bf16, la, lb, lc)) % 2**32)
    cv = O.f32_to_bf16 if bf16 else O.f32_to_f16
    to32 = O.bf16_to_f32 if bf16 else O.f16_to_f32
    a = cv(rng.standard_normal(m * k).astype(np.float32))
    b = cv(rng.standard_normal(k * n).astype(np.float32))
    c0 = cv(rng.standard_normal(m * n).astype(np.float32))
    A, B, C0 = (to32(v).reshape(r, q) for v, r, q in ((a, m, k), (b, k, n), (c0, m, n)))
    for alpha, beta in ((0.0, 1.0), (0.5, -2.0), (1.0, 0.25)):
        ab, bb = int(cv(np.float32(alpha))[0]), int(cv(np.float32(beta))[0])
        acc = np.zeros((m, n), np.float32)
        for l in range(k):
            acc = acc + A[:, l:l + 1] * B[l]
        prev = np.float32(alpha) * C0 if alpha != 0.0 else np.zeros((m, n), np.float32)
        want = cv((prev + np.float32(beta) * acc).ravel())
        abuf, ars, acs = _strided_layout(a, m, k, la, rng)
        bbuf, brs, bcs = _strided_layout(b, k, n, lb, rng)
        cin = c0 if alpha != 0.0 else np.full(m * n, 0x7E00, np.uint16)
        cbuf, crs, ccs = _strided_layout(cin, m, n, lc, rng)
        got = O.gemm_strided(cbuf, crs, ccs, abuf, ars, acs, bbuf, brs, bcs, m, n, k, ab, bb, bf16)
        cells = np.array([[got[i * crs + j * ccs] for j in range(n)] for i in range(m)]).ravel()
        assert np.array_equal(cells, want), (alpha, beta)
        if lc == "pad":
            assert np.all(got.reshape(m, crs)[:, n:] == 0x7E00)


def test_gemm_strided_closed_forms():
    """k = 0 leaves T(alpha * C) (an empty sum); alpha = 1, beta = 0 keeps C
    exactly; all-ones A over small-integer B gives exact column sums."""
    m, n = 4, 7
    rng = np.random.default_rng(8)
    c0 = O.f32_to_f16(rng.standard_normal(m * n).astype(np.float32))
    half = int(O.f32_to_f16(np.float32(0.5))[0])
    got = O.gemm_strided(c0, n, 1, np.zeros(0, np.uint16), 0, 1, np.zeros(0, np.uint16), n, 1, m, n, 0,
                         half, 0x3C00)
    assert np.array_equal(got, O.f32_to_f16(np.float32(0.5) * O.f16_to_f32(c0)))
    k = 11
    a = O.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    b = O.f32_to_f16(rng.standard_normal(k * n).astype(np.float32))
    assert np.array_equal(O.gemm_strided(c0, n, 1, a, k, 1, b, n, 1, m, n, k, 0x3C00, 0), c0)
    bi = rng.integers(-4, 5, k * n)
    ones = np.full(m * k, 0x3C00, np.uint16)
    got = O.gemm_strided(np.zeros(m * n, np.uint16), n, 1, ones, k, 1, bi.astype(np.float16).view(np.uint16),
                         n, 1, m, n, k, 0, 0x3C00)
    assert np.array_equal(got.view(np.float16).astype(np.int64).reshape(m, n),
                          np.tile(bi.reshape(k, n).sum(0), (m, 1)))


# ---- epilogue ----------------------------------------------------------------------

def _maxnum(x, y):
    """IEEE 754-2019 maximumNumber: NaN loses, -0 < +0."""
    import math
    if math.isnan(x):
        return y
    if math.isnan(y):
        return x
    if x == 0 and y == 0:
        return -0.0 if (math.copysign(1, x) < 0 and math.copysign(1, y) < 0) else 0.0
    return x if x > y else y


def _minnum(x, y):
    import math
    if math.isnan(x):
        return y
    if math.isnan(y):
        return x
    if x == 0 and y == 0:
        return -0.0 if (math.copysign(1, x) < 0 or math.copysign(1, y) < 0) else 0.0
    return x if x < y else y


def test_maxnum_minnum_zero_signs():
    """max(-0, +0) = +0 and min(-0, +0) = -0 in the op-graph (MAX/MIN nodes)."""
    c = np.array([0x8000, 0x0000, 0x8000, 0x7E00], np.uint16)  # -0, +0, -0, NaN
    got = O.apply_ep(c, 1, 4, [(9, 0, 0.0, None, 0)], None)
    assert list(got) == [0x0000, 0x0000, 0x0000, 0x0000]
    got = O.apply_ep(c, 1, 4, [(10, 0, 0.0, None, 0)], None)
    assert list(got) == [0x8000, 0x0000, 0x8000, 0x0000]
    got = O.apply_ep(c, 1, 4, [(10, 0, -0.0, None, 0)], None)
    assert list(got) == [0x8000, 0x8000, 0x8000, 0x8000]


def _np_act(kind, x, alpha=0.0):
    """act_apply_f64_a (src/epilogue/mod.rs:40-84), written against numpy f64."""
    import math
    x = float(x)
    if kind == 1: return _maxnum(x, 0.0)
    if kind == 2: return 0.5 * x * (1.0 + math.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)))
    if kind == 3: return x / (1.0 + math.exp(-x))
    if kind == 4: return math.tanh(x)
    if kind == 5: return 1.0 / (1.0 + math.exp(-x))
    if kind == 6: return x if x >= 0 else alpha * x
    if kind == 7: return min(max(x, 0.0), 6.0)
    if kind == 8: return min(max(x / 6.0 + 0.5, 0.0), 1.0)
    if kind == 9: return x * min(max(x / 6.0 + 0.5, 0.0), 1.0)
    if kind == 10: return abs(x)
    if kind == 11: return -x
    if kind == 12: return x * x
    if kind == 13: return 1.0 if x > 0 else (-1.0 if x < 0 else 0.0)
    if kind == 14: return math.sqrt(x) if x >= 0 else math.nan
    if kind == 15: return x / (1.0 + abs(x))
    if kind == 16: return 1.0 / x if x != 0 else math.copysign(math.inf, x)
    if kind == 17:  # sqrt(-0) = -0, so 1/sqrt(-0) = -inf
        return 1.0 / math.sqrt(x) if x > 0 else (math.copysign(math.inf, x) if x == 0 else math.nan)
    if kind == 18: return math.exp(x)
    if kind == 19: return math.log(x) if x > 0 else (-math.inf if x == 0 else math.nan)
    if kind == 20: return x if x >= 0 else alpha * math.expm1(x)
    if kind == 21: return 1.0507009873554805 * (x if x >= 0 else 1.6732632423543772 * math.expm1(x))
    if kind == 22: return _maxnum(x, 0.0) + math.log1p(math.exp(-abs(x)))
    if kind == 23: return x * math.tanh(_maxnum(x, 0.0) + math.log1p(math.exp(-abs(x))))
    if kind == 24:
        xe = x * 0.7071067811865476
        ax = abs(xe)
        t = 1.0 / (1.0 + 0.3275911 * ax)
        poly = ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t
                + 0.254829592) * t
        e = 1.0 - poly * math.exp(-ax * ax)
        return 0.5 * x * (1.0 + (-e if xe < 0 else e))
    return x


@pytest.mark.parametrize("kind", range(1, 25))
def test_activation_table(kind):
    xs = np.concatenate([np.linspace(-9, 9, 181), [0.0, -0.0, 1e-3, -1e-3, 30.0, -30.0]])
    xs = xs.astype(np.float32)
    got = O.act_f32(kind, xs, 0.3)
    want = np.array([np.float32(_np_act(kind, float(x), float(np.float32(0.3)))) for x in xs],
                    np.float32)
    both_nan = np.isnan(got) & np.isnan(want)
    assert np.array_equal(got[~both_nan].view(np.uint32), want[~both_nan].view(np.uint32))


def test_epilogue_nodes_closed_form():
    """ep_apply_cell (src/exec/scalar.rs:58-123): each node in order, in f32,
    on the f16-rounded product; trailing act last; IEEE maxNum/minNum."""
    m, n = 4, 6
    rng = np.random.default_rng(5)
    c = rng.uniform(-2, 2, m * n).astype(np.float16).view(np.uint16)
    row = rng.uniform(0.5, 2, m).astype(np.float16).view(np.uint16)
    col = rng.uniform(0.5, 2, n).astype(np.float16).view(np.uint16)
    ten = rng.uniform(-1, 1, m * (n + 2)).astype(np.float16).view(np.uint16)
    f = lambda h: np.asarray(h).view(np.float16).astype(np.float32)  # noqa: E731
    nodes = [(0, 0, 0.5, None, 0), (1, 0, 1.5, None, 0), (2, 0, 0.0, row, 0),
             (3, 0, 0.0, row, 0), (4, 0, 0.0, col, 0), (5, 0, 0.0, col, 0),
             (6, 0, 0.0, ten, n + 2), (7, 0, 0.0, ten, n + 2), (9, 0, -1.0, None, 0),
             (10, 0, 3.0, None, 0), (11, 0, 0.25, None, 0), (12, 0, 0.0, row, 0),
             (13, 0, 0.0, col, 0), (14, 0, 0.0, ten, n + 2), (15, 0, 2.0, None, 0),
             (16, 0, 0.0, row, 0), (17, 0, 0.0, col, 0), (18, 0, 0.0, ten, n + 2),
             (19, 0, 0.0, row, 0), (20, 0, 0.0, col, 0), (21, 0, 0.0, ten, n + 2),
             (22, 0, 0.0, row, 0), (23, 0, 0.0, col, 0), (24, 0, 0.0, ten, n + 2)]
    got = O.apply_ep(c, m, n, nodes, 3)
    want = np.empty(m * n, np.uint16)
    for i in range(m):
        for j in range(n):
            x = f(c[i * n + j])
            r, cc, t = f(row[i]), f(col[j]), f(ten[i * (n + 2) + j])
            x = x + np.float32(0.5); x = x * np.float32(1.5); x = x + r; x = x * r
            x = x + cc; x = x * cc; x = x + t; x = x * t
            mx = lambda u, v: np.float32(_maxnum(float(u), float(v)))  # noqa: E731
            mn = lambda u, v: np.float32(_minnum(float(u), float(v)))  # noqa: E731
            x = mx(x, np.float32(-1.0)); x = mn(x, np.float32(3.0))
            x = x - np.float32(0.25); x = x - r; x = x - cc; x = x - t
            x = x / np.float32(2.0); x = x / r; x = x / cc; x = x / t
            x = mx(x, r); x = mx(x, cc); x = mx(x, t)
            x = mn(x, r); x = mn(x, cc); x = mn(x, t)
            x = np.float32(_np_act(3, float(x)))
            want[i * n + j] = np.float32(x).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- low-bit quantize_row and reference ----------------------------------------------

def _np_quantize_row(a, k, block):
    """quantize_row (matmul.rs:354-371) in numpy float32."""
    x = np.asarray(a, np.uint16).view(np.float16).astype(np.float32)
    nbk = -(-k // block)
    q = np.zeros(k, np.int8)
    s = np.zeros(nbk, np.float32)
    for b in range(nbk):
        seg = x[b * block:(b + 1) * block]
        amax = np.float32(np.nan) if np.isnan(seg).any() else np.float32(np.max(np.abs(seg)))
        inv = np.float32(127.0) / amax if amax > 0 else np.float32(0.0)
        s[b] = amax / np.float32(127.0)
        with np.errstate(invalid="ignore"):
            r = np.rint(seg * np.float32(inv))
        r = np.where(np.isnan(r), 0, np.clip(r, -128, 127))
        q[b * block:(b + 1) * block] = r.astype(np.int8)
    return q, s


@pytest.mark.parametrize("k,block", [(1, 16), (37, 16), (300, 64), (513, 128), (256, 256)])
def test_quantize_row_matches_numpy(k, block):
    rng = np.random.default_rng(k + block)
    a = (rng.standard_normal(k) * 3).astype(np.float16).view(np.uint16)
    q, s = O.quantize_row(a, k, block)
    qn, sn = _np_quantize_row(a, k, block)
    assert np.array_equal(q, qn) and np.array_equal(s.view(np.uint32), sn.view(np.uint32))


def test_quantize_row_special_values():
    """NaN anywhere in a block: scale NaN, codes 0; inf: inv 0; all zero: 0."""
    a = np.zeros(48, np.float16)
    a[3] = np.nan
    a[16 + 5] = np.inf
    a[16 + 6] = 2.0
    q, s = O.quantize_row(a.view(np.uint16), 48, 16)
    assert np.isnan(s[0]) and np.all(q[:16] == 0)
    assert np.isinf(s[1]) and np.all(q[16:32] == 0)
    assert s[2] == 0 and np.all(q[32:] == 0)


def _round_f32(fr: Fraction) -> np.float32:
    """Exact rational -> nearest f32 (ties to even)."""
    x = np.float32(float(fr))
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - fr)
        key = (d, int(np.float32(c).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def _values(kind, codes, n, k, codebook=(-1, 0, 1, 0), inout=False):
    v = np.zeros((k, n), np.int64)
    for d in range(k):
        for j in range(n):
            if kind == 2:
                idx = d * n + j
                v[d, j] = codebook[(codes[idx // 4] >> (2 * (idx % 4))) & 3]
            else:
                idx = d * n + j if inout else j * k + d
                v[d, j] = 1 if (codes[idx // 8] >> (idx % 8)) & 1 else -1
    return v


def _scale_sweep():
    """f16 scales across the range: subnormals, the smallest normals, the
    config ranges, and values whose product with an int8 overflows f16."""
    fixed = [0x0001, 0x0003, 0x03FF, 0x0400, 0x0401, 0x1400, 0x2000, 0x211F, 0x2A8F, 0x3C00,
             0x3C01, 0x4B00, 0x5800, 0x5BFF, 0x7000, 0x7BFF]
    rng = np.random.default_rng(77)
    rand = rng.integers(1, 0x7C00, 48, dtype=np.int64).tolist()
    s = np.array(fixed + rand, np.uint16)
    return np.concatenate([s, s | 0x8000])  # and every one negated


@pytest.mark.parametrize("kind,inout,cb", [(2, False, (-1, 0, 1, 0)), (2, False, (-128, -3, 5, 127)),
                                           (1, False, None), (1, True, None)])
def test_lowbit_dequant_closed_form(kind, inout, cb):
    """Codes::dequant (matmul.rs:178-197), the MOPA route's f16 weights, against
    its closed form: f16_RNE(scale * codebook[code]) for Q2 (an f16 scale times
    an int8 is exact in f64, so numpy's one f64 -> f16 rounding is the
    reference's one rounding of the exact product) and +scale / -scale for Q1
    (set bit = +). Every code (all 4 Q2 codes, both signs) meets every scale of
    a sweep, in both Q1 layouts; the codes are read by this file's own reader."""
    sweep = _scale_sweep()
    n = sweep.size                  # one column per scale value
    block = 16
    k = 64                          # 4 blocks: each column's blocks share its scale
    nbk = k // block
    scales = np.repeat(sweep, nbk)  # scales[j*nbk + b] = sweep[j]
    rng = np.random.default_rng(kind * 10 + inout)
    if kind == 2:
        # depth d of column j holds code (d + j) % 4: every code in every column
        codes = np.zeros((k * n + 3) // 4, np.uint8)
        for d in range(k):
            for j in range(n):
                idx = d * n + j
                codes[idx // 4] |= ((d + j) % 4) << (2 * (idx % 4))
    else:
        codes = rng.integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
    cbk = cb if cb is not None else (-1, 0, 1, 0)
    got = O.lowbit_dequant(kind, codes, scales, n, k, block, cbk, inout).reshape(k, n)
    vals = _values(kind, codes, n, k, cbk, inout)
    s64 = sweep.view(np.float16).astype(np.float64)
    if kind == 2:
        with np.errstate(over="ignore"):  # large scales times 127 round to +-inf, as in f16
            want = (s64[None, :] * vals.astype(np.float64)).astype(np.float16).view(np.uint16)
    else:
        want = np.where(vals > 0, sweep[None, :], sweep[None, :] ^ np.uint16(0x8000)).astype(np.uint16)
    assert np.array_equal(got, want)
    if kind == 2:
        assert set(np.unique((np.arange(k)[:, None] + np.arange(n)[None, :]) % 4)) == {0, 1, 2, 3}
    else:
        assert (vals > 0).any() and (vals < 0).any()


def test_lowbit_dequant_planted_mistakes_are_caught():
    """The closed form above would catch the plausible mistakes: a sign-bit
    flip (Q1 set bit = -scale), a transposed codebook, or rounding through
    bf16; each is planted on the CPU copy and must differ somewhere."""
    sweep = _scale_sweep()[:32]
    n, k, block = sweep.size, 16, 16
    codes = np.zeros((k * n + 3) // 4, np.uint8)
    for d in range(k):
        for j in range(n):
            idx = d * n + j
            codes[idx // 4] |= ((d + j) % 4) << (2 * (idx % 4))
    good = O.lowbit_dequant(2, codes, sweep, n, k, block, (-2, -1, 1, 2)).reshape(k, n)
    swapped = O.lowbit_dequant(2, codes, sweep, n, k, block, (2, 1, -1, -2)).reshape(k, n)
    assert not np.array_equal(good, swapped)
    s32 = sweep.view(np.float16).astype(np.float32)
    vals = _values(2, codes, n, k, (-2, -1, 1, 2)).astype(np.float32)
    via_bf16 = O.f32_to_f16(O.bf16_to_f32(O.f32_to_bf16((s32[None, :] * vals).ravel())))
    assert not np.array_equal(good.ravel(), via_bf16)
    signs = np.random.default_rng(3).integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
    q1 = O.lowbit_dequant(1, signs, sweep, n, k, block).reshape(k, n)
    flipped = O.lowbit_dequant(1, signs ^ np.uint8(0xFF), sweep, n, k, block).reshape(k, n)
    assert np.array_equal(q1 ^ np.uint16(0x8000), flipped)


@pytest.mark.parametrize("kind", [2, 1])
@pytest.mark.parametrize("m,n,k,block", [(1, 7, 37, 16), (2, 5, 200, 64), (3, 4, 130, 128)])
def test_lowbit_reference_exact_rational(kind, m, n, k, block):
    """reference (matmul.rs:376-398) with the fused fold done in exact rational
    arithmetic: total = RNE32(f*(RNE32(scale*s)) + total)."""
    rng = np.random.default_rng(kind * 1000 + m + n + k)
    a = (rng.standard_normal(m * k)).astype(np.float16).view(np.uint16)
    nbk = -(-k // block)
    scales = rng.uniform(0.01, 0.05, n * nbk).astype(np.float16).view(np.uint16)
    cb = (-2, -1, 1, 2)
    codes = rng.integers(0, 256, (k * n + 3) // 4 if kind == 2 else (k * n + 7) // 8,
                         dtype=np.uint8)
    got = O.lowbit_reference(kind, a, codes, scales, m, n, k, block, cb)
    vals = _values(kind, codes, n, k, cb)
    sc = scales.view(np.float16).astype(np.float32)
    want = np.zeros(m * n, np.uint16)
    for i in range(m):
        q, s = _np_quantize_row(a[i * k:(i + 1) * k], k, block)
        for j in range(n):
            total = np.float32(0.0)
            for b in range(nbk):
                ssum = int(np.dot(q[b * block:(b + 1) * block].astype(np.int64),
                                  vals[b * block:(b + 1) * block, j]))
                f = np.float32(ssum)
                p = sc[j * nbk + b] * s[b]  # float32 product, rounded once
                total = _round_f32(Fraction(float(f)) * Fraction(float(p)) +
                                   Fraction(float(total)))
            want[i * n + j] = np.float32(total).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


SIZES = [(1, 1, 1), (7, 5, 3), (31, 31, 31), (32, 32, 32), (33, 17, 9), (64, 96, 48),
         (40, 8, 7), (7, 50, 200)]


@pytest.mark.parametrize("m,n,k", SIZES)
@pytest.mark.parametrize("block,cb", [(256, (-1, 0, 1, 0)), (32, (-2, -1, 1, 2))])
def test_q2_activation_rounding_bound(m, n, k, block, cb):
    """tests/correctness/q2.rs:39-77: |c - exact| <= sum_d |w| * amax/254 * 1.001
    + |exact|/1024 + 1e-6, with the reference's own data generators."""
    s = 0x0202_9401_DEAD_0001 ^ (m * 131 + n * 17 + k + block)
    nbk = -(-k // block)
    codes = O.lcg_bytes(s, (k * n + 3) // 4)
    for _ in range((k * n + 3) // 4):
        s = (s * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
    sb = O.lcg_bytes(s, n * nbk)
    for _ in range(n * nbk):
        s = (s * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
    scales = O.f32_to_f16(np.float32(0.005) + sb.astype(np.float32) * np.float32(1e-4))
    a, _ = O.lcg_fill(s, m * k)
    c = O.lowbit_reference(2, a, codes, scales, m, n, k, block, cb)
    vals = _values(2, codes, n, k, cb)
    w = vals * scales.view(np.float16).astype(np.float64).reshape(n, nbk).T[
        np.arange(k) // block]
    af = a.view(np.float16).astype(np.float64).reshape(m, k)
    for i in range(m):
        amax = np.array([np.max(np.abs(af[i, b * block:(b + 1) * block])) for b in range(nbk)])
        exact = af[i] @ w
        bound = (np.abs(w) * (amax[np.arange(k) // block] / 254.0)[:, None]).sum(0)
        got = c[i * n:(i + 1) * n].view(np.float16).astype(np.float64)
        tol = bound * 1.001 + np.abs(exact) / 1024.0 + 1e-6
        assert np.all(np.abs(got - exact) <= tol)


def test_lowbit_rows_are_independent():
    """Results depend only on their row (ARCHITECTURE.md:511-514)."""
    rng = np.random.default_rng(6)
    m, n, k = 5, 9, 100
    a = rng.standard_normal(m * k).astype(np.float16).view(np.uint16)
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = rng.uniform(0.01, 0.05, n * 2).astype(np.float16).view(np.uint16)
    full = O.lowbit_reference(2, a, codes, scales, m, n, k, 64)
    for i in range(m):
        one = O.lowbit_reference(2, a[i * k:(i + 1) * k], codes, scales, 1, n, k, 64)
        assert np.array_equal(one, full[i * n:(i + 1) * n])


def _lb_scale_index(sc_per_band, blk, j):
    c = j % 64
    return (j // 64) * sc_per_band + blk * 64 + (c // 32) * 32 + 2 * (c % 16) + (c % 32) // 16


@pytest.mark.parametrize("n,k,block", [(1, 1, 16), (65, 37, 16), (130, 300, 256)])
def test_lowbit_band_pack_round_trips(n, k, block):
    """q2.rs:197 / q1.rs:245: the band-major packs keep every code, sign and
    scale where code()/sign()/scale() read them."""
    nbk = -(-k // block)
    codes = (np.arange((k * n + 3) // 4) * 37 % 251).astype(np.uint8)
    signs = (np.arange((k * n + 7) // 8) * 37 % 251).astype(np.uint8)
    scales = (np.arange(n * nbk, dtype=np.float32) * 0.5).astype(np.float16).view(np.uint16)
    kp = -(-k // 16) * 16
    p2, s2 = O.lowbit_pack_band(2, codes, scales, n, k, block)
    for d in range(k):
        for j in range(n):
            idx = d * n + j
            want = (codes[idx // 4] >> (2 * (idx % 4))) & 3
            got = (p2[(j // 64) * kp * 16 + (d // 4) * 64 + j % 64] >> (2 * (d % 4))) & 3
            assert got == want
    for j in range(n):
        for b in range(nbk):
            assert s2[_lb_scale_index(nbk * 64, b, j)] == scales[j * nbk + b]
    for inout in (False, True):
        p1, s1 = O.lowbit_pack_band(1, signs, scales, n, k, block, inout)
        for j in range(n):
            for d in range(k):
                idx = d * n + j if inout else j * k + d
                want = (signs[idx // 8] >> (idx % 8)) & 1
                c = j % 64
                byte = (j // 64) * kp * 8 + (d // 4) * 32 + c // 2
                got = (p1[byte] >> (4 * (c % 2) + d % 4)) & 1
                assert got == want


def test_lcg_generators_match_reference_formula():
    """data()/fill() of the reference tests (matmul.rs:409-417, main.rs:36-46)."""
    s = 7
    bytes_ = O.lcg_bytes(7, 3)
    for i in range(3):
        s = (s * 6364136223846793005 + 1) % 2**64
        assert bytes_[i] == (s >> 40) & 0xFF
    vals, _ = O.lcg_fill(1, 2)
    s = (1 * 6364136223846793005 + 1442695040888963407) % 2**64
    assert vals[0] == np.float16(np.float32(s >> 40) / np.float32(2**24) - np.float32(0.5)) \
        .view(np.uint16)


@pytest.mark.parametrize("kind", [4, 2, 1])
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_threaded_baseline_is_the_single_threaded_path(kind, threads):
    """The CPU baseline's threaded mode splits columns over host threads; each
    output keeps its own arithmetic, so the bits equal the single-threaded
    oracle's."""
    rng = np.random.default_rng(kind * 10 + threads)
    m, n, k = 3, 131, 200
    a = rng.standard_normal(m * k).astype(np.float16).view(np.uint16)
    if kind == 4:
        codes = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
        scales = rng.uniform(0.005, 0.02, n * -(-k // 32)).astype(np.float16).view(np.uint16)
        want = O.matmul_q4_ep(a, codes, scales, None, m, n, k, 32)
        block = 32
    else:
        block = 64
        codes = rng.integers(0, 256, (k * n + (3 if kind == 2 else 7)) // (4 if kind == 2 else 8),
                             dtype=np.uint8)
        scales = rng.uniform(0.01, 0.05, n * -(-k // block)).astype(np.float16).view(np.uint16)
        want = O.lowbit_reference(kind, a, codes, scales, m, n, k, block)
    got = O.matmul_mt(kind, a, codes, scales, m, n, k, block, threads)
    assert np.array_equal(got, want)
