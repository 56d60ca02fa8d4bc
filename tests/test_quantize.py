"""Load-time quantizers (smg_q4_quantize / smg_q2_quantize / smg_q1_quantize):
host code in the product library, compared bit-exactly with the oracle's
restatement; the oracle itself is pinned by the reference's own quantizer tests
(src/kernels/q4/quantize.rs:99-134, src/kernels/lowbit/q2.rs:225-262,
src/kernels/lowbit/q1.rs:278-296) and by properties that do not restate the
formulas (argmin over the codebook, the block mean, the sign of each weight).
No device is touched: these run on the CPU."""
import numpy as np
import pytest

import oracle as O
import smegemm as S

OUT_IN, IN_OUT = S.WeightLayout.OutIn, S.WeightLayout.InOut


def _transpose(w, n, k):
    """The same weights in WeightLayout::InOut (k x n row-major)."""
    return np.ascontiguousarray(np.asarray(w, np.float32).reshape(n, k).T).ravel()


def _ref_weights(n, k):
    """quantize.rs:89-93: ((i * 2654435761) % 1000) / 500 - 1."""
    i = np.arange(n * k, dtype=np.uint64)
    return ((i * np.uint64(2_654_435_761)) % np.uint64(1000)).astype(np.float32) / np.float32(500.0) \
        - np.float32(1.0)


def _f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def _nibble_codes(quants, n, k):
    """Signed Q4 codes at idx = d * n + j (two per byte, low nibble first)."""
    q = np.asarray(quants, np.uint8)
    lo = (q & 0x0F).astype(np.int8)
    hi = (q >> 4).astype(np.int8)
    c = np.stack([lo, hi], 1).ravel()[: n * k]
    return np.where(c >= 8, c - 16, c).reshape(k, n)


def _q2_codes(codes, n, k):
    c = np.asarray(codes, np.uint8)
    return np.stack([(c >> s) & 3 for s in (0, 2, 4, 6)], 1).ravel()[: n * k].reshape(k, n)


def _q1_signs(signs, n, k):
    s = np.asarray(signs, np.uint8)
    return np.unpackbits(s, bitorder="little")[: n * k].reshape(n, k).astype(bool)


def _inputs(rng, n, k):
    w = rng.standard_normal(n * k).astype(np.float32)
    w[rng.random(n * k) < 0.02] = 0.0
    w[: min(k, 40)] = 0.0  # an all-zero block: scale 0, codes 0
    if n > 2:  # ties in magnitude: the first of equals decides the Q4_0 scale sign
        w[k + 3] = 2.5
        w[k + 7] = -2.5
    return w


SHAPES = [(1, 1, 32), (3, 17, 16), (33, 64, 32), (40, 100, 32), (7, 300, 64), (64, 1000, 128),
          (5, 4096, 256), (129, 70, 2048)]


# ---- Q4 ------------------------------------------------------------------------

@pytest.mark.parametrize("n,k,block", SHAPES)
@pytest.mark.parametrize("affine", [False, True])
def test_q4_library_matches_oracle(n, k, block, affine):
    rng = np.random.default_rng(n * 1000 + k)
    w = _inputs(rng, n, k)
    p = S.Q4Params(block).affine() if affine else S.Q4Params(block)
    for layout, x in ((OUT_IN, w), (IN_OUT, _transpose(w, n, k))):
        got = S.quantize_q4_arrays(x, layout, n, k, p)
        want = O.q4_quantize(x, layout, n, k, block, affine)
        assert np.array_equal(got[0], want[0]), f"quants {layout}"
        assert np.array_equal(got[1], want[1]), f"scales {layout}"
        if affine:
            assert np.array_equal(got[2], want[2]), f"mins {layout}"
        else:
            assert got[2] is None


@pytest.mark.parametrize("n,k,block", [(33, 64, 32), (40, 100, 32), (8, 96, 64)])
@pytest.mark.parametrize("affine", [False, True])
def test_q4_round_trip_within_half_a_step(n, k, block, affine):
    """quantize.rs:99-134 on the oracle and the library: both layouts
    dequantize identically, and every weight is within half a step of its
    block (a full step for Q4_0, whose code 7 sits opposite the largest
    magnitude) plus 0.01 for the f16 rounding of scale and min."""
    w = _ref_weights(n, k)
    t = _transpose(w, n, k)
    p = S.Q4Params(block).affine() if affine else S.Q4Params(block)
    for quantize in (lambda x, lay: O.q4_quantize(x, lay, n, k, block, affine),
                     lambda x, lay: S.quantize_q4_arrays(x, lay, n, k, p)):
        qa, sa, ma = quantize(w, OUT_IN)
        qb, sb, mb = quantize(t, IN_OUT)
        da = O.q4_dequant(qa, sa, ma, n, k, block)
        db = O.q4_dequant(qb, sb, mb, n, k, block)
        assert np.array_equal(da, db)
        got = _f16(da).reshape(k, n)
        wm = w.reshape(n, k)
        for j in range(n):
            for b0 in range(0, k, block):
                blk = wm[j, b0:b0 + block]
                lo, hi = blk.min(), blk.max()
                step, bound = ((hi - lo) / 15.0, 0.5) if affine else (max(abs(lo), abs(hi)) / 8.0, 1.0)
                err = np.abs(got[b0:b0 + block, j] - blk)
                assert err.max() <= step * bound + 0.01, (j, b0)


def test_q4_scale_form_codes_and_extremes():
    """Q4_0: the block's largest magnitude takes code -8 (scale = m / -8), all
    codes lie in [-8, 7]; affine: the minimum takes code -8 and the maximum
    code 7 (min = lo + 8 * scale)."""
    n, k, block = 9, 256, 64
    rng = np.random.default_rng(5)
    w = rng.uniform(-3, 3, n * k).astype(np.float32)
    wm = w.reshape(n, k)
    q, s, _ = O.q4_quantize(w, OUT_IN, n, k, block)
    codes = _nibble_codes(q, n, k)
    qa, sa, ma = O.q4_quantize(w, OUT_IN, n, k, block, affine=True)
    ca = _nibble_codes(qa, n, k)
    for j in range(n):
        for b in range(k // block):
            blk = wm[j, b * block:(b + 1) * block]
            at = b * block + int(np.argmax(np.abs(blk)))
            assert codes[at, j] == -8
            assert _f16(s[j * (k // block) + b]) * -8 == pytest.approx(blk[at - b * block], rel=1e-3)
            assert ca[b * block + int(np.argmin(blk)), j] == -8
            assert ca[b * block + int(np.argmax(blk)), j] == 7


def test_q4_rejects_bad_block():
    with pytest.raises(ValueError):
        S.Q4Params(48)


# ---- Q2 ------------------------------------------------------------------------

CODEBOOKS = [(-1, 0, 1, 0), (-2, -1, 1, 2), (-3, -1, 0, 2), (0, 0, 5, 0)]


@pytest.mark.parametrize("n,k,block", [s for s in SHAPES if s[2] >= 16])
@pytest.mark.parametrize("cb", CODEBOOKS)
def test_q2_library_matches_oracle(n, k, block, cb):
    rng = np.random.default_rng(n + 7 * k)
    w = _inputs(rng, n, k)
    p = S.Q2Params(block).with_codebook(cb)
    for layout, x in ((OUT_IN, w), (IN_OUT, _transpose(w, n, k))):
        got = S.quantize_q2_arrays(x, layout, n, k, p)
        want = O.q2_quantize(x, layout, n, k, block, cb)
        assert np.array_equal(got[0], want[0]), f"codes {layout}"
        assert np.array_equal(got[1], want[1]), f"scales {layout}"


@pytest.mark.parametrize("cb,levels", [((-1, 0, 1, 0), (-1.0, 0.0, 1.0)),
                                       ((-2, -1, 1, 2), (-2.0, -1.0, 1.0, 2.0))])
def test_q2_recovers_grid_weights(cb, levels):
    """q2.rs:225-262: weights on the codebook's grid come back exactly."""
    n, k = 70, 300
    i = np.arange(n * k)
    lv = np.asarray(levels, np.float32)
    w = (lv[(i * 7 + i // 5) % len(lv)] * np.float32(0.03125)
         * (1 + i // k % 3).astype(np.float32)).astype(np.float32)
    t = _transpose(w, n, k)
    p = S.Q2Params(64).with_codebook(cb)
    cbf = np.asarray(cb, np.float32)
    for quantize in (lambda x, lay: O.q2_quantize(x, lay, n, k, 64, cb),
                     lambda x, lay: S.quantize_q2_arrays(x, lay, n, k, p)):
        for layout, x in ((OUT_IN, w), (IN_OUT, t)):
            codes, scales = quantize(x, layout)
            c = _q2_codes(codes, n, k)
            nbk = -(-k // 64)
            d = np.arange(k)
            for j in range(n):
                got = _f16(scales[j * nbk + d // 64]) * cbf[c[:, j]]
                assert np.array_equal(got.view(np.uint32), w[j * k:(j + 1) * k].view(np.uint32)), (cb, j)


def test_q2_codes_are_nearest_first_of_ties():
    """Each code minimises |w - scale * codebook[code]|; on a tie the lower
    code index wins (min_by keeps the first). Scale = amax / max|codebook|."""
    n, k, block = 11, 320, 32
    rng = np.random.default_rng(9)
    w = (rng.integers(-8, 9, n * k) * 0.125).astype(np.float32)  # exact ties happen
    cb = (-2, -1, 1, 2)
    codes, scales = O.q2_quantize(w, OUT_IN, n, k, block, cb)
    c = _q2_codes(codes, n, k)
    cbf = np.asarray(cb, np.float64)
    wm = w.reshape(n, k).astype(np.float64)
    nbk = k // block
    s = _f16(scales).astype(np.float64).reshape(n, nbk)
    assert np.array_equal(s, np.abs(wm).reshape(n, nbk, block).max(2) / 2)  # exact: /2 of an f16 grid value
    dist = np.abs(wm[:, :, None] - np.repeat(s, block, 1)[:, :, None] * cbf)
    assert np.array_equal(c.T, np.argmin(dist, 2))  # argmin returns the first minimum


def test_q2_zero_codebook_is_an_error():
    w = np.ones(64, np.float32)
    with pytest.raises(ValueError):
        O.q2_quantize(w, OUT_IN, 1, 64, 64, (0, 0, 0, 0))
    with pytest.raises(S.SmeGemmError, match="all zeros"):
        S.quantize_q2_arrays(w, OUT_IN, 1, 64, S.Q2Params(64).with_codebook((0, 0, 0, 0)))


# ---- Q1 ------------------------------------------------------------------------

@pytest.mark.parametrize("n,k,block", [s for s in SHAPES if s[2] >= 16])
def test_q1_library_matches_oracle(n, k, block):
    rng = np.random.default_rng(3 * n + k)
    w = _inputs(rng, n, k)
    for layout, x in ((OUT_IN, w), (IN_OUT, _transpose(w, n, k))):
        got = S.quantize_q1_arrays(x, layout, n, k, block)
        want = O.q1_quantize(x, layout, n, k, block)
        assert np.array_equal(got[0], want[0]), f"signs {layout}"
        assert np.array_equal(got[1], want[1]), f"scales {layout}"


def test_q1_recovers_sign_grid():
    """q1.rs:278-296: weights of one magnitude per block come back exactly,
    from either layout."""
    n, k, block = 70, 300, 64
    i = np.arange(n * k)
    w = (np.where((i * 7 + i // 5) % 3 == 0, -1.0, 1.0) * 0.25 * (1 + i // k % 3)).astype(np.float32)
    t = _transpose(w, n, k)
    nbk = -(-k // block)
    d = np.arange(k)
    for quantize in (O.q1_quantize, S.quantize_q1_arrays):
        for layout, x in ((OUT_IN, w), (IN_OUT, t)):
            signs, scales = quantize(x, layout, n, k, block)
            sg = _q1_signs(signs, n, k)
            for j in range(n):
                got = _f16(scales[j * nbk + d // block]) * np.where(sg[j], 1.0, -1.0).astype(np.float32)
                assert np.array_equal(got.view(np.uint32), w[j * k:(j + 1) * k].view(np.uint32)), j


def test_q1_scale_is_block_mean_and_sign_follows_weight():
    n, k, block = 6, 1000, 128  # ragged last block of 104
    rng = np.random.default_rng(2)
    w = rng.standard_normal(n * k).astype(np.float32)
    w[5] = 0.0
    w[6] = -0.0
    signs, scales = O.q1_quantize(w, OUT_IN, n, k, block)
    sg = _q1_signs(signs, n, k)
    assert np.array_equal(sg.ravel(), w >= 0)  # -0.0 >= 0 too
    nbk = -(-k // block)
    wm = np.abs(w.reshape(n, k)).astype(np.float64)
    for j in range(n):
        for b in range(nbk):
            mean = wm[j, b * block:(b + 1) * block].mean()
            assert _f16(scales[j * nbk + b]) == pytest.approx(mean, rel=2 ** -10)
