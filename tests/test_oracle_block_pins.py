"""Pins for the oracle's decode-block passes (config 5), each checked against
something other than itself:

- rms_norm (src/nn.rs:127-161): an f64 computation (the reference's own
  norms_match_f64 data and bound, tests/correctness/model.rs:100-141, tightened
  to a few f32 ulps), closed forms (constant and zero rows), and planted
  mistakes (a dropped eps, a dim - 1 divisor) that the bound catches.
- RoPE (examples/bonsai/model.rs:30-99): inverse frequencies against numpy's
  f64 power, the position-0 identity bit for bit, norm preservation, the
  relative-position property <R(m)q, R(n)k> = <R(m+t)q, R(n+t)k>, and an f64
  rotation.
- attention_kv_f16 (src/kernels/kv_attention.rs:282-325): the reference's
  kv_f16_matches_oracle test restated (same shapes, lengths, LCG data and f64
  oracle, tests/correctness/kv_attention.rs:7-82), len = 1 giving V's row bit
  for bit, equal keys giving the mean of V.
- glu (src/linear.rs:804-826): an f64 silu / gelu within one f16 ulp, with a
  ragged last chunk, and a planted gate/up swap that must differ.
- the block step (src/block.rs:90-106 with bonsai's RoPE): an independent
  numpy f64 block (its own Q4 decoding, f64 products and softmax) on a small
  shape, within a whole-update tolerance.
"""
import numpy as np
import pytest

import oracle as O


def _ulps32(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def _rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


# ---- rms_norm ------------------------------------------------------------------

@pytest.mark.parametrize("dim", [8, 100, 384, 4096, 4099])
def test_rms_norm_matches_f64(dim):
    """norms_match_f64's data (x = fill*4 + 1, w = fill + 1, eps 1e-6) and its
    bound |y - f64| < 1e-4, plus a relative bound of 8 f32 ulps."""
    s = 0x11EA_0100 ^ dim
    x, s = O.lcg_fill_f32(s, 3 * dim)
    x = x * np.float32(4.0) + np.float32(1.0)
    w, s = O.lcg_fill_f32(s, dim)
    w = w + np.float32(1.0)
    for r in range(3):
        row = x[r * dim:(r + 1) * dim]
        got = O.rms_norm_row(row, w, 1e-6)
        want = _rms64(row, w, 1e-6)
        assert np.max(np.abs(got - want)) < 1e-4
        assert np.all(np.abs(got - want) <= 8 * np.spacing(np.abs(want).astype(np.float32)) + 1e-30)


def test_rms_norm_closed_forms():
    dim = 96
    w = np.linspace(0.5, 1.5, dim).astype(np.float32)
    # a constant row c: r = 1 / sqrt(c^2 + eps), the output c * r * w
    for c in (3.0, -0.25, 1e-3):
        got = O.rms_norm_row(np.full(dim, c, np.float32), w, 1e-5)
        want = _rms64(np.full(dim, c), w, 1e-5)
        assert np.all(_ulps32(got, want.astype(np.float32)) <= 2)
    # a zero row: every output +0 (0 * r * w + 0)
    got = O.rms_norm_row(np.zeros(dim, np.float32), w, 1e-5)
    assert np.all(got.view(np.uint32) == 0)
    z = O.rms_norm_row(-np.zeros(dim, np.float32), w, 1e-5)
    assert np.all(z.view(np.uint32) == 0)  # -0 plus +0 is +0
    # f16 output: the f32 row rounded once
    x = np.random.default_rng(2).standard_normal(2 * dim).astype(np.float32)
    y = O.rms_norm_f16(x, w, 1e-5, rows=2)
    for r in range(2):
        assert np.array_equal(y[r * dim:(r + 1) * dim],
                              O.f32_to_f16(O.rms_norm_row(x[r * dim:(r + 1) * dim], w, 1e-5)))


def test_rms_norm_planted_mistakes_exceed_the_bound():
    """The f64 bound above would catch a dropped eps or a dim - 1 divisor."""
    dim = 384
    x = (np.random.default_rng(3).standard_normal(dim) * 0.05).astype(np.float32)
    w = np.ones(dim, np.float32)
    eps = 1e-3  # comparable to mean(x^2) = 2.5e-3
    good = O.rms_norm_row(x, w, eps)
    assert np.max(np.abs(good - _rms64(x, w, eps))) < 1e-4
    no_eps = _rms64(x, w, 0.0)
    wrong_div = x / np.sqrt(np.sum(x.astype(np.float64) ** 2) / (dim - 1) + eps)
    assert np.max(np.abs(good - no_eps)) > 1e-2
    assert np.max(np.abs(good - wrong_div)) > 1e-4


# ---- RoPE ---------------------------------------------------------------------------

def test_rope_inverse_frequencies():
    for dim in (64, 128):
        inv = O.rope_inv_freq(dim, 10000.0)
        want = (1.0 / np.power(10000.0, np.arange(0, dim, 2, dtype=np.float64) / dim)).astype(np.float32)
        assert np.all(_ulps32(inv, want) <= 1)
        assert inv[0] == 1.0


def test_rope_rotation_properties():
    hd, heads = 128, 3
    inv = O.rope_inv_freq(hd, 10000.0)
    rng = np.random.default_rng(4)
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal(heads * hd).astype(np.float32)
    # position 0: cos 1, sin 0 -- the identity, bit for bit
    c0, s0 = O.rope_angles(inv, 0)
    assert np.all(c0 == 1.0) and np.all(s0.view(np.uint32) == 0)
    assert np.array_equal(O.rope_apply(q, c0, s0).view(np.uint32), q.view(np.uint32))

    def rot64(x, pos):
        a = pos * inv.astype(np.float64)
        x = x.astype(np.float64).reshape(heads, 2, hd // 2)
        u, v = x[:, 0], x[:, 1]
        return np.stack([u * np.cos(a) - v * np.sin(a), v * np.cos(a) + u * np.sin(a)], 1).ravel()

    for pos in (1, 7, 513, 4096):
        c, s = O.rope_angles(inv, pos)
        a32 = np.float32(pos) * inv
        assert np.all(np.abs(c - np.cos(a32.astype(np.float64))) <= 1.2e-7)
        assert np.all(np.abs(s - np.sin(a32.astype(np.float64))) <= 1.2e-7)
        r = O.rope_apply(q, c, s)
        # each (i, i + hd/2) pair keeps its length
        pr = r.astype(np.float64).reshape(heads, 2, hd // 2)
        pq = q.astype(np.float64).reshape(heads, 2, hd // 2)
        assert np.allclose((pr ** 2).sum(1), (pq ** 2).sum(1), rtol=2e-6, atol=1e-7)
        # the rotation itself (angles of the f32 product; the f32 angle rounds
        # by up to pos * 2^-24 rad, so compare at that scale)
        assert np.max(np.abs(r - rot64(q, pos))) < 4e-7 * max(1, pos) + 1e-6
    # relative position: <R(m) q, R(n) k> depends on m - n only
    def dot(m, n):
        cm, sm = O.rope_angles(inv, m)
        cn, sn = O.rope_angles(inv, n)
        return float(np.dot(O.rope_apply(q, cm, sm).astype(np.float64),
                            O.rope_apply(k, cn, sn).astype(np.float64)))
    for m, n, t in ((5, 2, 11), (40, 40, 100), (3, 9, 250)):
        assert abs(dot(m, n) - dot(m + t, n + t)) < 2e-4 * (1 + abs(dot(m, n)))
    # and a planted mistake (the halves rotated the other way) breaks it
    c, s = O.rope_angles(inv, 9)
    assert np.max(np.abs(O.rope_apply(q, c, -s) - rot64(q, 9))) > 1e-2


# ---- attention --------------------------------------------------------------------

def _attn_oracle64(q, k, v, length, heads, kv_heads, hd, scale):
    """tests/correctness/kv_attention.rs:7-41 in numpy f64."""
    ld = kv_heads * hd
    group = heads // kv_heads
    out = np.zeros(heads * hd)
    kf = O.f16_to_f32(k).astype(np.float64).reshape(-1, ld)
    vf = O.f16_to_f32(v).astype(np.float64).reshape(-1, ld)
    for h in range(heads):
        off = (h // group) * hd
        s = kf[:length, off:off + hd] @ (q[h * hd:(h + 1) * hd].astype(np.float64) * float(scale))
        e = np.exp(s - s.max())
        out[h * hd:(h + 1) * hd] = (e / e.sum()) @ vf[:length, off:off + hd]
    return out


@pytest.mark.parametrize("heads,kv_heads,hd", [(1, 1, 8), (6, 6, 64), (8, 2, 64), (4, 1, 128),
                                               (2, 2, 256), (12, 4, 72)])
def test_attention_matches_the_reference_test(heads, kv_heads, hd):
    """kv_f16_matches_oracle (tests/correctness/kv_attention.rs:43-82): its
    shapes, lengths, LCG data (q = fill_f32 * 8, k / v = fill) and bound."""
    for length in (1, 2, 3, 4, 5, 7, 31, 128, 257):
        s = 0x5EED_0000 ^ (heads * 1000 + hd * 10 + length)
        ld = kv_heads * hd
        q, s = O.lcg_fill_f32(s, heads * hd)
        q = q * np.float32(8.0)
        k, s = O.lcg_fill(s, length * ld)
        v, s = O.lcg_fill(s, length * ld)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        got = O.attention_kv_f16(q, k, v, length, heads, kv_heads, hd, scale)
        want = _attn_oracle64(q, k, v, length, heads, kv_heads, hd, scale)
        assert np.max(np.abs(got - want)) < 2e-3, (heads, kv_heads, hd, length)


def test_attention_special_cases():
    heads, kv_heads, hd = 4, 2, 64
    ld = kv_heads * hd
    rng = np.random.default_rng(8)
    q = rng.standard_normal(heads * hd).astype(np.float32)
    v = O.f32_to_f16(rng.standard_normal(5 * ld).astype(np.float32))
    k = O.f32_to_f16(rng.standard_normal(5 * ld).astype(np.float32))
    # one key: the output is its value row exactly (p = 1, sum = 1)
    out = O.attention_kv_f16(q, k[:ld], v[:ld], 1, heads, kv_heads, hd, 0.125)
    for h in range(heads):
        g = h // (heads // kv_heads)
        assert np.array_equal(out[h * hd:(h + 1) * hd], O.f16_to_f32(v[g * hd:(g + 1) * hd]))
    # equal keys: uniform weights, the mean of the values
    kk = np.tile(k[:ld], 5)
    out = O.attention_kv_f16(q, kk, v, 5, heads, kv_heads, hd, 0.125)
    vf = O.f16_to_f32(v).reshape(5, ld).astype(np.float64)
    for h in range(heads):
        g = h // (heads // kv_heads)
        assert np.allclose(out[h * hd:(h + 1) * hd], vf[:, g * hd:(g + 1) * hd].mean(0), atol=2e-6)


# ---- glu --------------------------------------------------------------------------

@pytest.mark.parametrize("n,gelu", [(100, False), (64, True), (14336, False), (5, False)])
def test_glu_matches_f64(n, gelu):
    m = 2
    rng = np.random.default_rng(n)
    g16 = O.f32_to_f16((rng.standard_normal(m * n) * 4).astype(np.float32))
    u16 = O.f32_to_f16((rng.standard_normal(m * n) * 4).astype(np.float32))
    both = np.concatenate([O.interleave32(g16[r * n:(r + 1) * n], u16[r * n:(r + 1) * n], n, 1).ravel()
                           for r in range(m)])
    y = O.glu_f16(both, m, n, gelu)
    g = O.f16_to_f32(g16).astype(np.float64)
    u = O.f16_to_f32(u16).astype(np.float64)
    a = 0.5 * g * (1 + np.tanh(0.7978846 * (g + 0.044715 * g ** 3))) if gelu else g / (1 + np.exp(-g))
    want = a * u
    got = O.f16_to_f32(y).astype(np.float64)
    # one f16 ulp, plus for gelu the f32 cancellation of 1 + tanh(x) near -1
    # that the reference's formula has (a few f32 ulps of 1, times 0.5 |g u|)
    cancel = 0.5 * np.abs(g * u) * 4 * 2.0 ** -23 if gelu else 0.0
    assert np.all(np.abs(got - want) <= np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
                  + cancel + 1e-7)
    # gate and up swapped: a different result (the interleave's roles matter)
    swapped = np.concatenate([O.interleave32(u16[r * n:(r + 1) * n], g16[r * n:(r + 1) * n], n, 1).ravel()
                              for r in range(m)])
    assert not np.array_equal(O.glu_f16(swapped, m, n, gelu), y)


# ---- the block ------------------------------------------------------------------------

def _q4_decode64(quants, scales, n, k, block=32):
    """Q4 row-major input (src/kernels/q4/mod.rs:206-214), decoded here on its own:
    weight (d, j) = scales[j*nbk + d/block] * code, code the two's-complement
    nibble idx % 2 (low first) of byte idx / 2, idx = d*n + j."""
    idx = np.arange(k * n)
    nib = np.where(idx % 2 == 0, quants[idx // 2] & 15, quants[idx // 2] >> 4).astype(np.int64)
    code = np.where(nib < 8, nib, nib - 16).reshape(k, n)
    nbk = -(-k // block)
    sc = scales.view(np.float16).astype(np.float64).reshape(n, nbk)
    return code * sc[:, np.arange(k) // block].T


def small_block(seed, d=256, heads=4, kv_heads=2, hd=64, ffn=320, past=37, theta=10000.0):
    """A small config-5-shaped block: Q4 linears (block 32, scales in
    [0.005, 0.02]), RMSNorm weights in [0.9, 1.1], eps 1e-5, `past` cached f16
    positions ~ N(0,1), a residual row ~ N(0,1)."""
    rng = np.random.default_rng(seed)

    def q4(n, k):
        quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
        scales = O.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32))
        return quants, scales

    nq = (heads + 2 * kv_heads) * hd
    p = dict(d=d, heads=heads, kv_heads=kv_heads, head_dim=hd, ffn=ffn, eps=1e-5, theta=theta)
    p["norm1"] = rng.uniform(0.9, 1.1, d).astype(np.float32)
    p["norm2"] = rng.uniform(0.9, 1.1, d).astype(np.float32)
    raw = {"qkv": (q4(nq, d), nq, d), "out": (q4(d, heads * hd), d, heads * hd),
           "gate": (q4(ffn, d), ffn, d), "up": (q4(ffn, d), ffn, d), "down": (q4(d, ffn), d, ffn)}
    p["raw"] = raw
    p["qkv"] = O.Q4Lin(*raw["qkv"][0], nq, d)
    p["out"] = O.Q4Lin(*raw["out"][0], d, heads * hd)
    p["down"] = O.Q4Lin(*raw["down"][0], d, ffn)
    # GatedLinear: gate and up interleaved 32 columns at a time (linear.rs:601-619)
    gq, gs = raw["gate"][0]
    uq, us = raw["up"][0]
    p["gate_up"] = O.Q4Lin(*O.q4_interleave32(gq, gs, uq, us, ffn, d), 2 * ffn, d)
    cap = past + 4
    ld = kv_heads * hd
    cache_k = np.zeros((cap, ld), np.uint16)
    cache_v = np.zeros((cap, ld), np.uint16)
    cache_k[:past] = O.f32_to_f16(rng.standard_normal(past * ld).astype(np.float32)).reshape(past, ld)
    cache_v[:past] = O.f32_to_f16(rng.standard_normal(past * ld).astype(np.float32)).reshape(past, ld)
    x = rng.standard_normal(d).astype(np.float32)
    return p, x, cache_k, cache_v


def _block64(p, x, cache_k, cache_v, pos):
    """The same step in numpy f64, from its own Q4 decoding: no f16 rounding
    of any intermediate."""
    d, H, KV, hd, eps = p["d"], p["heads"], p["kv_heads"], p["head_dim"], p["eps"]
    W = {name: _q4_decode64(q[0], q[1], n, k) for name, (q, n, k) in p["raw"].items()}
    x = x.astype(np.float64)
    h = _rms64(x, p["norm1"], eps)
    qkv = h @ W["qkv"]
    ql, kl = H * hd, KV * hd
    inv = 1.0 / np.power(p["theta"], np.arange(0, hd, 2) / hd)
    a = pos * inv

    def rope(v):
        v = v.reshape(-1, 2, hd // 2)
        return np.stack([v[:, 0] * np.cos(a) - v[:, 1] * np.sin(a),
                         v[:, 1] * np.cos(a) + v[:, 0] * np.sin(a)], 1).ravel()
    q, k, v = rope(qkv[:ql]), rope(qkv[ql:ql + kl]), qkv[ql + kl:]
    K = np.vstack([O.f16_to_f32(cache_k[:pos]).astype(np.float64).reshape(pos, kl), k])
    V = np.vstack([O.f16_to_f32(cache_v[:pos]).astype(np.float64).reshape(pos, kl), v])
    att = np.zeros(ql)
    g = H // KV
    for hh in range(H):
        off = (hh // g) * hd
        s = K[:, off:off + hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
        e = np.exp(s - s.max())
        att[hh * hd:(hh + 1) * hd] = (e / e.sum()) @ V[:, off:off + hd]
    x = x + att @ W["out"]
    h = _rms64(x, p["norm2"], eps)
    gg, uu = h @ W["gate"], h @ W["up"]
    x = x + (gg / (1 + np.exp(-gg)) * uu) @ W["down"]
    return x


def test_block_step_matches_an_f64_block():
    """The oracle's step (f16 at every point the reference rounds) against an
    f64 block with no roundings: the residual update agrees to the f16
    roundings' size, and the appended key row is the rotated projection."""
    p, x, ck, cv = small_block(21)
    pos = 37
    ck0, cv0 = ck.copy(), cv.copy()
    got = O.block_decode(x, ck, cv, pos, p)
    want = _block64(p, x, ck0, cv0, pos)
    upd_g, upd_w = got.astype(np.float64) - x, want - x
    assert np.linalg.norm(upd_g - upd_w) <= 1e-2 * np.linalg.norm(upd_w)
    assert np.array_equal(ck[:pos], ck0[:pos]) and np.array_equal(cv[:pos], cv0[:pos])
    assert np.any(ck[pos] != 0) and np.any(cv[pos] != 0)
    # without RoPE the key row is the projection's own f16 output
    p2 = dict(p, theta=0.0)
    ck2, cv2 = ck0.copy(), cv0.copy()
    O.block_decode(x, ck2, cv2, pos, p2)
    h = O.rms_norm_f16(x, p["norm1"], p["eps"])
    qkv = p["qkv"].forward(h)
    ql, kl = p["heads"] * p["head_dim"], p["kv_heads"] * p["head_dim"]
    assert np.array_equal(ck2[pos], qkv[ql:ql + kl]) and np.array_equal(cv2[pos], qkv[ql + kl:])


def test_interleaved_q4_is_gate_and_up_side_by_side():
    """The interleaved Q4 arrays decode to gate's and up's columns in the
    32-column pattern (checked through the independent decoder)."""
    rng = np.random.default_rng(5)
    n, k = 100, 64
    gq = rng.integers(0, 256, k * n // 2, dtype=np.uint8)
    uq = rng.integers(0, 256, k * n // 2, dtype=np.uint8)
    gs = O.f32_to_f16(rng.uniform(0.1, 1, n * 2).astype(np.float32))
    us = O.f32_to_f16(rng.uniform(0.1, 1, n * 2).astype(np.float32))
    q, s = O.q4_interleave32(gq, gs, uq, us, n, k)
    both = _q4_decode64(q, s, 2 * n, k)
    G, U = _q4_decode64(gq, gs, n, k), _q4_decode64(uq, us, n, k)
    assert np.array_equal(both, O.interleave32(G, U, n, k))


# ---- LayerNorm, causal attention, blocks of rows ----------------------------------------

def _ln64(x, w, b, eps):
    x = np.asarray(x, np.float64)
    mu = np.mean(x)
    y = (x - mu) / np.sqrt(np.mean((x - mu) ** 2) + eps) * np.asarray(w, np.float64)
    return y + (0.0 if b is None else np.asarray(b, np.float64))


@pytest.mark.parametrize("dim,bias", [(4, False), (8, True), (100, True), (384, False), (4099, True)])
def test_layer_norm_matches_f64(dim, bias):
    """norm_row's LayerNorm form (src/nn.rs:133-143: two lane_sum passes in
    f32) against an f64 two-pass LayerNorm: within 1e-4 and 16 f32 ulps (the
    f32 mean's rounding enters every centred value)."""
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal(dim) * 3 + 0.7).astype(np.float32)
    w = rng.uniform(0.9, 1.1, dim).astype(np.float32)
    b = rng.normal(0, 0.1, dim).astype(np.float32) if bias else None
    got = O.layer_norm_row(x, w, b, 1e-5)
    want = _ln64(x, w, b, 1e-5)
    assert np.max(np.abs(got - want)) < 1e-4
    assert np.all(np.abs(got - want) <= 16 * np.spacing(np.abs(want).astype(np.float32)) + 1e-6)


def test_layer_norm_doc_example_and_closed_forms():
    """nn::layer_norm's own doc example (src/nn.rs:64-68: x = 1, 2, 3, 4, unit
    weights, eps 1e-5): mean 2.5, variance 1.25, so (x - 2.5) / sqrt(1.25001);
    a constant row gives the bias (zero centred values); f16 output is the f32
    row rounded once."""
    x = np.array([1, 2, 3, 4], np.float32)
    got = O.layer_norm_row(x, np.ones(4, np.float32), None, 1e-5)
    want = (x.astype(np.float64) - 2.5) / np.sqrt(1.25 + 1e-5)
    assert np.all(_ulps32(got, want.astype(np.float32)) <= 2)
    b = np.linspace(-1, 1, 96).astype(np.float32)
    const = O.layer_norm_row(np.full(96, 7.25, np.float32), np.ones(96, np.float32), b, 1e-5)
    assert np.array_equal(const, b)
    xs = np.random.default_rng(2).standard_normal(2 * 96).astype(np.float32)
    w = np.linspace(0.5, 1.5, 96).astype(np.float32)
    y = O.layer_norm_f16(xs, w, b, 1e-5, rows=2)
    for r in range(2):
        assert np.array_equal(y[r * 96:(r + 1) * 96], O.f32_to_f16(O.layer_norm_row(xs[r * 96:(r + 1) * 96], w, b,
                                                                                    1e-5)))


def test_layer_norm_planted_mistakes_exceed_the_bound():
    """The f64 bound would catch a missing centring (RMS in place of the
    variance), a dim - 1 divisor and a dropped bias."""
    dim = 384
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(dim) * 0.5 + 1.0).astype(np.float32)
    w = np.ones(dim, np.float32)
    b = rng.normal(0, 0.1, dim).astype(np.float32)
    good = O.layer_norm_row(x, w, b, 1e-5)
    assert np.max(np.abs(good - _ln64(x, w, b, 1e-5))) < 1e-4
    x64 = x.astype(np.float64)
    mu = x64.mean()
    uncentred = (x64 - mu) / np.sqrt(np.mean(x64 ** 2) + 1e-5) + b
    wrong_div = (x64 - mu) / np.sqrt(np.sum((x64 - mu) ** 2) / (dim - 1) + 1e-5) + b
    no_bias = _ln64(x, w, None, 1e-5)
    for bad in (uncentred, wrong_div, no_bias):
        assert np.max(np.abs(good - bad)) > 1e-3


def _causal64(q, k, v, start, rows, heads, kv_heads, hd, scale):
    ld = kv_heads * hd
    K = O.f16_to_f32(k).astype(np.float64).reshape(-1, ld)
    V = O.f16_to_f32(v).astype(np.float64).reshape(-1, ld)
    g = heads // kv_heads
    out = np.zeros((rows, heads * hd))
    for i in range(rows):
        n = start + i + 1
        for h in range(heads):
            off = (h // g) * hd
            # q rounded as one_row rounds it (f16(q * scale), kv_attention.rs:298-302)
            qh = O.f16_to_f32(O.f32_to_f16(q[i * heads * hd + h * hd:i * heads * hd + (h + 1) * hd] * scale))
            s = K[:n, off:off + hd] @ qh.astype(np.float64)
            e = np.exp(s - s.max())
            out[i, h * hd:(h + 1) * hd] = (e / e.sum()) @ V[:n, off:off + hd]
    return out.ravel()


@pytest.mark.parametrize("heads,kv_heads,hd,start,rows", [(4, 2, 64, 0, 5), (6, 6, 64, 10, 7), (8, 1, 32, 3, 12)])
def test_causal_attention_matches_f64(heads, kv_heads, hd, start, rows):
    """attention_kv_causal_f16's portable path (kv_attention.rs:214-238):
    against an f64 masked softmax (row i sees keys 0 .. start + i; q rounded
    to f16 after the scale, as one_row rounds it) within 2e-4, and with a
    planted off-by-one in the mask (row i seeing start + i keys, or
    start + i + 2) failing that bound by far."""
    rng = np.random.default_rng(heads + start + rows)
    ld = kv_heads * hd
    q = (rng.standard_normal(rows * heads * hd) * 4).astype(np.float32)
    k = O.f32_to_f16(rng.standard_normal((start + rows + 1) * ld).astype(np.float32))
    v = O.f32_to_f16(rng.standard_normal((start + rows + 1) * ld).astype(np.float32))
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    got = O.attention_kv_causal_f16(q, k, v, start, rows, heads, kv_heads, hd, scale)
    want = _causal64(q, k, v, start, rows, heads, kv_heads, hd, scale)
    assert np.max(np.abs(got - want)) < 2e-4
    short = _causal64(q, k, v, start - 1, rows, heads, kv_heads, hd, scale) if start > 0 else None
    long = _causal64(q, k, v, start + 1, rows, heads, kv_heads, hd, scale)
    for bad in (short, long):
        if bad is not None:
            assert np.max(np.abs(got - bad)) > 1e-2


def test_block_rows_match_an_f64_block_row_by_row():
    """block_rows (src/block.rs:90-106 for many rows): against the f64 block
    applied row by row with each row's own key and value appended in f64 --
    the whole block of rows agrees to the f16 roundings' size -- and a block
    of rows whose attention skipped the rows' own keys (every row seeing only
    the cached prefix) fails that bound."""
    p, x, ck, cv = small_block(31)
    rows, pos = 4, 37
    rng = np.random.default_rng(32)
    xs = rng.standard_normal((rows, p["d"])).astype(np.float32)
    cap = pos + rows + 1
    ck2 = np.zeros((cap, ck.shape[1]), np.uint16)
    cv2 = np.zeros_like(ck2)
    ck2[:pos], cv2[:pos] = ck[:pos], cv[:pos]
    got = O.block_rows(xs.ravel(), ck2, cv2, pos, rows, p).reshape(rows, -1)
    K64, V64 = ck2.copy(), cv2.copy()
    for r in range(rows):
        want = _block64(p, xs[r], K64, V64, pos + r)
        upd_g, upd_w = got[r].astype(np.float64) - xs[r], want - xs[r]
        assert np.linalg.norm(upd_g - upd_w) <= 1e-2 * np.linalg.norm(upd_w), r
    # the cache rows written are exactly the one-row steps' (row order kept)
    ck3, cv3 = ck2.copy(), cv2.copy()
    ck3[pos:], cv3[pos:] = 0, 0
    for r in range(rows):
        O.block_decode(xs[r], ck3, cv3, pos + r, p)
    assert np.array_equal(ck3, ck2) and np.array_equal(cv3, cv2)
    # planted: row 3 attending as if rows 0-2 had not been appended
    ck4, cv4 = ck2.copy(), cv2.copy()
    ck4[pos:pos + 3] = ck4[pos + 3]
    cv4[pos:pos + 3] = cv4[pos + 3]
    bad = O.block_decode(xs[3], np.delete(ck4, [pos, pos + 1, pos + 2], 0), np.delete(cv4, [pos, pos + 1, pos + 2], 0),
                         pos, p)
    assert np.linalg.norm(bad - got[3]) > 1e-2 * np.linalg.norm(got[3].astype(np.float64) - xs[3])


def _gpt2_64(p, raw, x, K, V, pos):
    """A GPT-2-style step in f64 from its own Q4 decoding: LayerNorm (with
    bias), multi-head attention without RoPE, up -> tanh-gelu -> down."""
    d, H, hd, eps = p["d"], p["heads"], p["head_dim"], p["eps"]
    W = {name: _q4_decode64(q[0], q[1], n, k) for name, (q, n, k) in raw.items()}
    x = x.astype(np.float64)
    h = _ln64(x, p["norm1"], p["bias1"], eps)
    qkv = h @ W["qkv"]
    ql = H * hd
    q, k, v = qkv[:ql], qkv[ql:2 * ql], qkv[2 * ql:]
    Kf = np.vstack([O.f16_to_f32(K[:pos]).astype(np.float64).reshape(pos, ql), k])
    Vf = np.vstack([O.f16_to_f32(V[:pos]).astype(np.float64).reshape(pos, ql), v])
    att = np.zeros(ql)
    for hh in range(H):
        s = Kf[:, hh * hd:(hh + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
        e = np.exp(s - s.max())
        att[hh * hd:(hh + 1) * hd] = (e / e.sum()) @ Vf[:, hh * hd:(hh + 1) * hd]
    x = x + att @ W["out"]
    h = _ln64(x, p["norm2"], p["bias2"], eps)
    u = h @ W["up"]
    g = 0.5 * u * (1 + np.tanh(0.7978845608028654 * (u + 0.044715 * u ** 3)))
    return x + g @ W["down"]


def test_gpt2_style_block_step_matches_f64():
    """The oracle's one-row step with Norm::layer norms and Mlp::new(up, gelu,
    down), no RoPE, heads = kv_heads (examples/shakespeare/model.rs:91-112)
    against the f64 step: the update to the f16 roundings' size."""
    rng = np.random.default_rng(51)
    d, H, hd, ffn, pos = 128, 4, 32, 256, 9

    def q4(n, k):
        return (rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8),
                O.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32)))
    raw = {"qkv": (q4(3 * H * hd, d), 3 * H * hd, d), "out": (q4(d, H * hd), d, H * hd),
           "up": (q4(ffn, d), ffn, d), "down": (q4(d, ffn), d, ffn)}
    p = dict(d=d, heads=H, kv_heads=H, head_dim=hd, ffn=ffn, eps=1e-5, theta=0.0, norm="layer", act=2,
             norm1=rng.uniform(0.9, 1.1, d).astype(np.float32), norm2=rng.uniform(0.9, 1.1, d).astype(np.float32),
             bias1=rng.normal(0, 0.1, d).astype(np.float32), bias2=rng.normal(0, 0.1, d).astype(np.float32))
    for name, (q, n, k) in raw.items():
        p[name] = O.Q4Lin(*q, n, k)
    K = np.zeros((pos + 1, H * hd), np.uint16)
    V = np.zeros_like(K)
    K[:pos] = O.f32_to_f16(rng.standard_normal(pos * H * hd).astype(np.float32)).reshape(pos, -1)
    V[:pos] = O.f32_to_f16(rng.standard_normal(pos * H * hd).astype(np.float32)).reshape(pos, -1)
    x = rng.standard_normal(d).astype(np.float32)
    got = O.block_decode(x, K.copy(), V.copy(), pos, p)
    want = _gpt2_64(p, raw, x, K, V, pos)
    assert np.linalg.norm(got - want) <= 1e-2 * np.linalg.norm(want - x)
    # a silu in place of the gelu, or an RMS norm in place of the LayerNorm, fails it
    for bad_p in (dict(p, act=3), dict(p, norm="rms")):
        bad = O.block_decode(x, K.copy(), V.copy(), pos, bad_p)
        assert np.linalg.norm(bad - want) > 1e-2 * np.linalg.norm(want - x)
