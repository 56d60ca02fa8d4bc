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
