"""The decode block (config 5) and its parts on the GPU against the oracle's
restatement of the reference's portable path (oracle/: nn::rms_norm,
attention_kv_f16's one_row, glu, the Q4 GEMV, Block::accumulate with
examples/bonsai's RoPE).

Bars (rel = |g - w| / (1 + |w|), the reference's max_rel,
tests/correctness/main.rs:63-68):
- f16 GEMV-derived values (projections, the hidden layer): rel <= f16_tol(K),
  the north star's 2e-3 * sqrt(K)/64 at the GEMV's depth;
- the block's f32 residual: it adds two f16 terms, the out projection's A
  (K = heads*head_dim) and the down projection's M (K = ffn), each held to the
  GEMV bar, so |g - w| <= f16_tol(K_A)(1 + |A|) + f16_tol(K_M)(1 + |M|) + P
  per element with A, M the oracle's terms (an error relative to the result
  would be wrong where A and M cancel) and P how far A's error moves M, which
  is computed from the residual A lands in (the oracle's MLP half re-run on
  that residual shifted by A's tolerance); and the whole update within 1e-3
  of the oracle's in relative norm;
- a term added into a residual (Linear / Mlp / SelfAttention accumulate):
  held to its GEMV bar relative to the term, plus how far the term moves when
  an f16 input that is itself a GEMV result (the hidden layer, qkv) moves by
  its own tolerance -- measured on the oracle with seeded random signs;
- rms_norm: within one f16 ulp (the sum of squares runs in another order);
- attention: within 2e-3 absolute of the f64 oracle on the reference's own
  test data (tests/correctness/kv_attention.rs:43-82), and within
  1e-4 * (1 + max |v|) of the portable one_row (same q rounding, sums in other
  orders); one cached key gives its value row bit for bit.
"""
import numpy as np
import pytest

import workloads as WL
from conftest import f16_tol, max_rel, ulp_dist

pytestmark = pytest.mark.gpu


def _h16(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.float16)).cuda()


def _f32(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def _np16(t):
    return t.cpu().numpy().view(np.uint16).ravel()


def _check_term(got, y0, term, tol, moved=0.0):
    """y = y0 + term: the added term held to the bar relative to the term
    (not to the sum, which can cancel), plus `moved`, the part of its error
    inherited from an f16 input that is itself a tolerance-checked result."""
    err = np.abs(np.asarray(got, np.float64) - (np.asarray(y0, np.float64) + term))
    bound = tol * (1 + np.abs(term)) + moved
    assert np.all(err <= bound), float(np.max(err / bound))


# ---- row passes --------------------------------------------------------------------

@pytest.mark.parametrize("rows,dim", [(1, 8), (3, 100), (2, 384), (1, 4096), (2, 4099), (1, 14336)])
def test_rms_norm_within_one_ulp(smg, orc, rows, dim):
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal(rows * dim) * 3 + 0.5).astype(np.float32)
    w = rng.uniform(0.9, 1.1, dim).astype(np.float32)
    import torch
    y = torch.empty(rows * dim, dtype=torch.float16, device="cuda")
    smg.rms_norm(_f32(x), _f32(w), 1e-5, y)
    torch.cuda.synchronize()
    want = orc.rms_norm_f16(x, w, 1e-5, rows)
    got = _np16(y)
    assert ulp_dist(got, want) <= 1
    assert np.mean(got == want) > 0.99


@pytest.mark.parametrize("n,gate", [(100, "Silu"), (64, "Gelu"), (14336, "Silu"), (5, "Silu")])
def test_glu_matches_oracle(smg, orc, n, gate):
    import torch
    m = 3
    rng = np.random.default_rng(n + len(gate))
    both = orc.f32_to_f16((rng.standard_normal(m * 2 * n) * 4).astype(np.float32))
    y = torch.empty(m * n, dtype=torch.float16, device="cuda")
    smg.glu(_h16(both), m, n, getattr(smg.Gate, gate), y)
    torch.cuda.synchronize()
    want = orc.glu_f16(both, m, n, gate == "Gelu")
    got = _np16(y)
    # tests/correctness/model.rs:283: |got - want| <= 2e-3 (1 + |want|)
    assert max_rel(got, want) <= 2e-3
    if gate == "Silu":
        # the same formula, the device's exp: nearly every value the same bits
        # (gelu's 1 + tanh(x) cancels for negative gates, where the two libms'
        # tanh near -1 decide the low bits and even the sign of a zero)
        assert np.mean(got == want) > 0.98


# ---- attention -----------------------------------------------------------------------

def _attn64(q, k, v, length, heads, kv_heads, hd, scale):
    ld = kv_heads * hd
    g = heads // kv_heads
    kf = np.asarray(k, np.uint16).view(np.float16).astype(np.float64).reshape(-1, ld)
    vf = np.asarray(v, np.uint16).view(np.float16).astype(np.float64).reshape(-1, ld)
    out = np.zeros(heads * hd)
    for h in range(heads):
        off = (h // g) * hd
        s = kf[:length, off:off + hd] @ (q[h * hd:(h + 1) * hd].astype(np.float64) * float(scale))
        e = np.exp(s - s.max())
        out[h * hd:(h + 1) * hd] = (e / e.sum()) @ vf[:length, off:off + hd]
    return out


@pytest.mark.parametrize("heads,kv_heads,hd", [(1, 1, 8), (6, 6, 64), (8, 2, 64), (4, 1, 128),
                                               (2, 2, 256), (12, 4, 72), (64, 1, 32)])
def test_attention_reference_cases(smg, orc, heads, kv_heads, hd):
    """kv_f16_matches_oracle's shapes, lengths and LCG data, plus 4097 keys."""
    import torch
    for length in (1, 2, 3, 4, 5, 7, 31, 128, 257, 4097):
        s = 0x5EED_0000 ^ (heads * 1000 + hd * 10 + length)
        ld = kv_heads * hd
        q, s = orc.lcg_fill_f32(s, heads * hd)
        q = q * np.float32(8.0)
        k, s = orc.lcg_fill(s, length * ld)
        v, s = orc.lcg_fill(s, length * ld)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        out = torch.empty(heads * hd, dtype=torch.float32, device="cuda")
        smg.attention_kv_f16(_f32(q), _h16(k), _h16(v), length, heads, kv_heads, hd, float(scale), out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        tag = (heads, kv_heads, hd, length)
        assert np.max(np.abs(got - _attn64(q, k, v, length, heads, kv_heads, hd, scale))) < 2e-3, tag
        one = orc.attention_kv_f16(q, k, v, length, heads, kv_heads, hd, scale)
        assert np.max(np.abs(got - one)) <= 1e-4 * (1 + 0.5), tag
        if length == 1:
            g = heads // kv_heads
            vrow = np.concatenate([orc.f16_to_f32(v[(h // g) * hd:(h // g + 1) * hd]) for h in range(heads)])
            assert np.array_equal(got, vrow), tag


def test_attention_config5_shape(smg, orc):
    """32 query heads over 8 KV heads of 128, 4097 keys ~ N(0,1), q ~ N(0, 4)."""
    import torch
    heads, kv_heads, hd, length = 32, 8, 128, 4097
    rng = np.random.default_rng(5)
    q = (rng.standard_normal(heads * hd) * 4).astype(np.float32)
    k = orc.f32_to_f16(rng.standard_normal(length * kv_heads * hd).astype(np.float32))
    v = orc.f32_to_f16(rng.standard_normal(length * kv_heads * hd).astype(np.float32))
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    out = torch.empty(heads * hd, dtype=torch.float32, device="cuda")
    smg.attention_kv_f16(_f32(q), _h16(k), _h16(v), length, heads, kv_heads, hd, float(scale), out)
    torch.cuda.synchronize()
    want = orc.attention_kv_f16(q, k, v, length, heads, kv_heads, hd, scale)
    vmax = float(np.max(np.abs(orc.f16_to_f32(v))))
    assert np.max(np.abs(out.cpu().numpy() - want)) <= 1e-4 * (1 + vmax)


def test_attention_merge_repeats_and_replays(smg, orc):
    """The split partials and their merge (two launches on the stream's own
    scratch): calls of 1 to 65 splits (head dims 32 to 256, decode and causal
    rows, up to 64 query heads a KV head) agree with the oracle, give the same
    bits when repeated in another order, and a HIP graph that captured them
    replays them bit for bit three times, with eager calls between the
    replays."""
    import torch
    rng = np.random.default_rng(11)
    cases = []
    for heads, kv_heads, hd, length, rows in [(32, 8, 128, 4097, 1), (8, 2, 64, 300, 1), (2, 2, 256, 1000, 1),
                                              (32, 8, 128, 700, 5), (4, 1, 128, 64, 1), (64, 1, 32, 3100, 3)]:
        q = (rng.standard_normal(rows * heads * hd) * 4).astype(np.float32)
        k = orc.f32_to_f16(rng.standard_normal(length * kv_heads * hd).astype(np.float32))
        v = orc.f32_to_f16(rng.standard_normal(length * kv_heads * hd).astype(np.float32))
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        out = torch.empty(rows * heads * hd, dtype=torch.float32, device="cuda")
        cases.append(dict(shape=(heads, kv_heads, hd, length, rows), q=q, k=k, v=v, qd=_f32(q), kd=_h16(k),
                          vd=_h16(v), scale=scale, out=out))

    def call(c):
        heads, kv_heads, hd, length, rows = c["shape"]
        if rows == 1:
            smg.attention_kv_f16(c["qd"], c["kd"], c["vd"], length, heads, kv_heads, hd, c["scale"], c["out"])
        else:
            smg.attention_kv_causal_f16(c["qd"], c["kd"], c["vd"], length - rows, rows, heads, kv_heads, hd,
                                        c["scale"], c["out"])

    for c in cases:
        call(c)
    torch.cuda.synchronize()
    first = [c["out"].cpu().numpy().copy() for c in cases]
    for c, got in zip(cases, first):
        heads, kv_heads, hd, length, rows = c["shape"]
        if rows == 1:
            want = orc.attention_kv_f16(c["q"], c["k"], c["v"], length, heads, kv_heads, hd, np.float32(c["scale"]))
        else:
            want = orc.attention_kv_causal_f16(c["q"], c["k"], c["v"], length - rows, rows, heads, kv_heads, hd,
                                               np.float32(c["scale"]))
        vmax = float(np.max(np.abs(orc.f16_to_f32(c["v"]))))
        assert np.max(np.abs(got - want)) <= 1e-4 * (1 + vmax), c["shape"]
    for c in reversed(cases):
        c["out"].zero_()
        call(c)
    torch.cuda.synchronize()
    for c, got in zip(cases, first):
        assert np.array_equal(c["out"].cpu().numpy(), got), ("repeat", c["shape"])
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in cases:  # the capture stream's own scratch and counters, before capture
            call(c)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=side):
            for c in cases:
                call(c)
    torch.cuda.synchronize()
    for rep in range(3):
        for c in cases:
            c["out"].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, got in zip(cases, first):
            assert np.array_equal(c["out"].cpu().numpy(), got), ("replay", rep, c["shape"])
        for c in cases:  # eager calls between replays
            call(c)
        torch.cuda.synchronize()
        for c, got in zip(cases, first):
            assert np.array_equal(c["out"].cpu().numpy(), got), ("eager after replay", rep, c["shape"])


def test_kv_cache_api(smg, orc):
    """KvCache on the device (kv_attention.rs:342-578; the reference's
    kv_cache_matches_free_functions): rows pushed one at a time and in blocks
    hold the same keys, attend is attention_kv_f16 over them, truncate and
    clear, and a full cache refuses more rows."""
    import torch
    heads, kv_heads, hd = 8, 2, 64
    ld = kv_heads * hd
    rng = np.random.default_rng(9)
    length = 37
    k = orc.f32_to_f16((rng.standard_normal(length * ld) * 0.5).astype(np.float32))
    v = orc.f32_to_f16((rng.standard_normal(length * ld) * 0.5).astype(np.float32))
    one = smg.KvCache(heads, kv_heads, hd, 64)
    for t in range(length):
        one.push(_h16(k[t * ld:(t + 1) * ld]), _h16(v[t * ld:(t + 1) * ld]))
    block = smg.KvCache(heads, kv_heads, hd, 64)
    block.extend(_h16(k[:10 * ld]), _h16(v[:10 * ld]))
    block.extend(_h16(k[10 * ld:]), _h16(v[10 * ld:]))
    torch.cuda.synchronize()
    assert one.len() == block.len() == length and one.capacity() == 64
    assert np.array_equal(_np16(one.keys()), k) and np.array_equal(_np16(block.values()), v)
    assert abs(one.scale() - 1.0 / np.sqrt(64.0)) < 1e-7
    q = (rng.standard_normal(heads * hd) * 8).astype(np.float32)
    got = torch.empty(heads * hd, dtype=torch.float32, device="cuda")
    free = torch.empty(heads * hd, dtype=torch.float32, device="cuda")
    one.attend(_f32(q), got)
    smg.attention_kv_f16(_f32(q), _h16(k), _h16(v), length, heads, kv_heads, hd, one.scale(), free)
    torch.cuda.synchronize()
    assert torch.equal(got, free)
    one.truncate(3)
    assert one.len() == 3
    one.clear()
    assert one.is_empty()
    full = smg.KvCache(1, 1, 8, 1)
    row = _h16(np.zeros(8, np.uint16))
    full.push(row, row)
    with pytest.raises(smg.SmeGemmError, match="KvCache full"):
        full.push(row, row)
    with pytest.raises(smg.SmeGemmError):
        smg.KvCache(3, 2, 64, 4)  # heads not a multiple of kv_heads
    with pytest.raises(smg.SmeGemmError):
        smg.KvCache(2, 2, 12, 4)  # head_dim not a multiple of 8


# ---- projections ----------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (3, 200, 96), (8, 512, 1024), (12, 256, 512),
                                   (64, 4100, 4096), (200, 1000, 512)])
def test_linear_accumulate(smg, orc, m, n, k):
    """Linear::accumulate (src/linear.rs:425-432): y += f32(f16(x @ W))."""
    import torch
    a, quants, scales, _ = WL.q4_inputs(m, n, k, seed=m + n)
    lin = smg.Linear(smg.Q4Weights(quants, scales, n, k))
    y0 = np.random.default_rng(1).standard_normal(m * n).astype(np.float32)
    y = _f32(y0)
    lin.accumulate(_h16(a), y, m)
    torch.cuda.synchronize()
    out = orc.f16_to_f32(orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32))
    _check_term(y.cpu().numpy(), y0, out, f16_tol(k))


@pytest.mark.parametrize("m,n,k", [(64, 4100, 4096), (33, 4096, 4096), (512, 4096, 4096), (200, 1000, 512)])
def test_linear_accumulate_adds_forward(smg, m, n, k):
    """Linear::accumulate (src/linear.rs:425-432) is y + f32(forward's f16
    output), bit for bit: the split-K GEMM adds into y in its reduce, from the
    value the split GEMM of forward stores."""
    import torch
    a, quants, scales, _ = WL.q4_inputs(m, n, k, seed=3 * m + n)
    lin = smg.Linear(smg.Q4Weights(quants, scales, n, k))
    y0 = np.random.default_rng(2).standard_normal(m * n).astype(np.float32)
    y = _f32(y0)
    out = torch.empty(m * n, dtype=torch.float16, device="cuda")
    lin.forward(_h16(a), out, m)
    lin.accumulate(_h16(a), y, m)
    torch.cuda.synchronize()
    want = y0 + out.float().cpu().numpy()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


# One row on the all-steps-in-flight decode GEMV: one or two tiles a compute
# unit (N up to 8192 on 256 CUs), 4, 8, 14 or 16 weight steps a lane (K up to
# 16384), ragged N and K, and the shapes it hands to the other kernels
# (two tiles with more than 4 steps, more than two tiles).
@pytest.mark.parametrize("n,k", [(5000, 4096), (8192, 4096), (200, 5000), (1000, 10000), (96, 16384),
                                 (333, 14336), (4100, 5000), (9000, 2048), (4096, 100)])
def test_linear_accumulate_one_row_shapes(smg, orc, n, k):
    """Linear::accumulate (src/linear.rs:425-432) for one row."""
    import torch
    a, quants, scales, _ = WL.q4_inputs(1, n, k, seed=n + k)
    lin = smg.Linear(smg.Q4Weights(quants, scales, n, k))
    y0 = np.random.default_rng(2).standard_normal(n).astype(np.float32)
    y = _f32(y0)
    lin.accumulate(_h16(a), y, 1)
    torch.cuda.synchronize()
    out = orc.f16_to_f32(orc.matmul_q4_ep(a, quants, scales, None, 1, n, k, 32))
    _check_term(y.cpu().numpy(), y0, out, f16_tol(k))


def _mlp_oracle(orc, x16, inp, m, d, ffn, gated, gelu=False, parts=None):
    gq, gs, _, _ = inp["gate"]
    dq, ds, _, _ = inp["down"]
    if gated:
        uq, us, _, _ = inp["up"]
        iq, isc = orc.q4_interleave32(gq, gs, uq, us, ffn, d)
        both = orc.matmul_q4_ep(x16, iq, isc, None, m, 2 * ffn, d, 32)
        hid = orc.glu_f16(both, m, ffn, gelu)
    else:
        hid = orc.matmul_q4_ep(x16, gq, gs, None, m, ffn, d, 32, (), 2 if gelu else 3)
    if parts is not None:
        parts["hid"] = hid
    return orc.f16_to_f32(orc.matmul_q4_ep(hid, dq, ds, None, m, d, ffn, 32))


def _down_moved(orc, inp, hid, m, d, ffn):
    """How far the down projection's output moves when its f16 input (the
    hidden layer, itself a GEMV result held to f16_tol(d)) moves by that
    tolerance, with seeded random signs: the part of the MLP term's error that
    comes from the hidden layer rather than from the down GEMV itself."""
    dq, ds, _, _ = inp["down"]
    h = orc.f16_to_f32(hid).astype(np.float64)
    sign = np.where(np.random.default_rng(3).random(h.size) < 0.5, -1.0, 1.0)
    h2 = orc.f32_to_f16((h + sign * f16_tol(d) * (1 + np.abs(h))).astype(np.float32))
    a = orc.f16_to_f32(orc.matmul_q4_ep(hid, dq, ds, None, m, d, ffn, 32)).astype(np.float64)
    b = orc.f16_to_f32(orc.matmul_q4_ep(h2, dq, ds, None, m, d, ffn, 32)).astype(np.float64)
    return np.abs(b - a)


@pytest.mark.parametrize("gated,gelu,m,d,ffn", [(True, False, 1, 4096, 14336), (True, False, 3, 256, 320),
                                                (True, True, 1, 256, 100), (False, True, 2, 256, 320),
                                                (False, False, 1, 512, 1024), (True, False, 12, 256, 320),
                                                (True, False, 640, 256, 3204), (True, True, 520, 256, 3300)])
def test_mlp_accumulate(smg, orc, gated, gelu, m, d, ffn):
    """Mlp::gated / Mlp::new accumulate (src/mlp.rs:113-149): the up GEMV with
    its activation (or glu) at the store, then down adding into y. The 640- and
    520-row cases fill the device with one GEMM pass, which applies glu at its
    store (hidden widths that are not whole groups of 8 included)."""
    import torch
    inp = WL.block_inputs(d, 2, 1, 64, ffn, 1, seed=ffn + m)
    gate = smg.Gate.Gelu if gelu else smg.Gate.Silu
    W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
    if gated:
        mlp = smg.Mlp.gated(smg.GatedLinear.from_q4(W("gate"), W("up"), gate), smg.Linear(W("down")))
    else:
        mlp = smg.Mlp.new(smg.Linear(W("gate")), gate, smg.Linear(W("down")))
    assert (mlp.k(), mlp.n(), mlp.hidden()) == (d, d, ffn)
    x16 = orc.f32_to_f16(np.random.default_rng(m).standard_normal(m * d).astype(np.float32))
    y0 = np.full(m * d, 0.25, np.float32)
    y = _f32(y0)
    mlp.accumulate(_h16(x16), y, m)
    torch.cuda.synchronize()
    parts = {}
    term = _mlp_oracle(orc, x16, inp, m, d, ffn, gated, gelu, parts)
    _check_term(y.cpu().numpy(), y0, term, f16_tol(ffn), _down_moved(orc, inp, parts["hid"], m, d, ffn))


def test_gated_linear_forward(smg, orc):
    """GatedLinear::forward (src/linear.rs:779-791) from two Q4 weight sets:
    the interleaved GEMV then glu, against the oracle's interleave."""
    import torch
    n, k, m = 100, 256, 2
    inp = WL.block_inputs(k, 2, 1, 64, n, 1, seed=3)
    gl = smg.GatedLinear.from_q4(smg.Q4Weights(*inp["gate"][:2], n, k), smg.Q4Weights(*inp["up"][:2], n, k),
                                 smg.Gate.Silu)
    x16 = orc.f32_to_f16(np.random.default_rng(4).standard_normal(m * k).astype(np.float32))
    y = torch.empty(m * n, dtype=torch.float16, device="cuda")
    gl.forward(_h16(x16), y, m)
    torch.cuda.synchronize()
    iq, isc = orc.q4_interleave32(*inp["gate"][:2], *inp["up"][:2], n, k)
    want = orc.glu_f16(orc.matmul_q4_ep(x16, iq, isc, None, m, 2 * n, k, 32), m, n)
    assert max_rel(_np16(y), want) <= f16_tol(k)


# ---- attention half and the block ----------------------------------------------------------------

def _oracle_params(orc, inp, d, heads, kv_heads, hd, ffn, eps, theta):
    p = dict(d=d, heads=heads, kv_heads=kv_heads, head_dim=hd, ffn=ffn, eps=eps, theta=theta,
             norm1=inp["norm1"], norm2=inp["norm2"])
    for key in ("qkv", "out", "down"):
        q, s, n, k = inp[key]
        p[key] = orc.Q4Lin(q, s, n, k)
    iq, isc = orc.q4_interleave32(*inp["gate"][:2], *inp["up"][:2], ffn, d)
    p["gate_up"] = orc.Q4Lin(iq, isc, 2 * ffn, d)
    return p


def _gpu_block(smg, inp, d, heads, kv_heads, hd, eps, theta):
    W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
    attn = smg.SelfAttention(smg.Linear(W("qkv")), smg.Linear(W("out")), heads, kv_heads, hd, rope_theta=theta)
    mlp = smg.Mlp.gated(smg.GatedLinear.from_q4(W("gate"), W("up"), smg.Gate.Silu), smg.Linear(W("down")))
    return smg.Block(smg.Norm.rms(inp["norm1"], eps), attn, smg.Norm.rms(inp["norm2"], eps), mlp)


def _check_step(orc, p, got_x, want_x, x0, parts, k_attn, k_mlp):
    """Per element: the attention term's own tolerance, the MLP term's own
    tolerance, and how far the attention half's error moves the MLP term --
    measured by re-running the oracle's MLP half on the post-attention
    residual shifted by the attention tolerance itself (seeded random signs),
    since the MLP term is a function of that residual, not only a sum beside
    it. That response is noise-like over the row (a norm and a 4096-wide
    product between it and the term), so one draw can come out near zero at an
    element where another error pattern of the same size does not: each
    element's allowance is at least four times the response's RMS over the
    row. Then the whole update within 1e-3 in relative norm."""
    err = np.abs(got_x.astype(np.float64) - want_x)
    tol_a = f16_tol(k_attn) * (1 + np.abs(parts["attn"]))
    sign = np.where(np.random.default_rng(7).random(tol_a.size) < 0.5, -1.0, 1.0)
    x1 = parts["x1"].astype(np.float64)
    moved = orc.block_mlp_term((x1 + sign * tol_a).astype(np.float32), p)
    resp = np.abs(moved.astype(np.float64) - parts["mlp"])
    prop = np.maximum(resp, 4.0 * np.sqrt(np.mean(resp * resp)))
    bound = tol_a + f16_tol(k_mlp) * (1 + np.abs(parts["mlp"])) + prop
    assert np.all(err <= bound), float(np.max(err / bound))
    upd_g, upd_w = got_x.astype(np.float64) - x0, want_x.astype(np.float64) - x0
    assert np.linalg.norm(upd_g - upd_w) <= 1e-3 * np.linalg.norm(upd_w)


def test_block_config5_decode_step(smg, orc):
    """Config 5 at full size: d 4096, 32 / 8 heads of 128, SwiGLU 14336, 4096
    cached positions, RoPE 10000, eps 1e-5: one Block::accumulate step against
    the oracle's, and the cache row it appends."""
    import torch
    c = WL.CONFIG5
    d, H, KV, hd, ffn, past = c["d"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"], c["past"]
    inp = WL.block_inputs(d, H, KV, hd, ffn, past, seed=0)
    blk = _gpu_block(smg, inp, d, H, KV, hd, c["eps"], c["theta"])
    cache = blk.cache(past + 8)
    cache.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    x = _f32(inp["x"])
    blk.accumulate(x, cache, 1)
    torch.cuda.synchronize()
    p = _oracle_params(orc, inp, d, H, KV, hd, ffn, c["eps"], c["theta"])
    ck, cv = inp["cache_k"].copy(), inp["cache_v"].copy()
    parts = {}
    want = orc.block_decode(inp["x"], ck, cv, past, p, parts)
    _check_step(orc, p, x.cpu().numpy(), want, inp["x"], parts, H * hd, ffn)
    assert cache.len() == past + 1
    keys = _np16(cache.keys()).reshape(past + 1, KV * hd)
    vals = _np16(cache.values()).reshape(past + 1, KV * hd)
    assert np.array_equal(keys[:past], inp["cache_k"][:past])
    kg, kw = orc.f16_to_f32(keys[past]), orc.f16_to_f32(ck[past])
    assert np.max(np.abs(kg - kw)) <= 4e-3 * (1 + np.max(np.abs(kw)))
    assert max_rel(vals[past], cv[past]) <= f16_tol(d)


@pytest.mark.parametrize("theta", [10000.0, 0.0])
def test_block_decode_steps(smg, orc, theta):
    """Eight decode steps of a small block (d 256, 4 / 2 heads of 64, SwiGLU
    320) from 37 cached positions, with and without RoPE; each step's residual
    against the oracle's fed the same input."""
    import torch
    d, H, KV, hd, ffn, past, eps = 256, 4, 2, 64, 320, 37, 1e-5
    inp = WL.block_inputs(d, H, KV, hd, ffn, past, seed=11, cap_extra=16)
    blk = _gpu_block(smg, inp, d, H, KV, hd, eps, theta)
    cache = blk.cache(past + 16)
    cache.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    p = _oracle_params(orc, inp, d, H, KV, hd, ffn, eps, theta)
    ck, cv = inp["cache_k"].copy(), inp["cache_v"].copy()
    rng = np.random.default_rng(12)
    for step in range(8):
        x0 = (rng.standard_normal(d) * 2).astype(np.float32)
        x = _f32(x0)
        blk.accumulate(x, cache, 1)
        torch.cuda.synchronize()
        parts = {}
        want = orc.block_decode(x0, ck, cv, past + step, p, parts)
        # the oracle's cache continues from the GPU's rows, so each step is
        # checked on the same state
        keys = _np16(cache.keys()).reshape(-1, KV * hd)
        ck[past + step] = keys[past + step]
        cv[past + step] = _np16(cache.values()).reshape(-1, KV * hd)[past + step]
        _check_step(orc, p, x.cpu().numpy(), want, x0, parts, H * hd, ffn)


def test_self_attention_accumulate(smg, orc):
    """SelfAttention::accumulate (self_attention.rs:148-183) on its own: y +=
    out(attention(qkv(x))) for an f16 row, appending the cache."""
    import torch
    d, H, KV, hd, past = 512, 8, 2, 64, 100
    inp = WL.block_inputs(d, H, KV, hd, 64, past, seed=21)
    W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
    attn = smg.SelfAttention(smg.Linear(W("qkv")), smg.Linear(W("out")), H, KV, hd, rope_theta=10000.0)
    cache = attn.cache(past + 4)
    cache.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    x16 = orc.f32_to_f16(np.random.default_rng(22).standard_normal(d).astype(np.float32))
    y0 = np.full(d, 0.25, np.float32)
    y = _f32(y0)
    attn.accumulate(_h16(x16), cache, y, 1)
    torch.cuda.synchronize()
    # the oracle's attention half: the block step without norms or MLP
    qkv = orc.matmul_q4_ep(x16, *inp["qkv"][:2], None, 1, inp["qkv"][2], d, 32)
    ql, kl = H * hd, KV * hd
    cs, sn = orc.rope_angles(orc.rope_inv_freq(hd, 10000.0), past)

    def half(qkv16):
        q = orc.rope_apply(orc.f16_to_f32(qkv16[:ql]), cs, sn)
        k = orc.rope_apply(orc.f16_to_f32(qkv16[ql:ql + kl]), cs, sn)
        ck, cv = inp["cache_k"].copy(), inp["cache_v"].copy()
        ck[past], cv[past] = orc.f32_to_f16(k), qkv16[ql + kl:]
        att = orc.attention_kv_f16(q, ck[:past + 1], cv[:past + 1], past + 1, H, KV, hd,
                                   np.float32(1) / np.sqrt(np.float32(hd)))
        return orc.f16_to_f32(orc.matmul_q4_ep(orc.f32_to_f16(att), *inp["out"][:2], None, 1, d, H * hd, 32))
    term = half(qkv)
    # the qkv projection is itself a GEMV held to f16_tol(d): how far the term
    # moves when it moves by that tolerance (seeded random signs)
    v = orc.f16_to_f32(qkv).astype(np.float64)
    sign = np.where(np.random.default_rng(4).random(v.size) < 0.5, -1.0, 1.0)
    moved = np.abs(half(orc.f32_to_f16((v + sign * f16_tol(d) * (1 + np.abs(v))).astype(np.float32))) - term)
    _check_term(y.cpu().numpy(), y0, term, f16_tol(H * hd), moved)
    assert cache.len() == past + 1


def test_decode_parts_refuse_bad_calls(smg, orc):
    import torch
    d, H, KV, hd, ffn = 256, 4, 2, 64, 320
    inp = WL.block_inputs(d, H, KV, hd, ffn, 2, seed=31)
    blk = _gpu_block(smg, inp, d, H, KV, hd, 1e-5, 10000.0)
    cache = blk.cache(2)
    x = _f32(inp["x"])
    blk.accumulate(x, cache, 1)
    blk.accumulate(x, cache, 1)
    torch.cuda.synchronize()
    with pytest.raises(smg.SmeGemmError, match="KvCache full"):
        blk.accumulate(x, cache, 1)
    with pytest.raises(smg.SmeGemmError, match="KvCache full"):  # rows that do not fit: nothing appended
        c3 = blk.cache(3)
        blk.accumulate(_f32(np.zeros(4 * d, np.float32)), c3, 4)
    assert c3.len() == 0
    with pytest.raises(smg.SmeGemmError, match="heads match"):
        blk.accumulate(x, smg.KvCache(8, 2, 64, 8), 1)
    # a part takes its layers over (the Rust constructors move them): the
    # weights cannot be handed to a second part
    up = smg.Linear(smg.Q4Weights(*inp["gate"][:2], ffn, d))
    smg.Mlp.new(up, smg.Gate.Silu, smg.Linear(smg.Q4Weights(*inp["down"][:2], d, ffn)))
    assert up.q4._h is None
    with pytest.raises(smg.SmeGemmError, match="null weights"):
        smg.Mlp.new(up, smg.Gate.Silu, smg.Linear(smg.Q4Weights(*inp["down"][:2], d, ffn)))


# ---- many rows: causal attention, LayerNorm, prefill through the block ----------------------

@pytest.mark.parametrize("heads,kv_heads,hd,start,rows", [(8, 2, 64, 0, 3), (8, 2, 64, 100, 40), (6, 6, 64, 5, 17),
                                                          (32, 8, 128, 4096, 80), (4, 1, 128, 63, 66),
                                                          (6, 6, 64, 10, 31), (6, 6, 64, 10, 32),
                                                          (2, 2, 256, 10, 40), (16, 2, 64, 30, 48),
                                                          (8, 8, 16, 0, 33)])
def test_attention_causal_rows_match_one_row(smg, orc, heads, kv_heads, hd, start, rows):
    """attention_kv_causal_f16 (kv_attention.rs:140-240): query row i attends
    to keys 0 .. start + i. As the reference's kv_causal_rows_match_one_row
    (tests/correctness/kv_attention.rs:81-165): a block below 32 rows gives
    every row the bits of attention_kv_f16 over its prefix (same splits, same
    q rounding); a larger block runs the matrix-core form (probabilities
    rounded to f16, sums in another order) and each row is within an f16
    rounding of a probability of the one-row call: 2^-11 max |v| (+ f32 sum
    order). Against the oracle's per-row one_row within 1e-4 (1 + max |v|),
    plus that rounding for the larger blocks."""
    import torch
    ld = kv_heads * hd
    rng = np.random.default_rng(start + rows + hd)
    q = (rng.standard_normal(rows * heads * hd) * 4).astype(np.float32)
    k = orc.f32_to_f16(rng.standard_normal((start + rows) * ld).astype(np.float32))
    v = orc.f32_to_f16(rng.standard_normal((start + rows) * ld).astype(np.float32))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    vmax = float(np.max(np.abs(orc.f16_to_f32(v))))
    p_round = 0.0 if rows < 32 else 2.0 ** -11 * vmax + 2e-5 * (1 + vmax)
    out = torch.empty(rows * heads * hd, dtype=torch.float32, device="cuda")
    smg.attention_kv_causal_f16(_f32(q), _h16(k), _h16(v), start, rows, heads, kv_heads, hd, scale, out)
    one = torch.empty(heads * hd, dtype=torch.float32, device="cuda")
    got = out.cpu().numpy().reshape(rows, heads * hd)
    for i in sorted({0, 1, rows // 2, rows - 1} & set(range(rows))):
        smg.attention_kv_f16(_f32(q[i * heads * hd:(i + 1) * heads * hd]), _h16(k), _h16(v), start + i + 1,
                             heads, kv_heads, hd, scale, one)
        torch.cuda.synchronize()
        if rows < 32:
            assert np.array_equal(got[i], one.cpu().numpy()), i
        else:
            assert np.max(np.abs(got[i] - one.cpu().numpy())) <= p_round, i
    want = orc.attention_kv_causal_f16(q, k, v, start, rows, heads, kv_heads, hd, np.float32(scale))
    assert np.max(np.abs(got.ravel() - want)) <= 1e-4 * (1 + vmax) + p_round


@pytest.mark.parametrize("heads,kv_heads,hd", [(6, 6, 64), (8, 2, 64), (4, 4, 128), (12, 4, 72), (64, 1, 32)])
def test_attention_causal_reference_cases(smg, orc, heads, kv_heads, hd):
    """kv_causal_rows_match_one_row's own shapes, blocks and LCG data
    (tests/correctness/kv_attention.rs:81-165): grouped heads with a tile of
    fewer positions than 32 rows (g = 3) or more heads than a workgroup takes
    (g = 64), a ragged head_dim (72), a long prefix. Blocks below 32 rows: each
    row bit for bit the one-row call; larger blocks: within 1e-3 of it, and
    every 37th row and the last within 2e-3 of the f64 attention."""
    import torch
    for start, rows in [(0, 1), (0, 7), (5, 3), (0, 31), (0, 32), (0, 256), (100, 300), (1500, 40)]:
        s = 0xCA05_0000 ^ (heads * 100 + start * 7 + rows)
        ld = kv_heads * hd
        q, s = orc.lcg_fill_f32(s, rows * heads * hd)
        q = q * np.float32(8.0)
        k, s = orc.lcg_fill(s, (start + rows) * ld)
        v, s = orc.lcg_fill(s, (start + rows) * ld)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        out = torch.empty(rows * heads * hd, dtype=torch.float32, device="cuda")
        smg.attention_kv_causal_f16(_f32(q), _h16(k), _h16(v), start, rows, heads, kv_heads, hd, scale, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(rows, heads * hd)
        qr = heads * hd
        one = torch.empty(qr, dtype=torch.float32, device="cuda")
        kd, vd = _h16(k), _h16(v)
        for i in range(rows):
            n = start + i + 1
            smg.attention_kv_f16(_f32(q[i * qr:(i + 1) * qr]), kd, vd, n, heads, kv_heads, hd, scale, one)
            torch.cuda.synchronize()
            tag = (heads, kv_heads, hd, start, rows, i)
            if rows < 32:
                assert np.array_equal(got[i], one.cpu().numpy()), tag
                continue
            assert np.max(np.abs(got[i] - one.cpu().numpy())) < 1e-3, tag
            if i % 37 == 0 or i == rows - 1:
                want = _attn64(q[i * qr:(i + 1) * qr], k[:n * ld], v[:n * ld], n, heads, kv_heads, hd, scale)
                assert np.max(np.abs(got[i].astype(np.float64) - want)) < 2e-3, tag


def test_kv_cache_attend_causal(smg, orc):
    """KvCache::attend_causal (kv_attention.rs:560-578) is the free causal
    function over the cache's last rows; more rows than cached is refused."""
    import torch
    heads, kv_heads, hd, length, rows = 8, 2, 64, 50, 9
    ld = kv_heads * hd
    rng = np.random.default_rng(31)
    k = orc.f32_to_f16(rng.standard_normal(length * ld).astype(np.float32))
    v = orc.f32_to_f16(rng.standard_normal(length * ld).astype(np.float32))
    cache = smg.KvCache(heads, kv_heads, hd, 64)
    cache.extend(_h16(k), _h16(v))
    q = (rng.standard_normal(rows * heads * hd) * 4).astype(np.float32)
    a = torch.empty(rows * heads * hd, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    cache.attend_causal(_f32(q), rows, a)
    smg.attention_kv_causal_f16(_f32(q), _h16(k), _h16(v), length - rows, rows, heads, kv_heads, hd,
                                cache.scale(), b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="attend_causal"):
        cache.attend_causal(_f32(np.zeros(51 * heads * hd, np.float32)), 51,
                            torch.empty(51 * heads * hd, dtype=torch.float32, device="cuda"))


@pytest.mark.parametrize("rows,dim,bias", [(1, 8, False), (3, 100, True), (2, 384, True), (4, 4096, False),
                                           (1, 4099, True)])
def test_layer_norm_within_one_ulp(smg, orc, rows, dim, bias):
    """nn::layer_norm (src/nn.rs:73-86,133-143) into f16: within one f16 ulp
    of the portable two-pass lane_sum form (the sums run in another order)."""
    import torch
    rng = np.random.default_rng(dim + rows)
    x = (rng.standard_normal(rows * dim) * 3 + 0.5).astype(np.float32)
    w = rng.uniform(0.9, 1.1, dim).astype(np.float32)
    b = rng.normal(0, 0.1, dim).astype(np.float32) if bias else None
    y = torch.empty(rows * dim, dtype=torch.float16, device="cuda")
    smg.layer_norm(_f32(x), _f32(w), None if b is None else _f32(b), 1e-5, y)
    torch.cuda.synchronize()
    want = orc.layer_norm_f16(x, w, b, 1e-5, rows)
    got = _np16(y)
    assert ulp_dist(got, want) <= 1
    assert np.mean(got == want) > 0.99


def _rows_vs_oracle(orc, p, x0_rows, got_rows, ck, cv, keys, vals, past, rows, d, k_attn, k_mlp, check_rows):
    """Row r of a block of rows against the oracle's one-row block step at
    position past + r, on the cache state the GPU left for the rows before it
    (the oracle's cache continues from the GPU's rows, as in the decode-step
    test), with the one-row step's bars; the cache row the GPU appended for r
    against the oracle's."""
    kv = ck.shape[1]
    for r in range(rows):
        if r in check_rows:
            parts = {}
            want = orc.block_decode(x0_rows[r], ck, cv, past + r, p, parts)
            _check_step(orc, p, got_rows[r], want, x0_rows[r], parts, k_attn, k_mlp)
            kg, kw = orc.f16_to_f32(keys[past + r]), orc.f16_to_f32(ck[past + r])
            assert np.max(np.abs(kg - kw)) <= 4e-3 * (1 + np.max(np.abs(kw))), r
            assert max_rel(vals[past + r], cv[past + r]) <= f16_tol(d), r
        ck[past + r] = keys[past + r].reshape(kv)
        cv[past + r] = vals[past + r].reshape(kv)


@pytest.mark.parametrize("rows,theta", [(2, 10000.0), (5, 0.0), (12, 10000.0), (40, 10000.0), (40, 0.0)])
def test_block_rows(smg, orc, rows, theta):
    """Block::accumulate with many rows (src/block.rs:90-106; the attention
    half's attend_rows, self_attention.rs:192-240): the qkv, out and MLP
    products over all rows (the 8-row GEMV launches, or the GEMM past them),
    RoPE and the cache append per row, causal attention. Each row against the
    oracle's one-row step at its position (d 256, 4 / 2 heads of 64, SwiGLU
    320, 37 cached positions)."""
    import torch
    d, H, KV, hd, ffn, past, eps = 256, 4, 2, 64, 320, 37, 1e-5
    inp = WL.block_inputs(d, H, KV, hd, ffn, past, seed=13, cap_extra=rows + 4)
    blk = _gpu_block(smg, inp, d, H, KV, hd, eps, theta)
    cache = blk.cache(past + rows + 4)
    cache.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    x0 = (np.random.default_rng(rows).standard_normal((rows, d)) * 2).astype(np.float32)
    x = _f32(x0.ravel())
    blk.accumulate(x, cache, rows)
    torch.cuda.synchronize()
    assert cache.len() == past + rows
    keys = _np16(cache.keys()).reshape(-1, KV * hd)
    vals = _np16(cache.values()).reshape(-1, KV * hd)
    assert np.array_equal(keys[:past], inp["cache_k"][:past])
    p = _oracle_params(orc, inp, d, H, KV, hd, ffn, eps, theta)
    ck, cv = inp["cache_k"].copy(), inp["cache_v"].copy()
    _rows_vs_oracle(orc, p, x0, x.cpu().numpy().reshape(rows, d), ck, cv, keys, vals, past, rows, d, H * hd, ffn,
                    set(range(rows)))


def test_self_attention_rows_match_one_row_calls(smg, orc):
    """SelfAttention::accumulate over m rows equals m one-row calls in order,
    within the two paths' tolerances (the m-row call runs its projections as
    one product and attends causally), and appends the same cache rows."""
    import torch
    d, H, KV, hd, past, m = 512, 8, 2, 64, 100, 24
    inp = WL.block_inputs(d, H, KV, hd, 64, past, seed=23, cap_extra=m + 4)

    def attn():
        W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
        return smg.SelfAttention(smg.Linear(W("qkv")), smg.Linear(W("out")), H, KV, hd, rope_theta=10000.0)
    a1, a2 = attn(), attn()
    c1, c2 = a1.cache(past + m + 4), a2.cache(past + m + 4)
    for c in (c1, c2):
        c.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    x16 = orc.f32_to_f16(np.random.default_rng(24).standard_normal(m * d).astype(np.float32))
    y1 = _f32(np.zeros(m * d, np.float32))
    y2 = _f32(np.zeros(m * d, np.float32))
    a1.accumulate(_h16(x16), c1, y1, m)
    for r in range(m):
        a2.accumulate(_h16(x16[r * d:(r + 1) * d]), c2, y2[r * d:(r + 1) * d], 1)
    torch.cuda.synchronize()
    g1, g2 = y1.cpu().numpy(), y2.cpu().numpy()
    assert np.max(np.abs(g1 - g2) / (1 + np.abs(g2))) <= 2 * f16_tol(H * hd) + 4e-3
    k1, k2 = _np16(c1.keys()), _np16(c2.keys())
    assert c1.len() == c2.len() == past + m
    assert max_rel(k1, k2) <= 2 * f16_tol(d) + 4e-3
    assert max_rel(_np16(c1.values()), _np16(c2.values())) <= 2 * f16_tol(d)


def test_block_config5_prefill_512_rows(smg, orc):
    """Config 5's block at full size over a 512-row prefill after 4096 cached
    positions: the rows against 512 one-row decode steps of a second copy of
    the block (the one-row step is itself held to the oracle at this size),
    the appended cache rows alike; and rows 0, 255 and 511 against the
    oracle's one-row step on the cache the prefill left, at that step's own
    bars. The row-update bound is twice the per-element bar of the update's
    deepest term (the down projection, K = ffn) taken over the whole update,
    in norm: 2 f16_tol(ffn) (sqrt(d) + |u|), as each path is held to the
    oracle at that bar."""
    import torch
    c = WL.CONFIG5
    d, H, KV, hd, ffn, past = c["d"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"], c["past"]
    rows = 512
    inp = WL.block_inputs(d, H, KV, hd, ffn, past, seed=2, cap_extra=rows + 8)
    b1 = _gpu_block(smg, inp, d, H, KV, hd, c["eps"], c["theta"])
    b2 = _gpu_block(smg, inp, d, H, KV, hd, c["eps"], c["theta"])
    c1, c2 = b1.cache(past + rows + 8), b2.cache(past + rows + 8)
    for cc in (c1, c2):
        cc.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    x0 = np.random.default_rng(3).standard_normal((rows, d)).astype(np.float32)
    x1 = _f32(x0.ravel())
    b1.accumulate(x1, c1, rows)
    x2 = _f32(x0.ravel())
    for r in range(rows):
        b2.accumulate(x2[r * d:(r + 1) * d], c2, 1)
    torch.cuda.synchronize()
    g1 = x1.cpu().numpy().reshape(rows, d).astype(np.float64)
    g2 = x2.cpu().numpy().reshape(rows, d).astype(np.float64)
    worst = 0.0
    for r in range(rows):
        u1, u2 = g1[r] - x0[r], g2[r] - x0[r]
        bound = 2 * f16_tol(ffn) * (np.sqrt(d) + np.linalg.norm(u2))
        worst = max(worst, np.linalg.norm(u1 - u2) / bound)
    assert worst <= 1.0, worst
    k1 = _np16(c1.keys()).reshape(-1, KV * hd)
    k2 = _np16(c2.keys()).reshape(-1, KV * hd)
    v1 = _np16(c1.values()).reshape(-1, KV * hd)
    v2 = _np16(c2.values()).reshape(-1, KV * hd)
    assert np.array_equal(k1[:past], k2[:past])
    kf1, kf2 = orc.f16_to_f32(k1[past:]), orc.f16_to_f32(k2[past:])
    assert np.max(np.abs(kf1 - kf2)) <= 8e-3 * (1 + np.max(np.abs(kf2)))
    assert max_rel(v1[past:].ravel(), v2[past:].ravel()) <= 2 * f16_tol(d)
    p = _oracle_params(orc, inp, d, H, KV, hd, ffn, c["eps"], c["theta"])
    ck = np.zeros((past + rows + 8, KV * hd), np.uint16)
    cv = np.zeros_like(ck)
    ck[:past + rows], cv[:past + rows] = k1, v1
    for r in (0, 255, 511):
        parts = {}
        cr, vr = ck.copy(), cv.copy()
        want = orc.block_decode(x0[r], cr, vr, past + r, p, parts)
        _check_step(orc, p, g1[r].astype(np.float32), want, x0[r], parts, H * hd, ffn)


@pytest.mark.parametrize("rows,bias", [(1, True), (1, False), (9, True), (33, False)])
def test_layer_norm_block_gpt2_style(smg, orc, rows, bias):
    """A GPT-2-style block as examples/shakespeare/model.rs:91-112 builds it:
    Norm::layer norms (with and without a bias), multi-head attention
    (heads = kv_heads) without RoPE, Mlp::new(up, Gate::Gelu, down); d 384,
    6 heads of 64, hidden 1536, 20 cached positions. Each row against the
    oracle's one-row step (norm_row's LayerNorm form) on the GPU's cache."""
    import torch
    d, H, hd, ffn, past, eps = 384, 6, 64, 1536, 20, 1e-5
    inp = WL.block_inputs(d, H, H, hd, ffn, past, seed=40 + rows, cap_extra=rows + 4)
    rng = np.random.default_rng(41)
    b1 = rng.normal(0, 0.1, d).astype(np.float32) if bias else None
    b2 = rng.normal(0, 0.1, d).astype(np.float32) if bias else None
    W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
    attn = smg.SelfAttention(smg.Linear(W("qkv")), smg.Linear(W("out")), H, H, hd)
    mlp = smg.Mlp.new(smg.Linear(W("gate")), smg.Gate.Gelu, smg.Linear(W("down")))
    blk = smg.Block(smg.Norm.layer(inp["norm1"], b1, eps), attn, smg.Norm.layer(inp["norm2"], b2, eps), mlp)
    cache = blk.cache(past + rows + 4)
    cache.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    x0 = (rng.standard_normal((rows, d)) * 2).astype(np.float32)
    x = _f32(x0.ravel())
    blk.accumulate(x, cache, rows)
    torch.cuda.synchronize()
    keys = _np16(cache.keys()).reshape(-1, H * hd)
    vals = _np16(cache.values()).reshape(-1, H * hd)
    p = dict(d=d, heads=H, kv_heads=H, head_dim=hd, ffn=ffn, eps=eps, theta=0.0, norm="layer",
             norm1=inp["norm1"], norm2=inp["norm2"], bias1=b1, bias2=b2, act=2)
    for key in ("qkv", "out", "down"):
        q, s, n, k = inp[key]
        p[key] = orc.Q4Lin(q, s, n, k)
    p["up"] = orc.Q4Lin(*inp["gate"])
    ck, cv = inp["cache_k"].copy(), inp["cache_v"].copy()
    _rows_vs_oracle(orc, p, x0, x.cpu().numpy().reshape(rows, d), ck, cv, keys, vals, past, rows, d, H * hd, ffn,
                    set(range(rows)))
