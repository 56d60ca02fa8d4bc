"""The host-slice forms of the model parts (smg_block_accumulate,
smg_attn_accumulate, smg_mlp_accumulate, smg_q4_accumulate, the KvCache and
attention / norm free functions): the reference's Block / SelfAttention / Mlp /
Linear::accumulate take host slices (src/block.rs:90, src/self_attention.rs:148,
src/mlp.rs:113, src/linear.rs:425). Each host form stages its arrays and runs
the device form's kernels, which are deterministic (no float atomics on these
paths), so the bar is bit-identity with the device form on the same inputs --
the device forms are themselves held to the oracle in test_gpu_block.py -- plus
the contract that a failed call leaves its host outputs untouched.
"""
import numpy as np
import pytest

import workloads as WL

pytestmark = pytest.mark.gpu


def _h16(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.float16)).cuda()


def _f32(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def _bits(t):
    """A device tensor's or host array's raw bits (f32 as uint32, f16 as uint16)."""
    a = t.cpu().numpy() if hasattr(t, "cpu") else np.asarray(t)
    return a.view(np.uint32 if a.dtype.itemsize == 4 else np.uint16).ravel()


def _block_pair(smg, inp, d, heads, kv_heads, hd, eps, theta):
    def one():
        W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
        attn = smg.SelfAttention(smg.Linear(W("qkv")), smg.Linear(W("out")), heads, kv_heads, hd,
                                 rope_theta=theta)
        mlp = smg.Mlp.gated(smg.GatedLinear.from_q4(W("gate"), W("up"), smg.Gate.Silu), smg.Linear(W("down")))
        return smg.Block(smg.Norm.rms(inp["norm1"], eps), attn, smg.Norm.rms(inp["norm2"], eps), mlp)
    return one(), one()


@pytest.mark.parametrize("rows", [1, 7, 40])
def test_block_host_equals_device(smg, orc, rows):
    """Block::accumulate on a host residual: a prefill of `rows` rows then two
    decode rows, against the device form step by step; the caches alike
    (keys_host / values_host against keys() / values())."""
    import torch
    d, H, KV, hd, ffn, past, eps = 256, 4, 2, 64, 320, 21, 1e-5
    inp = WL.block_inputs(d, H, KV, hd, ffn, past, seed=70 + rows, cap_extra=rows + 4)
    hb, db = _block_pair(smg, inp, d, H, KV, hd, eps, 10000.0)
    ch, cd = hb.cache(past + rows + 4), db.cache(past + rows + 4)
    ch.extend(inp["cache_k"][:past], inp["cache_v"][:past])            # host extend
    cd.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    rng = np.random.default_rng(rows)
    for step_rows in (rows, 1, 1):
        x0 = (rng.standard_normal(step_rows * d) * 2).astype(np.float32)
        xh = x0.copy()
        xd = _f32(x0)
        assert hb.accumulate(xh, ch, step_rows) is xh
        db.accumulate(xd, cd, step_rows)
        torch.cuda.synchronize()
        assert not np.array_equal(xh, x0)
        assert np.array_equal(_bits(xh), _bits(xd))
    assert ch.len() == cd.len() == past + rows + 2
    assert np.array_equal(_bits(ch.keys_host()), _bits(cd.keys()))
    assert np.array_equal(_bits(ch.values_host()), _bits(cd.values()))


@pytest.mark.parametrize("m", [1, 5])
def test_self_attention_host_equals_device(smg, orc, m):
    import torch
    d, H, KV, hd, past = 512, 8, 2, 64, 33
    inp = WL.block_inputs(d, H, KV, hd, 64, past, seed=80 + m, cap_extra=m + 4)

    def attn():
        W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
        return smg.SelfAttention(smg.Linear(W("qkv")), smg.Linear(W("out")), H, KV, hd, rope_theta=10000.0)
    ah, ad = attn(), attn()
    ch, cd = ah.cache(past + m + 4), ad.cache(past + m + 4)
    ch.extend(inp["cache_k"][:past], inp["cache_v"][:past])
    cd.extend(_h16(inp["cache_k"][:past]), _h16(inp["cache_v"][:past]))
    x16 = orc.f32_to_f16(np.random.default_rng(m).standard_normal(m * d).astype(np.float32))
    y0 = np.random.default_rng(m + 1).standard_normal(m * d).astype(np.float32)
    yh = y0.copy()
    yd = _f32(y0)
    ah.accumulate(x16, ch, yh, m)
    ad.accumulate(_h16(x16), cd, yd, m)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(yh), _bits(yd))
    assert np.array_equal(_bits(ch.keys_host()), _bits(cd.keys()))


@pytest.mark.parametrize("gated,m", [(True, 1), (True, 12), (False, 3)])
def test_mlp_host_equals_device(smg, orc, gated, m):
    import torch
    d, ffn = 256, 320
    inp = WL.block_inputs(d, 2, 1, 64, ffn, 1, seed=90 + m)

    def mlp():
        W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
        if gated:
            return smg.Mlp.gated(smg.GatedLinear.from_q4(W("gate"), W("up"), smg.Gate.Silu), smg.Linear(W("down")))
        return smg.Mlp.new(smg.Linear(W("gate")), smg.Gate.Gelu, smg.Linear(W("down")))
    mh, md = mlp(), mlp()
    x16 = orc.f32_to_f16(np.random.default_rng(m).standard_normal(m * d).astype(np.float32))
    yh = np.full(m * d, 0.25, np.float32)
    yd = _f32(yh)
    mh.accumulate(x16, yh, m)
    md.accumulate(_h16(x16), yd, m)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(yh), _bits(yd))


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (3, 200, 96), (40, 256, 512)])
def test_linear_host_equals_device(smg, orc, m, n, k):
    """Linear::accumulate with an f16 host x, and with an f32 host x (rounded
    to f16 as ModelFloat::as_f16 does, src/linear.rs:61-66)."""
    import torch
    a, quants, scales, _ = WL.q4_inputs(m, n, k, seed=m + n + 5)
    lh = smg.Linear(smg.Q4Weights(quants, scales, n, k))
    ld = smg.Linear(smg.Q4Weights(quants, scales, n, k))
    y0 = np.random.default_rng(2).standard_normal(m * n).astype(np.float32)
    yh = y0.copy()
    yd = _f32(y0)
    lh.accumulate(a, yh, m)
    ld.accumulate(_h16(a), yd, m)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(yh), _bits(yd))
    yf = y0.copy()
    lh.accumulate(orc.f16_to_f32(a), yf, m)  # f32 values that are exactly the f16 ones
    assert np.array_equal(yf, yh)


def test_attention_and_norms_host_equal_device(smg, orc):
    """attention_kv_f16, attention_kv_causal_f16, KvCache::attend /
    attend_causal, rms_norm and layer_norm on host arrays against the device
    forms."""
    import torch
    H, KV, hd, length, rows = 8, 2, 64, 300, 6
    ld, ql = KV * hd, H * hd
    rng = np.random.default_rng(5)
    k = orc.f32_to_f16(rng.standard_normal(length * ld).astype(np.float32))
    v = orc.f32_to_f16(rng.standard_normal(length * ld).astype(np.float32))
    q = rng.standard_normal(rows * ql).astype(np.float32)
    scale = 1.0 / np.sqrt(hd)
    oh = np.zeros(ql, np.float32)
    od = _f32(oh)
    smg.attention_kv_f16(q[:ql], k, v, length, H, KV, hd, scale, oh)
    smg.attention_kv_f16(_f32(q[:ql]), _h16(k), _h16(v), length, H, KV, hd, scale, od)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(oh), _bits(od))
    start = length - rows
    oh = np.zeros(rows * ql, np.float32)
    od = _f32(oh)
    smg.attention_kv_causal_f16(q, k, v, start, rows, H, KV, hd, scale, oh)
    smg.attention_kv_causal_f16(_f32(q), _h16(k), _h16(v), start, rows, H, KV, hd, scale, od)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(oh), _bits(od))
    cache = smg.KvCache(H, KV, hd, length + 2)
    cache.extend(k, v)
    assert np.array_equal(_bits(cache.keys_host()), k)
    ch = np.zeros(rows * ql, np.float32)
    cache.attend_causal(q, rows, ch)
    assert np.array_equal(_bits(ch), _bits(od))
    c1 = np.zeros(ql, np.float32)
    cache.attend(q[(rows - 1) * ql:], c1)
    assert np.array_equal(_bits(c1), _bits(od)[(rows - 1) * ql:])
    for dim, r in ((100, 3), (4096, 2)):
        x = (rng.standard_normal(r * dim) * 3).astype(np.float32)
        w = rng.uniform(0.9, 1.1, dim).astype(np.float32)
        b = rng.normal(0, 0.1, dim).astype(np.float32)
        for layer in (False, True):
            yh = np.zeros(r * dim, np.float16)
            yd = torch.zeros(r * dim, dtype=torch.float16, device="cuda")
            if layer:
                smg.layer_norm(x, w, b, 1e-5, yh)
                smg.layer_norm(_f32(x), _f32(w), _f32(b), 1e-5, yd)
            else:
                smg.rms_norm(x, w, 1e-5, yh)
                smg.rms_norm(_f32(x), _f32(w), 1e-5, yd)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(yh), _bits(yd)), (dim, layer)
        norm = smg.Norm.layer(w, b, 1e-5)
        yn = np.zeros(r * dim, np.float16)
        norm.forward(x, yn)
        assert np.array_equal(_bits(yn), _bits(yd))


def test_host_forms_leave_outputs_untouched_on_error(smg, orc):
    """A refused host-slice call (rows past the cache, a host/device mix)
    raises and leaves the host arrays and the cache as they were."""
    d, H, KV, hd, ffn, past, eps = 256, 4, 2, 64, 320, 5, 1e-5
    inp = WL.block_inputs(d, H, KV, hd, ffn, past, seed=99, cap_extra=4)
    blk, _ = _block_pair(smg, inp, d, H, KV, hd, eps, 0.0)
    cache = blk.cache(past + 2)
    cache.extend(inp["cache_k"][:past], inp["cache_v"][:past])
    x = np.arange(3 * d, dtype=np.float32)
    before = x.copy()
    with pytest.raises(smg.SmeGemmError, match="KvCache full"):
        blk.accumulate(x, cache, 3)
    assert np.array_equal(x, before)
    assert cache.len() == past
    with pytest.raises(smg.SmeGemmError, match="KvCache full"):
        cache.extend(inp["cache_k"][:3], inp["cache_v"][:3])
    assert cache.len() == past
    y = np.ones(2 * d, np.float32)
    with pytest.raises(ValueError, match="host arrays or all device tensors"):
        smg.Mlp.new(smg.Linear(smg.Q4Weights(*inp["gate"])), smg.Gate.Gelu,
                    smg.Linear(smg.Q4Weights(*inp["down"]))).accumulate(_h16(np.zeros(2 * d, np.uint16)), y, 2)
    assert np.all(y == 1)
