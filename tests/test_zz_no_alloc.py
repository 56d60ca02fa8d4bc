"""smg_lowbit_matmul_dev_noalloc, through the C ABI, against
smg_lowbit_matmul_dev (and the oracle): the same bits on two calls in a row,
the second with a smaller input, for Q2 and Q1 with a fused epilogue, and a
call needing more than SMG_NOALLOC_SCRATCH_BYTES refused with nothing
written. Runs alone in a fresh process or after the other tests."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 4 << 20  # SMG_NOALLOC_SCRATCH_BYTES


def _fns(smg):
    L = smg.lib()
    P, SZ = C.c_void_p, C.c_size_t
    L.smg_lowbit_matmul_dev_noalloc.argtypes = [SZ, P, P, P, P, P]
    return L.smg_lowbit_matmul_dev, L.smg_lowbit_matmul_dev_noalloc


def _run(fn, torch, m, w, ad, n, ep_ptr, fill=0):
    cd = torch.full((m * n,), fill, dtype=torch.int16, device="cuda")
    rc = fn(m, w._h, cd.data_ptr(), ad.data_ptr(), ep_ptr, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return rc, cd.cpu().numpy().view(np.uint16)


# blocks of 128 run on the persistent kernel, which quantizes in-kernel (no
# scratch); blocks of 64 quantize several rows into the static array first
@pytest.mark.parametrize("block", [128, 64])
@pytest.mark.parametrize("kind", [2, 1])
def test_noalloc_matches_the_allocating_entry_point(smg, orc, kind, block):
    import torch
    dev_fn, noalloc_fn = _fns(smg)
    rng = np.random.default_rng(70 + kind + block)
    n, k = 2048, 4096
    nbk = k // block
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * nbk).astype(np.float32))
    if kind == 2:
        codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
        w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block))
    else:
        codes = rng.integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
        w = smg.Q1Weights(codes, scales, smg.WeightLayout.OutIn, n, k, block)
    bias = orc.f32_to_f16(rng.normal(0, 0.5, n).astype(np.float32))
    biasd = torch.from_numpy(bias.view(np.int16)).cuda()
    ep = smg.Epilogue().add_col(biasd).silu()
    d, keep = ep.desc(n)
    ep_ptr = C.addressof(d)
    for m in (8, 3):  # the second call smaller: stale rows of the first stay behind it
        a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
        ad = torch.from_numpy(a.view(np.int16)).cuda()
        rc0, want = _run(dev_fn, torch, m, w, ad, n, ep_ptr)
        rc1, got = _run(noalloc_fn, torch, m, w, ad, n, ep_ptr, fill=0x1234)
        assert rc0 == 0 and rc1 == 0, smg.last_error()
        assert np.array_equal(got, want), f"kind {kind} block {block} m={m}"
        ref = orc.matmul_lowbit_ep(kind, a, codes, scales, m, n, k, block, [(4, 0, 0.0, bias, 0)], 3)
        assert np.array_equal(got, ref), f"kind {kind} block {block} m={m} vs oracle"


def test_noalloc_refuses_calls_past_its_scratch(smg, orc):
    import torch
    _, noalloc_fn = _fns(smg)
    rng = np.random.default_rng(79)
    n, k, block, m = 64, 1 << 19, 128, 8  # m*k = 4 MiB of int8 rows: more than the array
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * (k // block)).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block))
    ad = torch.zeros(m * k, dtype=torch.int16, device="cuda")
    rc, got = _run(noalloc_fn, torch, m, w, ad, n, None, fill=0x1234)
    assert rc == -1 and np.all(got == 0x1234)
    assert "SMG_NOALLOC_SCRATCH_BYTES" in smg.last_error()
    # one row of the same K needs an eighth of that: allowed
    rc, got = _run(noalloc_fn, torch, 1, w, ad[:k], n, None)
    assert rc == 0
    want = orc.matmul_lowbit_ep(2, np.zeros(k, np.uint16), codes, scales, 1, n, k, block)
    assert np.array_equal(got, want)
