"""Argument checks at the boundary and buffer lifetimes, on the GPU.

- A ROW / COL / TENSOR node with a NULL operand is refused by every entry
  point with SMG_EINVAL and the output left untouched (the reference's rc
  contract, src/kernels/q4/matmul.rs:85-90).
- The Python mirror refuses device tensors the kernels would misread: a dtype
  that is not 16 bits wide, a strided view, too few elements.
- A device-pointer call's scratch outlives later, larger calls on the same
  stream: a captured graph replays correctly after the pool has grown.
- bf16 silu / sigmoid far below zero (where 1 / (1 + e^-x) leaves f32's normal
  range) match the reference's f64 formula bit for bit at the GEMV and GEMM
  stores.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _q4(smg, orc, n, k, seed):
    rng = np.random.default_rng(seed)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32))
    return quants, scales, smg.Q4Weights(quants, scales, n, k)


def test_null_operand_is_refused_and_output_untouched(smg, orc):
    n, k, m = 256, 128, 1
    quants, scales, w = _q4(smg, orc, n, k, 1)
    a = orc.f32_to_f16(np.ones(m * k, np.float32))
    node = smg.EpNode(4, 0, 0.0, None, 0)  # add_col with no operand
    arr = (smg.EpNode * 1)(node)
    desc = smg.EpDesc16(1, C.cast(arr, C.POINTER(smg.EpNode)))
    L = smg.lib()
    c = np.full(m * n, 0x1234, np.uint16)
    rc = L.gemm_gpu_f16f16_q4(m, w._h, c.ctypes.data, a.ctypes.data, C.addressof(desc))
    assert rc == -1 and np.all(c == 0x1234)
    assert b"null operand" in L.smg_last_error()
    import torch
    ad = torch.from_numpy(a.view(np.int16)).cuda()
    cd = torch.full((m * n,), 0x1234, dtype=torch.int16, device="cuda")
    rc = L.smg_q4_matmul_dev(m, w._h, cd.data_ptr(), ad.data_ptr(), C.addressof(desc), 0,
                             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == -1 and bool((cd == 0x1234).all())


def test_mirror_refuses_device_tensors_the_kernels_would_misread(smg, orc):
    import torch
    n, k, m = 256, 128, 2
    _, _, w = _q4(smg, orc, n, k, 2)
    a = torch.zeros(m * k, dtype=torch.float16, device="cuda")
    with pytest.raises(TypeError):   # 1-byte output: the kernel would store 2*m*n bytes
        smg.matmul_q4(a, w, torch.zeros(m * n, dtype=torch.uint8, device="cuda"), m)
    with pytest.raises(TypeError):   # 4-byte input
        smg.matmul_q4(torch.zeros(m * k, dtype=torch.float32, device="cuda"), w,
                      torch.zeros(m * n, dtype=torch.float16, device="cuda"), m)
    with pytest.raises(ValueError):  # a strided view read as dense
        smg.matmul_q4(torch.zeros(2 * m * k, dtype=torch.float16, device="cuda")[::2], w,
                      torch.zeros(m * n, dtype=torch.float16, device="cuda"), m)
    with pytest.raises(ValueError):
        smg.matmul_q4(a, w, torch.zeros(m * n - 1, dtype=torch.float16, device="cuda"), m)
    with pytest.raises(TypeError):   # a 4-byte epilogue operand
        smg.matmul_q4_ep(a, w, torch.zeros(m * n, dtype=torch.float16, device="cuda"), m,
                         smg.Epilogue().add_col(torch.zeros(n, dtype=torch.float32, device="cuda")))
    assert w.device() == torch.cuda.current_device()


def test_dev_scratch_survives_growth_under_a_replayed_graph(smg, orc):
    """A multi-row *_dev call is captured (its quantized rows live in the
    stream's scratch); then, on the same stream, a call that needs far more
    scratch (the pool grows: a new buffer, the old one retired) and a large
    host-pointer call; the graph's replays still give the reference's bits."""
    import torch
    rng = np.random.default_rng(11)
    n, k, block, m = 1024, 1024, 128, 4
    codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.01, 0.05, n * (k // block)).astype(np.float32))
    w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    want = orc.matmul_lowbit_ep(2, a, codes, scales, m, n, k, block)
    to_dev = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()  # noqa: E731
    ad, cd = to_dev(a), torch.zeros(m * n, dtype=torch.int16, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        smg.matmul_q2(ad, w, cd, m)  # sizes this stream's scratch before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=side):
            smg.matmul_q2(ad, w, cd, m)
    torch.cuda.synchronize()
    # a long-K multi-row call: megabytes of quantized rows, more than the
    # first buffer holds
    n2, k2, m2 = 64, 1 << 18, 8
    codes2 = rng.integers(0, 256, (k2 * n2 + 3) // 4, dtype=np.uint8)
    scales2 = orc.f32_to_f16(rng.uniform(0.01, 0.05, n2 * (k2 // block)).astype(np.float32))
    w2 = smg.Q2Weights(codes2, scales2, n2, k2, smg.Q2Params(block))
    a2 = orc.f32_to_f16(rng.standard_normal(m2 * k2).astype(np.float32))
    want2 = orc.matmul_lowbit_ep(2, a2, codes2, scales2, m2, n2, k2, block)
    a2d, c2d = to_dev(a2), torch.zeros(m2 * n2, dtype=torch.int16, device="cuda")
    for rep in range(3):
        cd.zero_()
        with torch.cuda.stream(side):
            smg.matmul_q2(a2d, w2, c2d, m2)           # the grown scratch
        host_c = np.zeros(m2 * n2, np.uint16)
        smg.matmul_q2(a2, w2, host_c, m2)              # host staging grows too
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(cd.cpu().numpy().view(np.uint16), want), f"replay {rep}"
        assert np.array_equal(c2d.cpu().numpy().view(np.uint16), want2), f"large dev call {rep}"
        assert np.array_equal(host_c, want2), f"large host call {rep}"


@pytest.mark.parametrize("act", [3, 5])
@pytest.mark.parametrize("m", [1, 16])
def test_bf16_logistic_far_below_zero(smg, orc, act, m):
    """Pre-activation values from -130 to -60 (bias on a zero product): the
    bf16 silu of -90 is -7.4e-38, a normal bf16 value, and the sigmoid a bf16
    subnormal; the GEMV (m = 1) and GEMM (m = 16) stores give the oracle's
    bits (the f64 formula rounded to f32, then to bf16)."""
    n, k = 256, 64
    quants, scales, w = _q4(smg, orc, n, k, 3)
    xs = np.concatenate([[-130, -120, -104, -100, -96, -95, -92, -90, -89, -88, -87, -80, -70,
                          -69, -68, -60], np.linspace(-100, -60, n - 16)]).astype(np.float32)
    bias = orc.f32_to_bf16(xs)
    a = np.zeros(m * k, np.uint16)
    got = np.zeros(m * n, np.uint16)
    ep = smg.Epilogue(bf16=True).add_col(bias)
    ep = ep.silu() if act == 3 else ep.sigmoid()
    smg.matmul_q4_bf16_ep(a, w, got, m, ep)
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32, [(4, 0, 0.0, bias, 0)], act,
                            bf16=True)
    assert np.any(want[:n] & 0x7FFF), "some outputs are non-zero in bf16"
    assert np.array_equal(got, want)
