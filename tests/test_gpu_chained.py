"""The chained Q4 GEMV link (q4_chained, src/kernels/q4/matmul.rs:116-164;
gemm_sme_f16f16_q4_chained, csrc/gemm_f16f16_q4.h:541-549) on the GPU.

A chained call gives the plain call's bits (the whole op-graph in the kernel,
as the reference's chained call keeps it), reads A only once `ready` covers
it and raises `done` to n once C is stored. The reference chains an up-GEMV
into a down-GEMV through these words (src/mlp.rs:151-234); here that chain
runs as two kernels on two streams, the consumer awaiting the producer's
`done` word on the device. Outputs are compared bitwise with the plain call
and, to the f16 tolerance, with the CPU oracle.
"""
import ctypes as C
import threading
import time

import numpy as np
import pytest

from conftest import f16_tol, max_rel

pytestmark = pytest.mark.gpu


def _weights(smg, orc, n, k, seed):
    rng = np.random.default_rng(seed)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.002, 0.01, n * -(-k // 32)).astype(np.float32))
    return smg.Q4Weights(quants, scales, n, k), quants, scales


def _dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()


def _host(t):
    return t.cpu().numpy().view(np.uint16)


def test_host_link_waits_for_ready_and_raises_done(smg, orc):
    """Host words: A is written by another thread in four pieces, each
    published through `ready`; the call returns the plain call's bits and
    raises `done` to n."""
    m, n, k = 1, 1536, 2048
    w, quants, scales = _weights(smg, orc, n, k, 11)
    rng = np.random.default_rng(12)
    a_full = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    bias = orc.f32_to_f16(rng.normal(0, 0.1, n).astype(np.float32))
    ep = smg.Epilogue().add_col(bias).silu()
    plain = np.zeros(m * n, np.uint16)
    smg.matmul_q4_ep(a_full, w, plain, m, ep)

    a = np.full(m * k, 0x7E00, np.uint16)  # NaN until written: an early read would show
    ready, done = C.c_size_t(0), C.c_size_t(0)

    def produce():
        for i in range(4):
            time.sleep(0.02)
            lo, hi = i * k // 4, (i + 1) * k // 4
            a[lo:hi] = a_full[lo:hi]
            ready.value = hi

    th = threading.Thread(target=produce)
    th.start()
    c = np.zeros(m * n, np.uint16)
    ok = smg.q4_chained(a, w, c, ep, done=done, ready=ready)
    th.join()
    assert ok, smg.last_error()
    assert done.value == n
    assert np.array_equal(c, plain)
    want = orc.matmul_q4_ep(a_full, quants, scales, None, m, n, k, 32, [(4, 0, 0.0, bias, 0)], 3)
    assert max_rel(c, want) <= f16_tol(k)


def test_host_link_without_words_is_the_plain_call(smg, orc):
    m, n, k = 3, 700, 1000
    rng = np.random.default_rng(13)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.002, 0.01, n * 32).astype(np.float32))
    w = smg.Q4Weights(quants, scales, n, k)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    plain, c = np.zeros(m * n, np.uint16), np.zeros(m * n, np.uint16)
    smg.matmul_q4(a, w, plain, m)
    assert smg.q4_chained(a, w, c, m=m)
    assert np.array_equal(c, plain)


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 1000, 6000), (5, 520, 1024), (8, 96, 8192)])
def test_device_link_same_stream(smg, orc, m, n, k):
    """`ready` already covers A: the chained kernel gives the plain kernel's
    bits, raises `done` to n and leaves the sync words at zero; a second call
    on the same words does the same."""
    import torch
    w, quants, scales = _weights(smg, orc, n, k, m * 7 + n + k)
    rng = np.random.default_rng(n + k)
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    sc = orc.f32_to_f16(rng.uniform(0.5, 1.5, n).astype(np.float32))
    bias = orc.f32_to_f16(rng.normal(0, 0.1, n).astype(np.float32))
    ep = smg.Epilogue().mul_col(_dev(sc)).add_col(_dev(bias)).silu()
    ad = _dev(a)
    plain = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    smg.matmul_q4_ep(ad, w, plain, m, ep)
    ready = torch.tensor([k], dtype=torch.int64, device="cuda")
    sync = torch.zeros(2, dtype=torch.int32, device="cuda")
    for _ in range(2):
        done = torch.zeros(1, dtype=torch.int64, device="cuda")
        c = torch.zeros(m * n, dtype=torch.int16, device="cuda")
        assert smg.q4_chained(ad, w, c, ep, done=done, ready=ready, m=m, sync=sync), smg.last_error()
        torch.cuda.synchronize()
        assert done.item() == n
        assert sync.tolist() == [0, 0]
        assert torch.equal(c, plain)
    want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32,
                            [(5, 0, 0.0, sc, 0), (4, 0, 0.0, bias, 0)], 3)
    assert max_rel(_host(c), want) <= f16_tol(k)


def test_device_chain_across_streams(smg, orc):
    """The reference's up -> down chain (src/mlp.rs:215-231) as two kernels on
    two streams: the down GEMV reads the hidden row only once the up GEMV's
    `done` covers it. Both outputs equal the plain calls' bits."""
    import torch
    k, hid, n = 2048, 3072, 2048
    w_up, q_up, s_up = _weights(smg, orc, hid, k, 21)
    w_dn, q_dn, s_dn = _weights(smg, orc, n, hid, 22)
    rng = np.random.default_rng(23)
    x = orc.f32_to_f16(rng.standard_normal(k).astype(np.float32))
    xd = _dev(x)
    ep_up = smg.Epilogue().silu()
    h_plain = torch.zeros(hid, dtype=torch.int16, device="cuda")
    y_plain = torch.zeros(n, dtype=torch.int16, device="cuda")
    smg.matmul_q4_ep(xd, w_up, h_plain, 1, ep_up)
    smg.matmul_q4(h_plain, w_dn, y_plain, 1)

    for rep in range(3):
        h = torch.zeros(hid, dtype=torch.int16, device="cuda")
        y = torch.zeros(n, dtype=torch.int16, device="cuda")
        d_up = torch.zeros(1, dtype=torch.int64, device="cuda")
        d_dn = torch.zeros(1, dtype=torch.int64, device="cuda")
        s_a = torch.zeros(2, dtype=torch.int32, device="cuda")
        s_b = torch.zeros(2, dtype=torch.int32, device="cuda")
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        sa.wait_stream(torch.cuda.current_stream())
        sb.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(sa):
            assert smg.q4_chained(xd, w_up, h, ep_up, done=d_up, sync=s_a), smg.last_error()
        with torch.cuda.stream(sb):
            assert smg.q4_chained(h, w_dn, y, None, done=d_dn, ready=d_up, sync=s_b), smg.last_error()
        torch.cuda.synchronize()
        assert (d_up.item(), d_dn.item()) == (hid, n), f"rep {rep}"
        assert s_a.tolist() == [0, 0] and s_b.tolist() == [0, 0], f"rep {rep}"
        assert torch.equal(h, h_plain), f"rep {rep}"
        assert torch.equal(y, y_plain), f"rep {rep}"
    want_h = orc.matmul_q4_ep(x, q_up, s_up, None, 1, hid, k, 32, [], 3)
    assert max_rel(_host(h_plain), want_h) <= f16_tol(k)


def test_device_link_wait_expires_cleanly(smg, orc):
    """A `ready` that nobody raises: every workgroup's bounded wait (300 us)
    expires, nothing is stored, `done` stays put and sync[1] reports it; the
    same sync words then serve a good call once sync[1] is cleared."""
    import torch
    m, n, k = 1, 512, 1024
    w, _, _ = _weights(smg, orc, n, k, 31)
    a = orc.f32_to_f16(np.random.default_rng(32).standard_normal(m * k).astype(np.float32))
    ad = _dev(a)
    ready = torch.zeros(1, dtype=torch.int64, device="cuda")
    done = torch.zeros(1, dtype=torch.int64, device="cuda")
    sync = torch.zeros(2, dtype=torch.int32, device="cuda")
    c = torch.full((m * n,), 0x1234, dtype=torch.int16, device="cuda")
    assert smg.q4_chained(ad, w, c, None, done=done, ready=ready, sync=sync, wait_us=300)
    torch.cuda.synchronize()
    assert done.item() == 0
    assert sync.tolist() == [0, 1]
    assert bool((c == 0x1234).all())
    sync.zero_()
    ready.fill_(k)
    plain = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    smg.matmul_q4(ad, w, plain, m)
    assert smg.q4_chained(ad, w, c, None, done=done, ready=ready, sync=sync)
    torch.cuda.synchronize()
    assert done.item() == n and sync.tolist() == [0, 0]
    assert torch.equal(c, plain)


def test_device_link_outside_its_domain_returns_false(smg, orc):
    """Affine weights (or block < 32) are not served by the device link: False,
    with the reason, and nothing raised."""
    import torch
    m, n, k = 1, 64, 256
    rng = np.random.default_rng(41)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(np.full(n * (k // 32), 0.01, np.float32))
    mins = orc.f32_to_f16(np.full(n * (k // 32), -0.05, np.float32))
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, smg.Q4Params(32).affine())
    done = torch.zeros(1, dtype=torch.int64, device="cuda")
    sync = torch.zeros(2, dtype=torch.int32, device="cuda")
    c = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    ad = _dev(orc.f32_to_f16(rng.standard_normal(k).astype(np.float32)))
    assert not smg.q4_chained(ad, w, c, None, done=done, sync=sync)
    assert "scale-only" in smg.last_error()
    torch.cuda.synchronize()
    assert done.item() == 0


def test_device_link_wait_expiry_is_reported_without_done(smg, orc):
    """With `ready` and no `done`, an expired wait still shows in sync[1], and
    nothing is stored; without sync words the call is refused."""
    import torch
    m, n, k = 2, 256, 512
    w, _, _ = _weights(smg, orc, n, k, 51)
    ad = _dev(orc.f32_to_f16(np.random.default_rng(52).standard_normal(m * k).astype(np.float32)))
    ready = torch.zeros(1, dtype=torch.int64, device="cuda")
    sync = torch.zeros(2, dtype=torch.int32, device="cuda")
    c = torch.full((m * n,), 0x1234, dtype=torch.int16, device="cuda")
    assert not smg.q4_chained(ad, w, c, None, ready=ready, m=m)
    assert "sync" in smg.last_error()
    assert smg.q4_chained(ad, w, c, None, ready=ready, m=m, sync=sync, wait_us=200)
    torch.cuda.synchronize()
    assert sync.tolist() == [0, 1]
    assert bool((c == 0x1234).all())
