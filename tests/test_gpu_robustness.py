"""Argument checks at the boundary and buffer lifetimes, on the GPU.

- A ROW / COL / TENSOR node with a NULL operand is refused by every entry
  point with SMG_EINVAL and the output left untouched (the reference's rc
  contract, src/kernels/q4/matmul.rs:85-90).
- The Python mirror refuses device tensors the kernels would misread: a dtype
  that is not 16 bits wide, a strided view, too few elements.
- A device-pointer call's scratch (the low-bit quantized rows, the split-K
  GEMM's partial sums) outlives later, larger calls on the same stream: a
  captured graph replays correctly after the pool has grown.
- A device call refuses pageable host memory (epilogue operands, A, C) in
  the mirror and at the C ABI; a host call refuses device operands.
- With SMG_TEST_FAIL_ALLOC=1 every device allocation fails: the calls return
  SMG_ENOMEM with dst untouched, and succeed once it is unset.
- bf16 silu / sigmoid far below zero (where 1 / (1 + e^-x) leaves f32's normal
  range) match the reference's f64 formula bit for bit at the GEMV and GEMM
  stores.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import f16_tol, max_rel

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


def test_split_k_partials_survive_growth_under_a_replayed_graph(smg, orc):
    """A Q4 call whose GEMM splits K is captured (its f32 partials live in the
    stream's partial buffer); then, on the same stream, a split call with far
    more partials (the buffer grows: a new one, the old one retired); every
    replay, with that eager work between, gives the eager call's bits."""
    import torch
    rng = np.random.default_rng(12)
    to_dev = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()  # noqa: E731

    def case(m, n, k):
        q = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
        s = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32))
        a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
        return smg.Q4Weights(q, s, n, k), to_dev(a), orc.matmul_q4_ep(a, q, s, None, m, n, k, 32)

    m, n, k = 48, 1024, 1024          # 4 tiles x 8 slices: 1.5 MB of partials
    w, ad, want = case(m, n, k)
    m2, n2, k2 = 256, 2304, 2048      # 18 tiles x 8 slices: 19 MB
    w2, a2d, want2 = case(m2, n2, k2)
    cd = torch.zeros(m * n, dtype=torch.int16, device="cuda")
    c2d = torch.zeros(m2 * n2, dtype=torch.int16, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        smg.matmul_q4(ad, w, cd, m)  # sizes this stream's partial buffer before capture
        torch.cuda.synchronize()
        eager = cd.cpu().numpy().view(np.uint16).copy()
        with torch.cuda.graph(g, stream=side):
            smg.matmul_q4(ad, w, cd, m)
    torch.cuda.synchronize()
    assert max_rel(eager, want) <= f16_tol(k)
    for rep in range(3):
        cd.zero_()
        with torch.cuda.stream(side):
            smg.matmul_q4(a2d, w2, c2d, m2)  # the grown buffer
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(cd.cpu().numpy().view(np.uint16), eager), f"replay {rep}"
        assert max_rel(c2d.cpu().numpy().view(np.uint16), want2) <= f16_tol(k2), f"large call {rep}"


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


_ALLOC_FAIL_CHILD = r"""
import ctypes as C, os, sys
import numpy as np
sys.path[:0] = sys.argv[1:4]
import smegemm as smg, oracle as orc, torch
from conftest import f16_tol, max_rel
L = smg.lib()
rng = np.random.default_rng(9)
n, k, m = 256, 128, 3
quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
scales = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * (k // 32)).astype(np.float32))
q4 = smg.Q4Weights(quants, scales, n, k)                       # created before the knob is set
codes = rng.integers(0, 256, -(-(k * n) // 4), dtype=np.uint8)
q2 = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(32))
a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
b = orc.f32_to_f16(rng.standard_normal(k * n).astype(np.float32))
ad = torch.from_numpy(a.view(np.int16)).cuda()
bd = torch.from_numpy(b.view(np.int16)).cuda()
cd = torch.full((m * n,), 0x1234, dtype=torch.int16, device="cuda")
# a Q4 call whose GEMM splits K (40 rows, one 128 x 256 tile, K = 512: 4 slices)
ms, ks = 40, 512
qs = rng.integers(0, 256, (ks * n + 1) // 2, dtype=np.uint8)
ss = orc.f32_to_f16(rng.uniform(0.005, 0.02, n * (ks // 32)).astype(np.float32))
q4s = smg.Q4Weights(qs, ss, n, ks)
a_s = orc.f32_to_f16(rng.standard_normal(ms * ks).astype(np.float32))
asd = torch.from_numpy(a_s.view(np.int16)).cuda()
csd = torch.full((ms * n,), 0x1234, dtype=torch.int16, device="cuda")
stream = torch.cuda.current_stream().cuda_stream
torch.cuda.synchronize()

os.environ["SMG_TEST_FAIL_ALLOC"] = "1"
c = np.full(m * n, 0x1234, np.uint16)
rc = L.gemm_gpu_f16f16_q4(m, q4._h, c.ctypes.data, a.ctypes.data, None)
print("host q4 (staging)", rc, flush=True)
assert rc == -2 and np.all(c == 0x1234)
rc = L.gemm_gpu_f16f16_run(m, n, k, c.ctypes.data, 1, n, 0, a.ctypes.data, 1, k, b.ctypes.data, 1, n, 0, 0x3C00)
print("host strided gemm (staging)", rc, flush=True)
assert rc == -2 and np.all(c == 0x1234)
h = C.c_void_p()
rc = L.smg_q4_create(quants.ctypes.data, scales.ctypes.data, None, n, k, 32, C.byref(h))
print("q4 create (weights)", rc, h.value, flush=True)
assert rc == -2 and not h.value
rc = L.smg_lowbit_matmul_dev(m, q2._h, cd.data_ptr(), ad.data_ptr(), None, stream)
print("device q2 (scratch pool)", rc, flush=True)
rc2 = L.smg_gemm_run_dev(0, m, n, k, cd.data_ptr(), 1, n, 0, ad.data_ptr(), 1, k, bd.data_ptr(), 1, n,
                         0, 0x3C00, stream)
print("device strided gemm (scratch pool)", rc2, flush=True)
rc3 = L.smg_q4_matmul_dev(ms, q4s._h, csd.data_ptr(), asd.data_ptr(), None, 0, stream)
print("device q4 split K (partials pool)", rc3, flush=True)
torch.cuda.synchronize()
assert rc == -2 and rc2 == -2 and rc3 == -2 and bool((cd == 0x1234).all()) and bool((csd == 0x1234).all())
assert b"split-K partials hipMalloc" in L.smg_last_error()

del os.environ["SMG_TEST_FAIL_ALLOC"]
rc = L.gemm_gpu_f16f16_q4(m, q4._h, c.ctypes.data, a.ctypes.data, None)
want = orc.matmul_q4_ep(a, quants, scales, None, m, n, k, 32)
print("host q4 after", rc, max_rel(c, want), flush=True)
assert rc == 0 and max_rel(c, want) <= f16_tol(k)
rc = L.smg_gemm_run_dev(0, m, n, k, cd.data_ptr(), 1, n, 0, ad.data_ptr(), 1, k, bd.data_ptr(), 1, n,
                        0, 0x3C00, stream)
torch.cuda.synchronize()
got = cd.cpu().numpy().view(np.uint16)
print("device strided gemm after", rc, max_rel(got, orc.gemm16(a, b, m, n, k)), flush=True)
assert rc == 0 and max_rel(got, orc.gemm16(a, b, m, n, k)) <= f16_tol(k)
rc = L.smg_q4_matmul_dev(ms, q4s._h, csd.data_ptr(), asd.data_ptr(), None, 0, stream)
torch.cuda.synchronize()
got = csd.cpu().numpy().view(np.uint16)
want = orc.matmul_q4_ep(a_s, qs, ss, None, ms, n, ks, 32)
print("device q4 split K after", rc, max_rel(got, want), flush=True)
assert rc == 0 and max_rel(got, want) <= f16_tol(ks)
print("alloc-fail ok", flush=True)
"""


def test_forced_allocation_failure_returns_enomem_and_leaves_output_untouched():
    """With SMG_TEST_FAIL_ALLOC=1 every device allocation fails: the host
    entry points (staging), weight creation and the device forms (scratch
    pool) return SMG_ENOMEM with dst untouched -- the reference's callers take
    their portable path on that (src/kernels/q4/matmul.rs:85-89) -- and once
    the variable is gone the same calls succeed. Run in a child process: the
    staging area and the scratch pool are kept once allocated, so only a
    process that has not allocated them yet sees the failure."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    env = dict(os.environ)
    env.pop("SMG_TEST_FAIL_ALLOC", None)
    r = subprocess.run([sys.executable, "-c", _ALLOC_FAIL_CHILD, here, os.path.join(root, "sme-gemm_amd"),
                        os.path.join(root, "oracle")], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "alloc-fail ok" in r.stdout, r.stdout + r.stderr


def _hip_runtime():
    """The HIP runtime this process has loaded (torch's), through ctypes."""
    with open("/proc/self/maps") as f:
        paths = {ln.split()[-1] for ln in f if "libamdhip64.so" in ln}
    assert paths, "no HIP runtime mapped"
    return C.CDLL(sorted(paths)[0])


def _query_says_unreadable(hip, ptr):
    """True when hipPointerGetAttributes reports ptr as memory no device can
    read (the query fails, or names it unregistered); the error a failed
    query leaves is cleared so no later call reports it."""
    class Attr(C.Structure):
        _fields_ = [("type", C.c_int), ("device", C.c_int), ("devicePointer", C.c_void_p),
                    ("hostPointer", C.c_void_p), ("isManaged", C.c_int), ("allocationFlags", C.c_uint)]
    at = Attr()
    rc = hip.hipPointerGetAttributes(C.byref(at), C.c_void_p(ptr))
    if rc != 0:
        hip.hipGetLastError()
        return True
    return at.type == 0


def test_device_call_refuses_host_operands(smg, orc):
    """A device call hands its pointers to the kernels, so a pageable host
    array there (an epilogue operand, A or C) is refused: by the mirror with
    TypeError / ValueError before any C call, and by the C ABI with SMG_EINVAL
    and C untouched. The C-level calls are made only where the runtime's own
    pointer query (the one the library asks) says the memory is not
    device-readable, so a kernel can never be launched with it. A host call
    given a device tensor as an epilogue operand is refused by the mirror."""
    import torch
    n, k, m = 256, 128, 2
    _, _, w = _q4(smg, orc, n, k, 7)
    ad = torch.zeros(m * k, dtype=torch.float16, device="cuda")
    cd = torch.full((m * n,), 0x1234, dtype=torch.int16, device="cuda")
    host_col = np.zeros(n, np.uint16)
    with pytest.raises(TypeError):
        smg.matmul_q4_ep(ad, w, cd.view(torch.float16), m, smg.Epilogue().add_col(host_col))
    with pytest.raises(TypeError):
        smg.matmul_q4_ep(np.zeros(m * k, np.uint16), w, np.zeros(m * n, np.uint16), m,
                         smg.Epilogue().add_col(torch.zeros(n, dtype=torch.float16, device="cuda")))
    hip = _hip_runtime()
    host_a = np.zeros(m * k, np.uint16)
    if not (_query_says_unreadable(hip, host_col.ctypes.data) and _query_says_unreadable(hip, host_a.ctypes.data)):
        pytest.skip("the runtime reports pageable host memory as device-readable here")
    L = smg.lib()
    stream = torch.cuda.current_stream().cuda_stream
    node = smg.EpNode(4, 0, 0.0, host_col.ctypes.data, 0)
    arr = (smg.EpNode * 1)(node)
    desc = smg.EpDesc16(1, C.cast(arr, C.POINTER(smg.EpNode)))
    rc = L.smg_q4_matmul_dev(m, w._h, cd.data_ptr(), ad.data_ptr(), C.addressof(desc), 0, stream)
    assert rc == -1 and b"epilogue operand" in L.smg_last_error()
    rc = L.smg_q4_matmul_dev(m, w._h, cd.data_ptr(), host_a.ctypes.data, None, 0, stream)
    assert rc == -1 and b"operand pointer" in L.smg_last_error()
    torch.cuda.synchronize()
    assert bool((cd == 0x1234).all())
    # the refusals leave no error behind: a correct device call still runs
    rc = L.smg_q4_matmul_dev(m, w._h, cd.data_ptr(), ad.data_ptr(), None, 0, stream)
    torch.cuda.synchronize()
    assert rc == 0 and bool((cd.view(torch.float16) == 0).all())


def test_device_call_refuses_host_operands_while_capturing(smg, orc):
    """The device entry points' pointer check also runs while the stream is
    being captured into a graph (the query is not a stream operation): a
    pageable host epilogue operand or A is refused with SMG_EINVAL and nothing
    is recorded for it, while a well-formed device call in the same capture is
    recorded and replays correctly. The graph is replayed only when every
    refused call returned before recording, i.e. it holds device pointers only
    (checked by its replay matching the eager result)."""
    import torch
    n, k, m = 256, 128, 2
    _, _, w = _q4(smg, orc, n, k, 8)
    hip = _hip_runtime()
    host_col = np.zeros(n, np.uint16)
    host_a = np.zeros(m * k, np.uint16)
    if not (_query_says_unreadable(hip, host_col.ctypes.data) and _query_says_unreadable(hip, host_a.ctypes.data)):
        pytest.skip("the runtime reports pageable host memory as device-readable here")
    L = smg.lib()
    ad = torch.randn(m * k, dtype=torch.float16, device="cuda")
    cd = torch.full((m * n,), 0x1234, dtype=torch.int16, device="cuda")
    want = torch.empty(m * n, dtype=torch.int16, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager reference (and any scratch sized before capture)
        assert L.smg_q4_matmul_dev(m, w._h, want.data_ptr(), ad.data_ptr(), None, 0, side.cuda_stream) == 0
    torch.cuda.synchronize()
    node = smg.EpNode(4, 0, 0.0, host_col.ctypes.data, 0)
    arr = (smg.EpNode * 1)(node)
    desc = smg.EpDesc16(1, C.cast(arr, C.POINTER(smg.EpNode)))
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            s = side.cuda_stream
            rcs.append(L.smg_q4_matmul_dev(m, w._h, cd.data_ptr(), ad.data_ptr(), C.addressof(desc), 0, s))
            e1 = L.smg_last_error()
            rcs.append(L.smg_q4_matmul_dev(m, w._h, cd.data_ptr(), host_a.ctypes.data, None, 0, s))
            e2 = L.smg_last_error()
            rcs.append(L.smg_q4_matmul_dev(m, w._h, cd.data_ptr(), ad.data_ptr(), None, 0, s))
    torch.cuda.synchronize()
    assert rcs[0] == -1 and b"epilogue operand" in e1, (rcs, e1)
    assert rcs[1] == -1 and b"operand pointer" in e2, (rcs, e2)
    assert rcs[2] == 0, rcs
    assert bool((cd == 0x1234).all())  # nothing ran at capture
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(cd, want)
        cd.fill_(0x1234)
        torch.cuda.synchronize()
