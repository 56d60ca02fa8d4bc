"""Host operands flush against inaccessible pages (tests/guard_page.rs:1-160):
every host array an entry point reads or writes -- A, C, the epilogue's
ROW / COL / TENSOR operands, the quants / scales / mins / codes / signs a
weight handle is created from, the dense B a Packed is built from -- either
ENDS at a PROT_NONE page (an overrun faults) or STARTS right after one (an
underrun faults). The host side copies exactly the bytes the header
documents, so the calls must survive. Results are not checked here (the
parity tests do that); the only bar is that nothing touches a guard page.

The calls run in a child process, so a stray host access shows up as that
child's SIGSEGV and a failed test rather than taking the test runner down.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

_CHILD = r"""
import ctypes as C, mmap, sys
import numpy as np
sys.path[:0] = sys.argv[1:3]
import smegemm as smg
import torch  # noqa: F401  (one HIP runtime for the library)

libc = C.CDLL(None, use_errno=True)
libc.mprotect.argtypes = [C.c_void_p, C.c_size_t, C.c_int]
PAGE = mmap.PAGESIZE
maps = []


def guarded(count, dtype, fill, where):
    "count elements flush against a PROT_NONE page: where 'end' or 'start'."
    dtype = np.dtype(dtype)
    nbytes = count * dtype.itemsize
    data_pages = max(1, -(-nbytes // PAGE))
    mm = mmap.mmap(-1, (data_pages + 1) * PAGE)
    base = C.addressof(C.c_char.from_buffer(mm))
    guard_off, data_off = (data_pages * PAGE, data_pages * PAGE - nbytes) if where == "end" else (0, PAGE)
    assert libc.mprotect(base + guard_off, PAGE, 0) == 0, C.get_errno()
    maps.append(mm)
    a = np.frombuffer(mm, dtype=dtype, count=count, offset=data_off)
    a[...] = fill
    return a


SHAPES = [(1, 1, 1), (1, 33, 257), (31, 32, 33), (32, 32, 32), (65, 65, 97), (65, 97, 129),
          (64, 16, 2048), (16, 1024, 129), (3, 200, 300), (8, 130, 513)]
ONE16, ONEB = 0x3C00, 0x3F80
for m, n, k in SHAPES:
    for where in ("end", "start"):
        print("case", m, n, k, where, flush=True)
        g = lambda count, fill=ONE16, dtype=np.uint16: guarded(count, dtype, fill, where)  # noqa: E731
        a = g(m * k, 0x3000)
        col, row, ten = g(n, 0x2E00), g(m, 0x2E00), g(m * n, 0x2E00)
        ep = smg.Epilogue().add_col(col).mul_row(row).add_tensor(ten).silu()
        # Q4, both forms and both output types
        for block in (32, 16):
            nbk = -(-k // block)
            quants = g((k * n + 1) // 2, 0x5A, np.uint8)
            scales, mins = g(n * nbk, 0x2000), g(n * nbk, 0x1000)
            for p, mn in ((smg.Q4Params(block), None), (smg.Q4Params(block).affine(), mins)):
                w = smg.Q4Weights.with_params(quants, scales, mn, n, k, p)
                smg.matmul_q4_ep(a, w, g(m * n, 0), m, ep)
                smg.matmul_q4(a, w, g(m * n, 0), m)
                eb = smg.Epilogue(bf16=True).add_col(col).add_tensor(ten).gelu()
                smg.matmul_q4_bf16_ep(g(m * k, 0x3E00), w, g(m * n, 0), m, eb)
        # Q2 / Q1 on the int8 path and through the MOPA dequant
        nbk = -(-k // 64)
        codes, signs, s = g((k * n + 3) // 4, 0x9C, np.uint8), g((k * n + 7) // 8, 0xA5, np.uint8), g(n * nbk, 0x2000)
        q2 = smg.Q2Weights(codes, s, n, k, smg.Q2Params(64))
        q1 = smg.Q1Weights(signs, s, smg.WeightLayout.InOut, n, k, 64)
        smg.matmul_q2_ep(a, q2, g(m * n, 0), m, ep)
        smg.matmul_q1_ep(a, q1, g(m * n, 0), m, ep)
        smg.matmul_q2_mopa_ep(a, q2, g(m * n, 0), m, ep)
        # dense: prepack from a guarded B, the builder with a column-major C,
        # and the strided unpacked GEMM with a column-major C and alpha
        b = g(k * n, 0x3400)
        packed = smg.prepack_f16(b, n, k)
        smg.Gemm(a, packed, m).col_major_output().add_col(col).mul_row(row).silu().run(g(m * n, 0))
        smg.gemm_f16(m, n, k, g(m * n, ONE16), 1, m, a, k, 1, b, n, 1, 0.5, 1.0)
        bb = g(k * n, 0x3E80)
        smg.gemm_bf16(m, n, k, g(m * n, ONEB), 1, m, g(m * k, 0x3F00), k, 1, bb, n, 1, 0.0, 1.0)
        del maps[:]  # every call above is synchronous: the mappings can go
print("guard pages ok", flush=True)
"""


def test_host_operands_against_guard_pages():
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    r = subprocess.run([sys.executable, "-c", _CHILD, os.path.join(root, "sme-gemm_amd"), here],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and "guard pages ok" in r.stdout, \
        f"rc {r.returncode}\n" + r.stdout[-3000:] + r.stderr[-3000:]
