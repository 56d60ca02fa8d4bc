"""Host-side code checked on the CPU, built with AddressSanitizer and
UndefinedBehaviorSanitizer (host code only; no GPU).

- The device-pointer scratch pool's growth rule (csrc/scratch_pool.h): a
  buffer handed to a stream is never freed or shared while the pool lives.
- The oracle (oracle/oracle.c): every function on ragged shapes.
- The library's host code (csrc/api.hip, csrc/quantize.hip): quantizers,
  descriptor checks, argument refusals.
(The library's own leak check is off: the HIP runtime it links keeps
process-lifetime allocations.)
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def _run(exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_scratch_pool_growth_rule_under_asan(tmp_path):
    exe = str(tmp_path / "scratch_pool_test")
    subprocess.run(["g++", "-std=c++17", *SAN, "-pthread", os.path.join(CPP, "scratch_pool_test.cpp"),
                    "-o", exe], check=True, timeout=300)
    assert "scratch pool ok" in _run(exe)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_oracle_under_asan(tmp_path):
    """Every oracle function on ragged shapes with exactly-sized buffers
    (tests/cpp/oracle_asan_test.c compiles oracle/oracle.c in)."""
    exe = str(tmp_path / "oracle_asan_test")
    subprocess.run(["gcc", "-std=gnu11", *SAN, "-pthread", os.path.join(CPP, "oracle_asan_test.c"), "-o", exe,
                    "-lm"], check=True, timeout=300)
    assert "oracle asan ok" in _run(exe)


HIPCC = "/opt/rocm/bin/hipcc"
# host side only: the device code is the ordinary build
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")
def test_library_host_code_under_asan(tmp_path):
    """csrc/api.hip and csrc/quantize.hip rebuilt with the sanitizers on their
    host side, linked with the library's other objects, driven on the CPU by
    tests/cpp/host_asan_test.cpp: the quantizers, descriptor checks and
    argument refusals (nothing reaches a GPU)."""
    build = os.path.join(ROOT, "sme-gemm_amd", "_build")
    others = [os.path.join(build, f + ".o") for f in ("q4_gemv", "lowbit_gemv", "gemm_mfma", "gemm_q4r",
                                                     "columns", "decode_block", "probes")]
    if not all(os.path.exists(o) for o in others):
        subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "sme-gemm_amd")], check=True, timeout=900)
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *HOST_SAN]
    objs = []
    for src in ("api", "quantize"):
        o = str(tmp_path / (src + ".o"))
        subprocess.run([HIPCC, *flags, "-c", os.path.join(ROOT, "sme-gemm_amd", "csrc", src + ".hip"), "-o", o],
                       check=True, timeout=600, capture_output=True)
        objs.append(o)
    drv = str(tmp_path / "drv.o")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", *HOST_SAN, "-c",
                    os.path.join(CPP, "host_asan_test.cpp"), "-o", drv], check=True, timeout=300,
                   capture_output=True)
    exe = str(tmp_path / "host_asan_test")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-Xarch_host", "-fsanitize=address", "-Xarch_host",
                    "-fsanitize=undefined", *objs, drv, *others, "-o", exe, "-lpthread"], check=True, timeout=300,
                   capture_output=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0 and "host asan ok" in r.stdout, r.stdout + r.stderr
