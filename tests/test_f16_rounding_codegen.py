"""f32_to_f16 (sme-gemm_amd/csrc/common.cuh) rounds the f32 value it is given:
the reference computes in f32 and rounds that to f16 (q * scale at
kv_attention.rs:298-302, glu's act(gate) * up at linear.rs:815-826). hipcc may
otherwise fold the producing multiply into one v_fma_mixlo_f16, which rounds
the exact product to f16 once. Compiles a small kernel for gfx950 (no GPU
needed) and reads its AMD assembly."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"

SRC = r'''
#include "common.cuh"
__global__ void probe(const float *a, const float *b, float s, unsigned short *o) {
    const int i = threadIdx.x;
    o[i] = smg::f32_to_f16(a[i] * s);
    o[64 + i] = smg::f32_to_f16(smg::glu_act(3, a[i]) * b[i]);
}
'''


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_f16_conversion_is_not_fused(tmp_path):
    src = tmp_path / "probe.hip"
    src.write_text(SRC)
    out = tmp_path / "probe.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
           "-I", os.path.join(ROOT, "sme-gemm_amd", "csrc"), str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    asm = out.read_text()
    assert "v_cvt_f16_f32" in asm
    assert "v_fma_mixlo_f16" not in asm and "v_mad_mixlo_f16" not in asm
    assert "v_fma_mixhi_f16" not in asm and "v_mad_mixhi_f16" not in asm
