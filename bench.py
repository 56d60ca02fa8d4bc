"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline (the JSON line's `value`): config 1 -- Q4 GEMV, m=1,
K=N=4096, block 32 -- as whole-job HBM throughput in GB/s. A "step" is one
GEMV call on its own copy of the weights: 64 device copies (605 MB) rotate so
every call streams its weights from HBM, not from the 256 MB MALL. The K timed
steps replay as one HIP graph on torch's current stream (launch-bound loop),
bracketed by torch.cuda.synchronize().

`roofline` covers the dominant kernel (the Q4 GEMV): achieved = algorithmic
bytes per call / average kernel duration, the duration measured with HIP
events around the K graph-replayed calls on the stream they run on (so it
includes the graph's inter-kernel gap, reported as `graph_gap_us` from a
graph of near-empty kernels). `traffic` is the HBM bytes per launch read from
the committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary in profiles/ (null if
absent). `extra` reports configs 2-4 the same way (config 4 against the f16
MFMA peak) plus a diagnostic per-launch event time (one event pair per eager
launch, which adds the event overhead). `cpu_baseline` times the C restatement
of the reference's portable path (oracle/) single-threaded on this host for a
bounded sample of config-1 calls.

--calib-copy first runs 16 device copies of 64 MiB (a kernel of known traffic)
so that a rocprofv3 --pmc run of this script can scale its counters.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
                       [--calib-copy]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sme-gemm_amd"))

HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20


def _events(torch, n):
    return [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(n)]


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemv_mfma_config1_traffic.md")


def committed_traffic():
    """HBM bytes per launch of the config-1 GEMV from the committed PMC summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def time_calls(torch, calls, reps: int, warmup: int):
    """Graph-replayed time per call (us; events around the whole replay on the
    stream it runs on) and a diagnostic per-launch time (an event pair around
    each eager launch). `calls` is a list of zero-arg callables launching one
    call each."""
    s = torch.cuda.current_stream()
    for i in range(warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    # per-launch durations
    ev = _events(torch, reps)
    for i in range(reps):
        ev[i][0].record(s)
        calls[i % len(calls)]()
        ev[i][1].record(s)
    torch.cuda.synchronize()
    durs = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
    per_launch = sum(durs) / len(durs)
    # whole job: K calls captured once into a graph, replayed
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(s)
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for i in range(reps):
                calls[i % len(calls)]()
    torch.cuda.synchronize()
    g.replay()  # warm replay
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(s)
    g.replay()
    t1.record(s)
    torch.cuda.synchronize()
    whole = t0.elapsed_time(t1) * 1e3 / reps
    return {"us_kernel_avg": whole, "us_event_per_launch_avg": per_launch,
            "us_event_per_launch_min": durs[0], "us_event_per_launch_median": durs[len(durs) // 2]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="config 1 only")
    ap.add_argument("--calib-copy", action="store_true",
                    help="16 x 64 MiB device copies first (PMC counter scale)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the calls are independent per weight matrix; sharding N across GPUs "
              "is left to the caller); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import smegemm as smg
    import workloads

    if not smg.available():
        raise SystemExit("libsmegemm_gpu.so not loadable or no gfx950 device")
    torch.cuda.init()
    dev = torch.device("cuda:0")
    to_dev = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).to(dev)  # noqa

    if args.calib_copy:
        src = torch.ones(32 << 20, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(16):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # inter-kernel gap of a replayed graph: near-empty kernels (1-element fill)
    tiny = torch.empty(1, dtype=torch.int16, device=dev)
    gap = time_calls(torch, [lambda: tiny.fill_(1)], args.steps, 8)["us_kernel_avg"]

    def rotate(w, per_copy_bytes):
        copies = max(1, -(-(2 * MALL_BYTES + 64 * 2**20) // per_copy_bytes))
        return [w] + [w.clone() for _ in range(copies - 1)]

    # ---- config 1: Q4 GEMV m=1, K=N=4096 ----
    m, n, k = 1, 4096, 4096
    a, quants, scales, _ = workloads.q4_inputs(m, n, k, seed=0)
    w0 = smg.Q4Weights(quants, scales, n, k)
    bytes1 = workloads.q4_bytes(m, n, k)
    ws = rotate(w0, bytes1)
    ad = to_dev(a)
    cs = [torch.empty(m * n, dtype=torch.int16, device=dev) for _ in range(4)]
    calls = [(lambda w=w, c=cs[i % 4]: smg.matmul_q4(ad, w, c, m)) for i, w in enumerate(ws)]
    cold = time_calls(torch, calls, args.steps, args.warmup)
    hot = time_calls(torch, calls[:1], args.steps, args.warmup)
    t_kernel = cold["us_kernel_avg"]
    achieved = bytes1 / (t_kernel * 1e-6) / 1e9
    value = bytes1 / (cold["us_kernel_avg"] * 1e-6) / 1e9

    extra = {"config1_q4_gemv": {
        "bytes": bytes1, "weight_copies": len(ws), "cold": cold, "hot_mall": hot,
        "GBps_cold_kernel": achieved, "GBps_hot_kernel": bytes1 / (hot["us_kernel_avg"] * 1e-6) / 1e9,
        "frac_hbm_cold_kernel": achieved / HBM_PEAK_GBS}}

    if not args.quick:
        # ---- config 2: Q2 ternary, m=1 and m=8, K=4096, N=11008, block 128 ----
        for m2 in (1, 8):
            n2, k2 = 11008, 4096
            a2, codes, sc2 = workloads.q2_inputs(m2, n2, k2, seed=0)
            w2 = smg.Q2Weights(codes, sc2, n2, k2, smg.Q2Params(128))
            b2 = workloads.q2_bytes(m2, n2, k2)
            ws2 = rotate(w2, b2)
            a2d = to_dev(a2)
            c2 = torch.empty(m2 * n2, dtype=torch.int16, device=dev)
            calls2 = [(lambda w=w: smg.matmul_q2(a2d, w, c2, m2)) for w in ws2]
            r = time_calls(torch, calls2, 256, 32)
            rh = time_calls(torch, calls2[:1], 256, 32)
            extra[f"config2_q2_m{m2}"] = {
                "bytes": b2, "cold": r, "hot_mall": rh,
                "GBps_cold_kernel": b2 / (r["us_kernel_avg"] * 1e-6) / 1e9,
                "frac_hbm_cold_kernel": b2 / (r["us_kernel_avg"] * 1e-6) / 1e9 / HBM_PEAK_GBS}
            del ws2
        # ---- config 3: Q1 + add_col + silu, m=1, K=4096, N=14336 ----
        n3, k3 = 14336, 4096
        a3, signs, sc3, bias = workloads.q1_inputs(1, n3, k3, seed=0)
        w3 = smg.Q1Weights(signs, sc3, smg.WeightLayout.OutIn, n3, k3, 128)
        b3 = workloads.q1_bytes(1, n3, k3)
        ws3 = rotate(w3, b3)
        a3d, biasd = to_dev(a3), to_dev(bias)
        c3 = torch.empty(n3, dtype=torch.int16, device=dev)
        ep3 = smg.Epilogue().add_col(biasd).silu()
        calls3 = [(lambda w=w: smg.matmul_q1_ep(a3d, w, c3, 1, ep3)) for w in ws3]
        r = time_calls(torch, calls3, 256, 32)
        rh = time_calls(torch, calls3[:1], 256, 32)
        extra["config3_q1_ep"] = {
            "bytes": b3, "cold": r, "hot_mall": rh,
            "GBps_cold_kernel": b3 / (r["us_kernel_avg"] * 1e-6) / 1e9,
            "frac_hbm_cold_kernel": b3 / (r["us_kernel_avg"] * 1e-6) / 1e9 / HBM_PEAK_GBS}
        del ws3
        # ---- config 4: Q4 GEMM m=512, K=4096, N=14336 + mul_col/add_col/silu ----
        m4, n4, k4 = 512, 14336, 4096
        a4, q4q, q4s, _ = workloads.q4_inputs(m4, n4, k4, seed=0)
        s4, bb4 = workloads.q4_gemm_epilogue_inputs(n4)
        w4 = smg.Q4Weights(q4q, q4s, n4, k4)
        a4d, s4d, b4d = to_dev(a4), to_dev(s4), to_dev(bb4)
        c4 = torch.empty(m4 * n4, dtype=torch.int16, device=dev)
        ep4 = smg.Epilogue().mul_col(s4d).add_col(b4d).silu()
        calls4 = [lambda: smg.matmul_q4_ep(a4d, w4, c4, m4, ep4)]
        r = time_calls(torch, calls4, 20, 3)
        flops = 2.0 * m4 * n4 * k4
        tf = flops / (r["us_kernel_avg"] * 1e-6) / 1e12
        extra["config4_q4_gemm"] = {"flops": flops, "timing": r, "TFLOPS_kernel": tf,
                                    "frac_f16_mfma": tf / F16_MFMA_PEAK_TFLOPS}

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        oracle.lib()
        t0 = time.perf_counter()
        calls_done = 0
        while calls_done < 3 or time.perf_counter() - t0 < 10.0:
            oracle.matmul_q4_ep(a, quants, scales, None, 1, 4096, 4096, 32)
            calls_done += 1
        dt = (time.perf_counter() - t0) / calls_done
        cpu = {"value": bytes1 / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{calls_done} config-1 calls (m=1, K=N=4096) of the portable path "
                         f"restated in C (per-call Q4 dequant + f32 GEMM), "
                         f"{dt * 1e3:.1f} ms/call, single thread"}

    line = {
        "metric": "Q4 GEMV HBM GB/s at K=N=4096 (config 1, m=1)",
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": cold["us_kernel_avg"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded; config 1 distributions)",
        "config": {"workload": "q4_gemv m=1 K=4096 N=4096 block=32, 64 rotating weight copies",
                   "m": 1, "k": 4096, "n": 4096, "block": 32},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": committed_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
        "graph_gap_us": gap,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
