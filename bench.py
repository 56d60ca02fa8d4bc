"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline (the JSON line's `value`): config 1 -- Q4 GEMV, m=1, K=N=4096,
block 32 -- as whole-job HBM throughput in GB/s. A step is one pass of GEMV
calls over 64 device copies of the weights (605 MB, more than twice the
256 MB MALL, so each call streams its weights from HBM: one call per copy,
as a decode step over a 64-layer stack would). The K timed steps are one HIP
graph replayed on torch's current stream, bracketed by
torch.cuda.synchronize(); before the replay the MALL is flushed by READING
1 GiB of other data (a write flush would leave 256 MB of dirty lines whose
write-back the first kernels after it pay for: about 40 us measured, 2 us a
call at 20 calls). HIP events around the replay on that stream give the time
per call, which includes the dispatch of each kernel (`launch_us`: a graph of
empty launches timed the same way).

`roofline` covers the dominant kernel (the Q4 GEMV): achieved = algorithmic
bytes per call / time per call. `traffic` is the HBM bytes per launch from
the committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary in profiles/.
`python bench.py --trace-summary DIR` prints, from a rocprofv3 kernel trace
of this script, each timed replay's span per call (which the line's per-call
times must match) and the average kernel duration inside it.

`extra` holds, timed the same way (every graph at least 256 calls):
  - configs 2-4 (config 4 against the f16 MFMA peak, with the shader clock
    measured right after its GEMMs and torch's dense f16 GEMM of the same shape
    as a same-box floor);
  - config 5, the Llama-style decode block (src/block.rs path) in tokens/s
    and its fraction of 139.5 MB/token at 8 TB/s, over 4 block copies (558 MB,
    a 4-layer model's worth) so each step's weights come from HBM;
  - `floors`: a plain streaming read of each config's bytes over the same
    rotation (the time a single launch reading that much needs on this box),
    and for config 1 the same read followed by a store of the GEMV's output
    (`config1_with_store`: a launch that writes its result pays for it).
`cpu_baseline` is the C restatement of the reference's portable path (oracle/)
on this host: config 1 single-threaded (faithful mode, a bounded sample) and
over `cores` threads (threaded mode, bit-identical); `extra.cpu` the other
configs' samples.

--calib-copy first runs 16 device copies of 64 MiB (a kernel of known traffic)
so that a rocprofv3 --pmc run of this script can scale its counters.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
                       [--only CONFIGS] [--calib-copy] [--trace-summary DIR]
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
FLUSH_BYTES = 1 << 30
MIN_CALLS = 256  # calls per timed graph outside the headline (the graph's fixed start amortized)

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemv_wave_config1_traffic.md")


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


class Timer:
    """Graph-replayed timing of `passes` passes over `calls` (one call per
    weight copy): captured once, warmed by `warmup` eager passes and one
    replay, then -- after a read flush of the MALL -- replayed once between
    events on the replaying stream. Returns microseconds per call."""

    def __init__(self, torch, smg):
        self.torch = torch
        self.smg = smg
        self.flush_buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
        self.mark_buf = torch.zeros(4, dtype=torch.int64, device="cuda")

    def mark(self):
        """A one-wave marker launch (clock_probe of 0 iterations) outside the
        timed region, so a kernel trace of this script shows where each timed
        replay begins and ends."""
        torch = self.torch
        self.smg.lib().smg_clock_probe_dev(self.mark_buf.data_ptr(), 0, torch.cuda.current_stream().cuda_stream)

    def flush(self):
        """Read 1 GiB (4x the MALL) so the cache holds only clean lines of it."""
        torch = self.torch
        rc = self.smg.lib().smg_stream_read_dev(self.flush_buf.data_ptr(), FLUSH_BYTES,
                                                torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError("smg_stream_read_dev failed")

    def __call__(self, calls, passes: int, warmup: int, flush: bool = True, min_calls: int = MIN_CALLS):
        torch = self.torch
        passes = max(passes, -(-min_calls // len(calls)))
        s = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(s)
        with torch.cuda.stream(side):
            for _ in range(max(1, warmup)):  # every call at least once: scratch sized before capture
                for c in calls:
                    c()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                for _ in range(passes):
                    for c in calls:
                        c()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        if flush:
            self.flush()
        self.mark()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(s)
        g.replay()
        t1.record(s)
        self.mark()
        torch.cuda.synchronize()
        n = passes * len(calls)
        del g
        return t0.elapsed_time(t1) * 1e3 / n


def trace_summary(d):
    """Each timed replay in a rocprofv3 kernel trace of this script: the
    dispatches between two marker launches (clock_probe kernels of under
    50 us). Prints the replay's dispatch count, the calls of its first kernel,
    its span (first start to last end) per call, and each kernel's average
    duration inside it. Under the profiler, dispatches of a graph replay are
    time-stamped back to back (the next start is the previous end), so a
    kernel's traced duration includes its dispatch, plus the profiler's own
    per-dispatch cost."""
    import csv
    import glob
    path = sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True))
    if not path:
        raise SystemExit(f"no *kernel_trace.csv under {d}")
    rows = []
    with open(path[0]) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    short = lambda nm: nm.replace("smg::(anonymous namespace)::", "").split("(")[0][:60]  # noqa: E731
    marks = [i for i, r in enumerate(rows) if "clock_probe" in r[2] and r[1] - r[0] < 50_000]
    print("replay  dispatches  calls  span_us  us/call  kernels (count, avg traced us)")
    nrep = 0
    for a, b in zip(marks, marks[1:]):
        rep = rows[a + 1:b]
        if len(rep) < 16:
            continue
        nrep += 1
        first = rep[0][2]
        calls = sum(1 for r in rep if r[2] == first)
        span = (rep[-1][1] - rep[0][0]) / 1e3
        per = {}
        for r in rep:
            per.setdefault(short(r[2]), []).append((r[1] - r[0]) / 1e3)
        ks = "; ".join(f"{k} x{len(v)} {sum(v) / len(v):.2f}" for k, v in per.items())
        print(f"{nrep:6d}  {len(rep):10d}  {calls:5d}  {span:7.1f}  {span / calls:7.3f}  {ks}")


def rotate(w, per_copy_bytes):
    """Enough device copies of a weight set that one pass over them reads
    more than twice the MALL."""
    copies = max(1, -(-(2 * MALL_BYTES + 64 * 2**20) // per_copy_bytes))
    return [w] + [w.clone() for _ in range(copies - 1)]


def stream_floor(smg, torch, timer, nbytes, steps, warmup, out_bytes=0):
    """A plain read of `nbytes` per call over a rotation past the MALL (with
    out_bytes, the same read that then stores that many bytes of output, as a
    GEMV stores its result)."""
    per = (nbytes + 4095) // 4096 * 4096
    copies = max(1, -(-(2 * MALL_BYTES + 64 * 2**20) // per))
    buf = torch.zeros(per * copies // 4, dtype=torch.int32, device="cuda")
    out = torch.empty(max(out_bytes, 2) // 2, dtype=torch.int16, device="cuda")
    base = buf.data_ptr()
    L = smg.lib()
    if out_bytes:
        calls = [(lambda i=i: L.smg_stream_read_store_dev(base + i * per, nbytes // 16 * 16, out.data_ptr(),
                                                          out_bytes, torch.cuda.current_stream().cuda_stream))
                 for i in range(copies)]
    else:
        calls = [(lambda i=i: L.smg_stream_read_dev(base + i * per, nbytes // 16 * 16,
                                                    torch.cuda.current_stream().cuda_stream))
                 for i in range(copies)]
    us = timer(calls, steps, warmup)
    del buf, out
    r = {"bytes": nbytes, "us": us, "GBps": nbytes / (us * 1e-6) / 1e9}
    if out_bytes:
        r["out_bytes"] = out_bytes
    return r


def shader_clock_mhz(smg, torch):
    """Shader clock from one wave's clock64 against the 100 MHz wall clock."""
    import ctypes as C
    out = torch.zeros(3, dtype=torch.int64, device="cuda")
    smg.lib().smg_clock_probe_dev(C.c_void_p(out.data_ptr()), 1 << 18, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ticks, wall = out[0].item(), out[1].item()
    return ticks / wall * 100.0 if wall > 0 else None


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="timed passes (config 1: 64 calls a pass)")
    ap.add_argument("--warmup", type=int, default=5, help="untimed eager passes before capture")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="config 1 only")
    ap.add_argument("--only", default="12345vr",
                    help="configs to run beside config 1 (digits; v: config 1's shape in the bf16 and affine "
                         "forms; r: 8 to 128 rows at config 1's K)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="16 x 64 MiB device copies first (PMC counter scale)")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="summarize a rocprofv3 --kernel-trace CSV output directory of this script and exit")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the calls are "
              "independent per weight matrix; sharding N across GPUs is left to the caller); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    only = "" if args.quick else args.only

    import numpy as np
    import torch

    import smegemm as smg
    import workloads

    if not smg.available():
        raise SystemExit("libsmegemm_gpu.so not loadable or no gfx950 device")
    torch.cuda.init()
    dev = torch.device("cuda:0")
    to_dev = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).to(dev)  # noqa: E731
    timer = Timer(torch, smg)
    steps, warm = args.steps, args.warmup

    if args.calib_copy:
        src = torch.ones(32 << 20, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(16):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    tiny = torch.empty(1, dtype=torch.int16, device=dev)
    launch_us = timer([lambda: tiny.fill_(1)], steps, 8, flush=False, min_calls=1024)

    # ---- config 1: Q4 GEMV m=1, K=N=4096 ----
    m, n, k = 1, 4096, 4096
    a, quants, scales, _ = workloads.q4_inputs(m, n, k, seed=0)
    w0 = smg.Q4Weights(quants, scales, n, k)
    bytes1 = workloads.q4_bytes(m, n, k)
    ws = rotate(w0, bytes1)
    ad = to_dev(a)
    cs = [torch.empty(m * n, dtype=torch.int16, device=dev) for _ in range(4)]
    calls = [(lambda w=w, c=cs[i % 4]: smg.matmul_q4(ad, w, c, m)) for i, w in enumerate(ws)]
    us1 = timer(calls, steps, warm, min_calls=0)  # exactly `steps` passes over the 64 copies
    us1_hot = timer(calls[:1], steps, warm, flush=False)
    achieved = bytes1 / (us1 * 1e-6) / 1e9
    floors = {"config1": stream_floor(smg, torch, timer, bytes1, steps, warm),
              "config1_with_store": stream_floor(smg, torch, timer, bytes1, steps, warm, out_bytes=2 * n)}
    extra = {"config1_q4_gemv": {
        "bytes": bytes1, "weight_copies": len(ws), "us_cold": us1, "us_hot_mall": us1_hot,
        "GBps_cold": achieved, "GBps_hot": bytes1 / (us1_hot * 1e-6) / 1e9,
        "frac_hbm_cold": achieved / HBM_PEAK_GBS,
        "vs_stream_floor": us1 / floors["config1"]["us"],
        "vs_store_floor": us1 / floors["config1_with_store"]["us"],
        "launch_us": launch_us, "kernel_us_est": us1 - launch_us}}
    len_rot1 = len(ws)
    del ws, calls

    if "v" in only:
        # ---- the config-1 shape in the other Q4 forms (same kernel family): bf16
        #      activations and weights, Q4_1 (affine) f16 and bf16 ----
        forms = {}
        for name, bf16, affine in (("bf16", True, False), ("affine_f16", False, True),
                                   ("affine_bf16", True, True)):
            av, qv, sv, mv = workloads.q4_inputs(m, n, k, seed=0, affine=affine)
            p = smg.Q4Params(32).affine() if affine else smg.Q4Params(32)
            wv = smg.Q4Weights.with_params(qv, sv, mv, n, k, p)
            bv = workloads.q4_bytes(m, n, k, affine=affine)
            wsv = rotate(wv, bv)
            avd = to_dev(av)
            if bf16:
                avd = avd.view(torch.float16).float().to(torch.bfloat16).view(torch.int16)
            cv = torch.empty(m * n, dtype=torch.bfloat16 if bf16 else torch.int16, device=dev)
            if bf16:
                avd = avd.view(torch.bfloat16)
            fn = smg.matmul_q4_bf16 if bf16 else smg.matmul_q4
            callsv = [(lambda w=w: fn(avd, w, cv, m)) for w in wsv]
            us = timer(callsv, steps, warm)
            forms[name] = {"bytes": bv, "us_cold": us, "GBps_cold": bv / (us * 1e-6) / 1e9,
                           "frac_hbm_cold": bv / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
            del wsv, callsv
        extra["config1_forms"] = forms

    if "r" in only:
        # ---- rows of prefill at config 1's K: the GEMV up to 32 rows, then the
        # GEMM with K split over the compute units (its tiles are few), beside
        # torch's dense f16 GEMM (hipBLASLt) of the same shape ----
        rows = {}
        for nr in (4096, 14336):
            for mr in (8, 16, 24, 64, 128):
                ar_, qr_, sr_, _ = workloads.q4_inputs(mr, nr, k, seed=0)
                wr = smg.Q4Weights(qr_, sr_, nr, k)
                br = workloads.q4_bytes(mr, nr, k)
                wsr = rotate(wr, br)
                ard = to_dev(ar_)
                cr = torch.empty(mr * nr, dtype=torch.int16, device=dev)
                callsr = [(lambda w=w: smg.matmul_q4(ard, w, cr, mr)) for w in wsr]
                us = timer(callsr, steps, warm)
                rows[f"m{mr}_n{nr}"] = {"bytes": br, "us_cold": us, "GBps_cold": br / (us * 1e-6) / 1e9}
                if mr > 32:
                    fl = 2.0 * mr * nr * k
                    ah = ard.view(torch.float16).view(mr, k)
                    tbs = [torch.randn(k, nr, dtype=torch.float16, device=dev) for _ in range(3)]
                    tcr = torch.empty(mr, nr, dtype=torch.float16, device=dev)
                    us_t = timer([(lambda b=b: torch.matmul(ah, b, out=tcr)) for b in tbs], steps, warm)
                    rows[f"m{mr}_n{nr}"].update({"TFLOPS": fl / (us * 1e-6) / 1e12,
                                                 "torch_dense_f16_gemm_us": us_t})
                    if mr == 64:  # bf16 activations: 16-row GEMV launches
                        callsb = [(lambda w=w: smg.matmul_q4_bf16(ard, w, cr, mr)) for w in wsr]
                        rows[f"m{mr}_n{nr}"]["us_cold_bf16"] = timer(callsb, steps, warm)
                        del callsb
                    del tbs, tcr
                del wsr, callsr
        extra["q4_few_rows_k4096"] = rows

    if "2" in only:
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
            us = timer(calls2, steps, warm)
            ush = timer(calls2[:1], steps, warm, flush=False)
            extra[f"config2_q2_m{m2}"] = {
                "bytes": b2, "us_cold": us, "us_hot_mall": ush, "GBps_cold": b2 / (us * 1e-6) / 1e9,
                "frac_hbm_cold": b2 / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
            del ws2, calls2
        floors["config2_m1"] = stream_floor(smg, torch, timer, workloads.q2_bytes(1, 11008, 4096), steps, warm)
    if "3" in only:
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
        us = timer(calls3, steps, warm)
        ush = timer(calls3[:1], steps, warm, flush=False)
        extra["config3_q1_ep"] = {
            "bytes": b3, "us_cold": us, "us_hot_mall": ush, "GBps_cold": b3 / (us * 1e-6) / 1e9,
            "frac_hbm_cold": b3 / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
        floors["config3"] = stream_floor(smg, torch, timer, b3, steps, warm)
        del ws3, calls3
    if "4" in only:
        # ---- config 4: Q4 GEMM m=512, K=4096, N=14336 + mul_col/add_col/silu ----
        m4, n4, k4 = 512, 14336, 4096
        a4, q4q, q4s, _ = workloads.q4_inputs(m4, n4, k4, seed=0)
        s4, bb4 = workloads.q4_gemm_epilogue_inputs(n4)
        w4 = smg.Q4Weights(q4q, q4s, n4, k4)
        a4d, s4d, b4d = to_dev(a4), to_dev(s4), to_dev(bb4)
        c4 = torch.empty(m4 * n4, dtype=torch.int16, device=dev)
        ep4 = smg.Epilogue().mul_col(s4d).add_col(b4d).silu()
        calls4 = [lambda: smg.matmul_q4_ep(a4d, w4, c4, m4, ep4)]
        us = timer(calls4, steps, 3, flush=False)
        mhz = shader_clock_mhz(smg, torch)  # right after the GEMMs
        flops = 2.0 * m4 * n4 * k4
        tf = flops / (us * 1e-6) / 1e12
        # torch's dense f16 GEMM (hipBLASLt) of the same shape: a same-box floor
        ta = torch.randn(m4, k4, dtype=torch.float16, device=dev)
        tb = torch.randn(k4, n4, dtype=torch.float16, device=dev)
        tc = torch.empty(m4, n4, dtype=torch.float16, device=dev)
        us_t = timer([lambda: torch.matmul(ta, tb, out=tc)], steps, 3, flush=False)
        # the same call with bf16 activations, scales and output (matmul_q4_bf16_ep)
        a4b = a4d.view(torch.float16).float().to(torch.bfloat16)
        s4b, b4b = (t.view(torch.float16).float().to(torch.bfloat16) for t in (s4d, b4d))
        c4b = torch.empty(m4 * n4, dtype=torch.bfloat16, device=dev)
        ep4b = smg.Epilogue(bf16=True).mul_col(s4b).add_col(b4b).silu()
        us_b = timer([lambda: smg.matmul_q4_bf16_ep(a4b, w4, c4b, m4, ep4b)], steps, 3, flush=False)
        props = torch.cuda.get_device_properties(0)
        extra["config4_q4_gemm"] = {
            "flops": flops, "us": us, "TFLOPS": tf, "frac_f16_mfma": tf / F16_MFMA_PEAK_TFLOPS,
            "shader_clock_mhz_after": mhz,
            "shader_clock_mhz_max": getattr(props, "clock_rate", 0) / 1000.0 or None,
            "torch_dense_f16_gemm": {"us": us_t, "TFLOPS": flops / (us_t * 1e-6) / 1e12},
            "bf16": {"us": us_b, "TFLOPS": flops / (us_b * 1e-6) / 1e12,
                     "frac_bf16_mfma": flops / (us_b * 1e-6) / 1e12 / F16_MFMA_PEAK_TFLOPS}}
        del ta, tb, tc, a4b, c4b
    if "5" in only:
        extra["config5_decode_block"] = bench_block(smg, torch, timer, workloads, steps, warm, to_dev)
        # each stage's bytes as one plain read (the floor a separate launch of
        # that size meets), and the whole step's bytes as one read
        c5 = workloads.CONFIG5
        stages = workloads.block_stage_bytes(c5["d"], c5["heads"], c5["kv_heads"], c5["head_dim"], c5["ffn"],
                                             c5["past"] + 1)
        f5 = {k: stream_floor(smg, torch, timer, v, steps, warm) for k, v in stages.items()}
        f5["whole_step"] = stream_floor(smg, torch, timer, extra["config5_decode_block"]["bytes_per_token"],
                                        steps, warm)
        f5["sum_of_stage_floors_us"] = sum(f5[k]["us"] for k in stages)
        floors["config5"] = f5
        extra["config5_mlp"] = bench_mlp(smg, torch, timer, workloads, steps, warm)

    extra["floors"] = floors
    cpu = None
    if not args.no_cpu:
        cpu, extra["cpu"] = cpu_baselines(np, workloads, a, quants, scales, bytes1, only)

    line = {
        "metric": "Q4 GEMV HBM GB/s at K=N=4096 (config 1, m=1)",
        "value": achieved,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": us1 * len_rot1 / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded; config 1 distributions)",
        "config": {"workload": "q4_gemv m=1 K=4096 N=4096 block=32; a step = one call on each of 64 weight "
                               "copies (605 MB, > 2x the MALL), K steps in one graph replay after a 1 GiB read "
                               "flush; value = algorithmic bytes per call / time per call (dispatch included)",
                   "m": 1, "k": 4096, "n": 4096, "block": 32, "calls_per_step": len_rot1},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": committed_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
        "launch_us": launch_us,
    }
    print(json.dumps(line))


def bench_block(smg, torch, timer, workloads, steps, warm, to_dev):
    """Config 5: one decode step of a Llama-style block (d 4096, 32 / 8 heads
    of 128, SwiGLU 14336, 4096 cached positions, RoPE 10000) per call, cycling
    over 4 block copies (each with its own cache) so each step streams its
    139.5 MB from HBM; every captured step appends at position 4096 and the
    replays repeat it."""
    import numpy as np
    c = workloads.CONFIG5
    d, H, KV, hd, ffn, past = c["d"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"], c["past"]
    copies = 4
    blocks, caches, xs = [], [], []
    for i in range(copies):
        inp = workloads.block_inputs(d, H, KV, hd, ffn, past, seed=100 + i)
        W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
        attn = smg.SelfAttention(smg.Linear(W("qkv")), smg.Linear(W("out")), H, KV, hd, rope_theta=c["theta"])
        mlp = smg.Mlp.gated(smg.GatedLinear.from_q4(W("gate"), W("up"), smg.Gate.Silu), smg.Linear(W("down")))
        blk = smg.Block(smg.Norm.rms(inp["norm1"], c["eps"]), attn, smg.Norm.rms(inp["norm2"], c["eps"]), mlp)
        cache = blk.cache(past + 8)  # every step appends at position `past`
        cache.extend(to_dev(inp["cache_k"][:past]), to_dev(inp["cache_v"][:past]))
        if i == 0:
            kv0 = (to_dev(inp["cache_k"][:past]), to_dev(inp["cache_v"][:past]))
        blocks.append(blk)
        caches.append(cache)
        xs.append(torch.from_numpy(inp["x"]).cuda())
        del inp
    torch.cuda.synchronize()

    def step(i):
        caches[i].truncate(past)  # every captured step appends at position `past`
        blocks[i].accumulate(xs[i], caches[i], 1)
    calls = [(lambda i=i: step(i)) for i in range(copies)]
    us = timer(calls, steps, warm)
    us_hot = timer(calls[:1], steps, warm, flush=False)
    nbytes = workloads.block_bytes(d, H, KV, hd, ffn, past + 1)
    tok_s = 1e6 / us
    # prefill: 512 rows in one Block::accumulate (causal among them) after the
    # 4096 cached positions, block copy 0 (its cache holds past + 520 rows)
    rows = 512
    pc = blocks[0].cache(past + rows + 8)
    pc.extend(*kv0)
    xp = torch.from_numpy(np.random.default_rng(5).standard_normal(rows * d).astype(np.float32)).cuda()

    def prefill():
        pc.truncate(past)
        blocks[0].accumulate(xp, pc, rows)
    us_pre = timer([prefill], max(1, steps // 4), 2, flush=False, min_calls=1)
    # FLOPs of the prefill's projections (2 per weight per row) and causal attention
    # (QK and PV: 4 * heads * head_dim per (row, key) pair)
    proj = 2.0 * rows * (d * (H + 2 * KV) * hd + H * hd * d + 3 * ffn * d)
    att = 4.0 * H * hd * sum(past + r + 1 for r in range(rows))
    return {"workload": "Block::accumulate, 1 row, d=4096, 32/8 heads x 128, SwiGLU 14336, "
                        "4096 cached positions, RoPE theta 10000, Q4 block 32; 4 block copies",
            "bytes_per_token": nbytes, "us_per_token": us, "tokens_per_s": tok_s,
            "us_per_token_hot_mall": us_hot, "GBps": nbytes / (us * 1e-6) / 1e9,
            "roofline_tokens_per_s": HBM_PEAK_GBS * 1e9 / nbytes,
            "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, "launches_per_token": 6,
            "prefill_512_rows": {"us": us_pre, "tokens_per_s": rows / (us_pre * 1e-6),
                                 "TFLOPS": (proj + att) / (us_pre * 1e-6) / 1e12,
                                 "workload": "one Block::accumulate of 512 rows after 4096 cached positions "
                                             "(weights and cache MALL-warm: the same call replayed)"}}


def bench_mlp(smg, torch, timer, workloads, steps, warm):
    """Config 5's MLP on one row (d 4096, SwiGLU 14336, Q4 block 32):
    Mlp::accumulate as this library runs it -- the gate/up GEMV with glu at
    its store, then the down GEMV adding into the f32 row, two launches in
    stream order (the GPU form of Mlp::chained, src/mlp.rs:151-234) --
    against the same work as plain calls: the 2n-column GEMV to f16, the glu
    pass, the down GEMV to f16 and the add, four launches whose intermediates
    round-trip through memory. Four weight copies cycle (99 MB each)."""
    import numpy as np
    c = workloads.CONFIG5
    d, ffn = c["d"], c["ffn"]
    inp = workloads.block_inputs(d, 2, 1, 64, ffn, 1, seed=7)
    W = lambda key: smg.Q4Weights(inp[key][0], inp[key][1], inp[key][2], inp[key][3])  # noqa: E731
    gate, up, down = W("gate"), W("up"), W("down")
    copies = 4
    fused, plain = [], []
    for _ in range(copies):
        fused.append(smg.Mlp.gated(smg.GatedLinear.from_q4(gate.clone(), up.clone(), smg.Gate.Silu),
                                   smg.Linear(down.clone())))
        plain.append((smg.GatedLinear.from_q4(gate.clone(), up.clone(), smg.Gate.Silu).inner,
                      smg.Linear(down.clone())))
    x16 = torch.from_numpy(np.random.default_rng(1).standard_normal(d).astype(np.float16)).cuda()
    y = torch.zeros(d, dtype=torch.float32, device="cuda")
    both = torch.empty(2 * ffn, dtype=torch.float16, device="cuda")
    hid = torch.empty(ffn, dtype=torch.float16, device="cuda")
    out = torch.empty(d, dtype=torch.float16, device="cuda")

    def run_plain(i):
        gu, dn = plain[i]
        gu.forward(x16, both, 1)
        smg.glu(both, 1, ffn, smg.Gate.Silu, hid)
        dn.forward(hid, out, 1)
        y.add_(out.float())
    us_fused = timer([(lambda i=i: fused[i].accumulate(x16, y, 1)) for i in range(copies)], steps, warm)
    us_plain = timer([(lambda i=i: run_plain(i)) for i in range(copies)], steps, warm)
    nbytes = workloads.block_stage_bytes(d, 2, 1, 64, ffn, 1)
    mb = nbytes["gate_up"] + nbytes["down"]
    return {"workload": "Mlp::accumulate, 1 row, d=4096, SwiGLU 14336, Q4 block 32; 4 weight copies",
            "bytes": mb, "us_fused": us_fused, "us_plain_calls": us_plain, "speedup": us_plain / us_fused,
            "GBps_fused": mb / (us_fused * 1e-6) / 1e9, "launches": {"fused": 2, "plain": 4}}


def cpu_baselines(np, workloads, a, quants, scales, bytes1, only):
    """The oracle (the reference's portable path restated in C) on this host's
    cores, on bounded samples of each config."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    oracle.lib()
    threads = max(1, min(16, os.cpu_count() or 1))
    model = cpu_model()

    def timed(fn, budget_s, min_calls=1):
        t0 = time.perf_counter()
        calls = 0
        while calls < min_calls or time.perf_counter() - t0 < budget_s:
            fn()
            calls += 1
        return (time.perf_counter() - t0) / calls, calls

    dt1, n1 = timed(lambda: oracle.matmul_q4_ep(a, quants, scales, None, 1, 4096, 4096, 32), 10.0, 3)
    dtt, nt = timed(lambda: oracle.matmul_mt(4, a, quants, scales, 1, 4096, 4096, 32, threads), 3.0, 3)
    cpu = {"value": bytes1 / dt1 / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{n1} config-1 calls (m=1, K=N=4096) of the portable path restated in C "
                     f"(per-call Q4 dequant + f32 GEMM), {dt1 * 1e3:.1f} ms/call, single thread",
           "threaded": {"value": bytes1 / dtt / 1e9, "unit": "GB/s", "cores": threads,
                        "ms_per_call": dtt * 1e3, "calls": nt},
           "cpu_model": model, "host_cpus": os.cpu_count()}
    extra = {}
    if "2" in only:
        a2, codes, sc2 = workloads.q2_inputs(1, 11008, 4096, seed=0)
        d1, c1 = timed(lambda: oracle.matmul_lowbit_ep(2, a2, codes, sc2, 1, 11008, 4096, 128), 3.0, 1)
        dmt, cmt = timed(lambda: oracle.matmul_mt(2, a2, codes, sc2, 1, 11008, 4096, 128, threads), 2.0, 2)
        b = workloads.q2_bytes(1, 11008, 4096)
        extra["config2_q2_m1"] = {"single_GBps": b / d1 / 1e9, "single_ms": d1 * 1e3,
                                  "threaded_GBps": b / dmt / 1e9, "threaded_ms": dmt * 1e3, "cores": threads}
    if "3" in only:
        a3, signs, sc3, bias = workloads.q1_inputs(1, 14336, 4096, seed=0)
        d1, _ = timed(lambda: oracle.matmul_lowbit_ep(1, a3, signs, sc3, 1, 14336, 4096, 128,
                                                      [(4, 0, 0.0, bias, 0)], 3), 3.0, 1)
        b = workloads.q1_bytes(1, 14336, 4096)
        extra["config3_q1_ep"] = {"single_GBps": b / d1 / 1e9, "single_ms": d1 * 1e3}
    if "4" in only:
        # a 16-row slice of config 4 (m=512), threaded; TFLOPS scale with the rows
        mrows = 16
        a4, q4q, q4s, _ = workloads.q4_inputs(mrows, 14336, 4096, seed=0)
        dmt, _ = timed(lambda: oracle.matmul_mt(4, a4, q4q, q4s, mrows, 14336, 4096, 32, threads), 4.0, 1)
        extra["config4_q4_gemm"] = {"sample": f"rows 0..{mrows} of config 4 (the per-call dequant of all "
                                              f"14336 x 4096 weights included), threaded",
                                    "TFLOPS": 2.0 * mrows * 14336 * 4096 / dmt / 1e12, "s_per_call": dmt,
                                    "cores": threads}
    if "5" in only:
        c = workloads.CONFIG5
        d, H, KV, hd, ffn, past = c["d"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"], c["past"]
        inp = workloads.block_inputs(d, H, KV, hd, ffn, past, seed=100)
        p = dict(d=d, heads=H, kv_heads=KV, head_dim=hd, ffn=ffn, eps=c["eps"], theta=c["theta"],
                 norm1=inp["norm1"], norm2=inp["norm2"])
        for key in ("qkv", "out", "down"):
            p[key] = oracle.Q4Lin(*inp[key])
        p["gate_up"] = oracle.Q4Lin(*oracle.q4_interleave32(*inp["gate"][:2], *inp["up"][:2], ffn, d),
                                    2 * ffn, d)
        t0 = time.perf_counter()
        oracle.block_decode(inp["x"], inp["cache_k"], inp["cache_v"], past, p)
        dt = time.perf_counter() - t0
        extra["config5_decode_block"] = {"sample": "one Block::accumulate step of the portable path "
                                                   "restated in C (single thread)",
                                         "tokens_per_s": 1.0 / dt, "s_per_token": dt}
    return cpu, extra


if __name__ == "__main__":
    main()
