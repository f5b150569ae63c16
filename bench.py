#!/usr/bin/env python3
"""Benchmark of neso's hot path on one MI355X: prints ONE JSON line.

A "step" is one FA2 forward launch over BASELINE's headline workload
(B=1, H=16, N=2048, d=64, non-causal, fp16 in / fp32 out), inputs resident
in HBM.  ``value`` = 4*B*H*N^2*d / (ms_per_step) in TFLOP/s.

Launches are captured in a HIP graph (16 per graph) and the graph is
replayed; HIP events recorded on the replay stream bracket the timed
launches.  The per-launch time therefore includes the GPU's dispatch gap
between consecutive kernels but not Python's launch cost, which exceeds the
runtime of the smaller kernels (``eager_ms_per_step`` reports the eager
rate for comparison).  The same line carries:

* ``roofline`` for that kernel against dense-fp16 MFMA peak (2516.6 TFLOP/s
  = 256 CU x 2.4 GHz x 4096 FLOP/clk);
* ``cpu_baseline``: the CPU oracle (torch fp32, all host threads) on the
  same workload, rank 0 only;
* ``qmatmul``: the int4 qmatmul at M=1, K=4096, N=11008 in HBM GB/s
  (algorithmic bytes K*N/2 + (K/32)*N*2 + M*K*2 + M*N*2), over 16 rotated
  weight copies (> 256 MiB, so the Infinity Cache cannot hold them), with
  its own roofline against 8 TB/s and its CPU baseline;
* ``sweep``: the other BASELINE configs (FA2 N sweep, d=128 causal, rel-pos
  N=1500, qmatmul M=16/256), one entry each.

``--calibrate-copy`` instead times a plain device-to-device copy of 256 MiB
(torch's copy kernel), the reference for scaling the FETCH_SIZE/WRITE_SIZE
counters to bytes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]
       python bench.py --calibrate-copy
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

MFMA_F16_PEAK_TFLOPS = 2516.6  # 256 CUs * 2.4 GHz * 4096 dense fp16 FLOP/clk/CU
FP32_MFMA_PEAK_TFLOPS = 157.3  # published dense fp32 MFMA peak
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
METRIC = "FA2 fwd TFLOP/s (d64,N2048) + % MFMA peak; int4 qmatmul HBM GB/s"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--ramp", type=float, default=CLOCK_RAMP_S,
                    help="seconds of untimed load before each measurement (clock ramp); "
                         "0 for counter runs, whose per-dispatch figures do not depend on the clock")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


GRAPH_LAUNCHES = 16


# Seconds the GPU is kept busy with the timed workload before each
# measurement.  An idle MI355X starts a burst of kernels at 1.5-1.7 GHz and
# reaches its sustained ~2.2 GHz only after tens of milliseconds of load;
# without this the first cases would be timed at the idle clock.
CLOCK_RAMP_S = 0.3


def ramp_clock(run_once, torch, seconds=None):
    """Repeat ``run_once()`` (asynchronous GPU work) for ``seconds`` of wall time."""
    seconds = CLOCK_RAMP_S if seconds is None else seconds
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            run_once()
        torch.cuda.synchronize()


def time_launches(launch, steps, warmup, torch, per_graph=GRAPH_LAUNCHES):
    """ms per launch of ``launch(i)``, replayed from a HIP graph.

    ``per_graph`` consecutive launches (i = 0 .. per_graph-1) are captured
    once; the graph is replayed ceil(steps / per_graph) times between two
    events recorded on the current stream, which is the stream the replays
    run on.  ``warmup`` launches run eagerly first (and compile nothing),
    then the graph is replayed for CLOCK_RAMP_S seconds (untimed).
    """
    for i in range(warmup):
        launch(i % per_graph)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    ramp_clock(graph.replay, torch)
    replays = max(1, -(-steps // per_graph))
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / (replays * per_graph)


def time_eager(launch, steps, torch):
    """ms per launch when launched one by one from Python (host-bound for short kernels)."""
    launch(0)
    torch.cuda.synchronize()
    ramp_clock(lambda: launch(0), torch, CLOCK_RAMP_S / 3)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        launch(i)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def measured_traffic(key):
    """HBM bytes per launch from the committed counter summary, or None.

    profiles/traffic.json holds FETCH_SIZE + WRITE_SIZE per dispatch (two
    rocprofv3 --pmc passes over this script) already scaled by the plain-copy
    calibration factor; the counters cannot be read from inside the process.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f)["kernels"].get(key)
    except (OSError, ValueError, KeyError):
        return None
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def best_time(launch, steps, warmup, torch):
    """(ms per launch, mode, graph ms, eager ms): the faster of graph replay and eager launches.

    Short kernels are host-bound when launched from Python, so graph replay
    is their rate; long kernels keep the queue full either way and the
    graph's per-node overhead can make eager launches faster.
    """
    g = time_launches(launch, steps, warmup, torch)
    e = time_eager(launch, min(steps, 64), torch)
    return (g, "graph", g, e) if g <= e else (e, "eager", g, e)


def calibrate_copy(torch):
    """Plain 256 MiB device copy: bytes moved per launch and its time."""
    nbytes = 256 << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    ms = time_launches(lambda i: dst.copy_(src), 20, 3, torch, per_graph=4)
    return {"metric": "device copy GB/s (read + write)", "bytes_read": nbytes,
            "bytes_written": nbytes, "ms_per_copy": round(ms, 6),
            "value": round(2 * nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s"}


def cpu_time(fn, reps):
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def fa2_case(neso_amd, torch, I, B, H, N, d, causal, steps, warmup, seed=0):
    from oracle import attention as A  # FLOP formula only
    q, k, v = (t.cuda() for t in I.fa2_inputs(B, H, N, d, seed=seed))
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    ms, mode, g, e = best_time(lambda i: neso_amd.attention(q, k, v, causal=causal, out=out),
                               steps, warmup, torch)
    flop = A.flops(B, H, N, d, causal)
    return ms, flop / (ms * 1e-3) / 1e12, (q, k, v), {"timing": mode, "graph_ms": round(g, 6),
                                                      "eager_ms": round(e, 6)}


def main():
    global CLOCK_RAMP_S
    args = parse()
    CLOCK_RAMP_S = max(0.0, args.ramp)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        return 2
    import torch

    import neso_amd
    from oracle import inputs as I

    torch.manual_seed(0)
    if args.calibrate_copy:
        print(json.dumps(calibrate_copy(torch)), flush=True)
        return 0
    dev = torch.cuda.get_device_properties(0)
    log(f"device {dev.name} {dev.gcnArchName} CUs={dev.multi_processor_count}")

    # ---- headline: FA2 forward, B1 H16 N2048 d64 non-causal ----
    hb = I.FA2_HEADLINE
    ms, tflops, (q, k, v), tmode = fa2_case(neso_amd, torch, I, hb["B"], hb["H"], hb["N"],
                                            hb["d"], False, args.steps, args.warmup)
    log(f"fa2 headline {ms * 1e3:.2f} us/launch {tflops:.1f} TFLOP/s ({tmode})")
    flop = 4.0 * hb["B"] * hb["H"] * hb["N"] ** 2 * hb["d"]
    result = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "timing": tmode,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "flash_attention_fwd B=1 H=16 N=2048 d=64 non-causal, "
                               "fp16 Q/K/V ~ N(0,1), fp32 accumulation and output",
                   "B": 1, "H": 16, "N": 2048, "d": 64, "causal": False},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic("fa2_headline"),
                     "kernel": "fa2_fast_kernel<64,false,false,2,false>",
                     "algorithmic_flop_per_launch": flop},
    }

    # ---- int4 qmatmul, M=1 (HBM-bound), rotated weights ----
    qc = I.QMM_CONFIGS[0]
    result["qmatmul"] = qmm_case(neso_amd, torch, I, qc, args.steps, args.warmup,
                                 rotate=16, want_cpu=not args.no_cpu)
    log(f"qmm M=1 {result['qmatmul']['value']:.1f} GB/s")

    # ---- CPU baseline (rank 0, N=1): the oracle on the same workload ----
    if not args.no_cpu:
        from oracle import attention as A
        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        qc_, kc_, vc_ = (t.cpu() for t in (q, k, v))
        sec = cpu_time(lambda: A.attention(qc_, kc_, vc_, 1 / 8), reps=3)
        result["cpu_baseline"] = {
            "value": round(flop / sec / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": "oracle.attention (torch fp32 CPU, chunked rows) on the full headline "
                      "workload B1 H16 N2048 d64, median of 3 after 1 warm-up",
            "seconds_per_step": round(sec, 4)}
        log(f"cpu baseline {sec:.3f} s/step")

    if not args.no_sweep:
        result["sweep"] = sweep(neso_amd, torch, I, max(20, args.steps // 4), 5)

    print(json.dumps(result), flush=True)
    return 0


def qmm_case(neso_amd, torch, I, cfg, steps, warmup, rotate=1, want_cpu=False):
    from oracle import qmatmul as Q
    import numpy as np
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    x, codes, scales = I.qmatmul_inputs(M, K, N, seed=0)
    words = torch.from_numpy(Q.pack_int4(codes.numpy()))
    xs = x.cuda()
    ws = [words.cuda() for _ in range(rotate)]
    ss = [scales.cuda() for _ in range(rotate)]
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    launch = lambda i: neso_amd.w4a16_matmul(xs, ws[i % rotate], ss[i % rotate], y, M, N, K, K,
                                             N)
    ms, mode, g_ms, e_ms = best_time(launch, steps, warmup, torch)
    nbytes = Q.algorithmic_bytes(M, N, K)
    gbs = nbytes / (ms * 1e-3) / 1e9
    tflops = Q.flops(M, N, K) / (ms * 1e-3) / 1e12
    out = {"metric": "int4 qmatmul HBM GB/s", "value": round(gbs, 2), "unit": "GB/s",
           "ms_per_step": round(ms, 6),
           "timing": {"timing": mode, "graph_ms": round(g_ms, 6), "eager_ms": round(e_ms, 6)},
           "tflops": round(tflops, 3),
           "config": {"workload": f"w4a16_matmul M={M} K={K} N={N} group=32 zero=8, fp16 "
                                  f"X, fp16 out, {rotate} rotated weight copies",
                      "M": M, "K": K, "N": N},
           "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "traffic": measured_traffic(f"w4a16_M{M}"),
                        "algorithmic_bytes_per_launch": nbytes}}
    if want_cpu:
        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        xc = x.float()
        wdq = torch.from_numpy(Q.dequant_int4(words.numpy(), scales.numpy(), dtype=np.float32))

        def full():
            w = torch.from_numpy(Q.dequant_int4(words.numpy(), scales.numpy(), dtype=np.float32))
            return xc @ w.T

        t_full = cpu_time(full, reps=3)
        t_mm = cpu_time(lambda: xc @ wdq.T, reps=5)
        out["cpu_baseline"] = {
            "value": round(nbytes / t_full / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": "oracle dequant_int4 (numpy) + torch fp32 matmul on the full M=1 "
                      "workload, median of 3; matmul-only with pre-dequantised weights in "
                      "matmul_only_gbs",
            "matmul_only_gbs": round(nbytes / t_mm / 1e9, 3)}
    return out


def sweep(neso_amd, torch, I, steps, warmup):
    rows = []
    for cfg in I.FA2_SWEEP:
        ms, tf, _, tm = fa2_case(neso_amd, torch, I, cfg["B"], cfg["H"], cfg["N"], cfg["d"],
                                 cfg["causal"], steps, warmup)
        rows.append({"kernel": "fa2", **cfg, "us": round(ms * 1e3, 2), "tflops": round(tf, 2),
                     "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "timing": tm["timing"]})
    c = I.FA2_D128
    ms, tf, _, tm = fa2_case(neso_amd, torch, I, c["B"], c["H"], c["N"], c["d"], c["causal"],
                             max(16, steps // 4), 2)
    rows.append({"kernel": "fa2", **c, "us": round(ms * 1e3, 2), "tflops": round(tf, 2),
                 "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "timing": tm["timing"]})
    # fp32 Q/K/V (the reference's default qkv_dtype) at the headline shape:
    # three fp16 MFMAs per product, so the useful-FLOP rate is compared with
    # the fp32 dense MFMA peak, the unit that computes in this precision.
    hb = I.FA2_HEADLINE
    q, k, v = (t.cuda().float() for t in I.fa2_inputs(hb["B"], hb["H"], hb["N"], hb["d"]))
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    ms, mode, _, _ = best_time(lambda i: neso_amd.attention(q, k, v, out=out), steps, warmup,
                               torch)
    tf = 4.0 * hb["B"] * hb["H"] * hb["N"] ** 2 * hb["d"] / (ms * 1e-3) / 1e12
    rows.append({"kernel": "fa2_f32_qkv", **hb, "causal": False, "us": round(ms * 1e3, 2),
                 "tflops": round(tf, 2), "fp32_mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
                 "timing": mode})
    rc = I.RELPOS_CONFIG
    q, k, v, table = (t.cuda() for t in I.relpos_inputs(**rc, seed=0))
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    ms, mode, _, _ = best_time(lambda i: neso_amd.rel_pos_attention(q, k, v, table, out=out),
                               steps, warmup, torch)
    flop = 4.0 * rc["H"] * rc["N"] ** 2 * rc["d"]
    tf = flop / (ms * 1e-3) / 1e12
    rows.append({"kernel": "rel_pos_fa2", **rc, "us": round(ms * 1e3, 2), "tflops": round(tf, 2),
                 "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "timing": mode})
    # Reference-format W8A16 at the size the reference publishes (4096^3,
    # PERFORMANCE.md:61-63 and :77-81: 5,744 and 5,976 GFLOP/s on Apple M2 Max).
    m = n = k = 4096
    a = torch.randn(m, k, dtype=torch.float16, device="cuda")
    b = torch.randint(-128, 128, (k, n), dtype=torch.int8, device="cuda")
    c = torch.empty(m, n, dtype=torch.float32, device="cuda")
    sc = (torch.rand(n, device="cuda") * 0.1 + 0.001).half()
    for name, fn, ref_gflops in (
            ("w8a16_matmul", lambda i: neso_amd.w8a16_matmul(a, b, c, k, k, n, n, M=m, N=n),
             5744.0),
            ("w8a16_scaled_matmul",
             lambda i: neso_amd.w8a16_scaled_matmul(a, b, c, sc, k, k, n, n, M=m, N=n), 5976.0)):
        ms, mode, _, _ = best_time(fn, max(16, steps // 4), 2, torch)
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        rows.append({"kernel": name, "M": m, "N": n, "K": k, "us": round(ms * 1e3, 2),
                     "tflops": round(tf, 2), "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                     "reference_m2max_tflops": ref_gflops / 1e3,
                     "x_reference": round(tf / (ref_gflops / 1e3), 1), "timing": mode})
    for cfg in I.QMM_CONFIGS[1:]:
        r = qmm_case(neso_amd, torch, I, cfg, steps, warmup, rotate=8)
        rows.append({"kernel": "w4a16", **cfg, "us": round(r["ms_per_step"] * 1e3, 2),
                     "gbs": r["value"], "tflops": r["tflops"],
                     "hbm_frac": r["roofline"]["frac"],
                     "mfma_frac": round(r["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                     "timing": r["timing"]["timing"]})
    return rows


if __name__ == "__main__":
    sys.exit(main())
