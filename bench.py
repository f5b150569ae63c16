#!/usr/bin/env python3
"""Benchmark of neso's hot path on one MI355X: prints ONE JSON line.

A "step" is one FA2 forward launch over BASELINE's headline workload
(B=1, H=16, N=2048, d=64, non-causal, fp16 in / fp32 out), inputs resident
in HBM.  ``value`` = 4*B*H*N^2*d / ms_per_step in TFLOP/s, where
``ms_per_step`` is the time of exactly ``--steps`` consecutive launches
(captured in one HIP graph, replayed once between two HIP events on the
replay stream, bracketed by device synchronisation) divided by ``--steps``;
it includes the GPU's dispatch gap between consecutive kernels but not
Python's launch cost.  ``timing`` adds the median (and 10th/90th
percentiles) over 64 separately timed replays of a 16-launch graph, and the
eager rate (launches one by one from Python, host-bound for short kernels).

The same line carries:

* ``roofline`` for that kernel against dense-fp16 MFMA peak (2516.6 TFLOP/s
  = 256 CU x 2.4 GHz x 4096 FLOP/clk), with the HBM traffic per launch from
  the committed counter summary, and ``roofline.clock``: the shader clock
  sampled over replays right after the timed ones (the part lowers its clock
  under MFMA load), the peak at that clock, and board power and clock after
  a 1 s soak;
* ``cpu_baseline``: the CPU oracle (torch fp32, all host threads) on the
  same workload, with the host CPU model;
* ``qmatmul``: the int4 qmatmul at M=1, K=4096, N=11008 in HBM GB/s
  (algorithmic bytes K*N/2 + (K/32)*N*2 + M*K*2 + M*N*2), over 16 rotated
  weight copies (> 256 MiB, more than the Infinity Cache holds), with its
  own roofline against 8 TB/s and its CPU baseline, and ``roofline.floor``:
  at the GEMV's grid, in the same run, an empty kernel and a read-only
  stream of the same bytes over 16 rotated buffers (what the launch costs
  when it only moves its bytes);
* ``sweep``: every other BASELINE config (FA2 config 1 and the N sweep,
  d=128 causal, rel-pos N=1500, qmatmul M=16/256), the GPU rel-pos bias
  precompute at config 4's shape, the fp32-input FA2 at d=64 and d=128 and
  the reference-format W8A16 at 4096^3, each with its GPU rate, its
  roofline fraction and its CPU baseline.

``--case NAME`` runs one workload only (for counter runs under rocprofv3);
``--calibrate-copy`` times a plain 256 MiB device-to-device copy, the
reference for scaling the FETCH_SIZE/WRITE_SIZE counters to bytes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]
       python bench.py --case fa2_headline|fa2_d128|relpos|w4a16_m1|... [--steps K]
       python bench.py --calibrate-copy
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

MFMA_F16_PEAK_TFLOPS = 2516.6  # 256 CUs * 2.4 GHz * 4096 dense fp16 FLOP/clk/CU
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
METRIC = "FA2 fwd TFLOP/s (d64,N2048) + % MFMA peak; int4 qmatmul HBM GB/s"
GRAPH_LAUNCHES = 16
MEDIAN_REPLAYS = 64
ROTATE = 16  # weight copies for the qmatmul cases: 16 x 24.2 MB > 256 MB Infinity Cache

# Seconds the GPU is kept busy with the timed workload before each
# measurement.  An idle MI355X starts a burst of kernels at 1.5-1.7 GHz and
# reaches its sustained ~2.2 GHz only after tens of milliseconds of load;
# without this the first cases would be timed at the idle clock.
CLOCK_RAMP_S = 0.3


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--case", default=None, help="run one workload only (see CASES)")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--ramp", type=float, default=CLOCK_RAMP_S,
                    help="seconds of untimed load before each measurement (clock ramp); "
                         "0 for counter runs, whose per-dispatch figures do not depend on the clock")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def ramp_clock(run_once, torch):
    """Repeat ``run_once()`` (asynchronous GPU work) for CLOCK_RAMP_S of wall time."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < CLOCK_RAMP_S:
        for _ in range(8):
            run_once()
        torch.cuda.synchronize()


def capture(launch, n, torch):
    """A HIP graph of launch(0) .. launch(n-1) on a side stream."""
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n):
            launch(i)
    return graph


def time_case(launch, steps, warmup, torch, power=False):
    """Per-launch timing of ``launch(i)``.

    Returns (ms per launch over exactly ``steps`` launches, timing dict).
    The ``steps`` launches are one graph replayed once between HIP events on
    the current stream (the graph replays on it), with device
    synchronisation on both sides.  The dict adds the median / p10 / p90
    over MEDIAN_REPLAYS separately timed replays of a GRAPH_LAUNCHES-launch
    graph, the shader clock sampled over ~3 ms of further replays, the eager
    (one-by-one from Python) rate and, with ``power``, the board power after
    a 1 s soak.
    """
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    g_steps = capture(launch, steps, torch)
    g_small = capture(launch, GRAPH_LAUNCHES, torch)
    g_small.replay()
    torch.cuda.synchronize()
    ramp_clock(g_small.replay, torch)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * MEDIAN_REPLAYS + 2)]
    torch.cuda.synchronize()
    ev[0].record()
    g_steps.replay()
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / steps
    for r in range(MEDIAN_REPLAYS):
        ev[2 + 2 * r].record()
        g_small.replay()
        ev[3 + 2 * r].record()
    # The shader clock over further replays right after (untimed: the
    # sampler's wave on one CU measurably slows that CU's workgroup).
    clock = ClockSampler(torch)
    n_clock = int(3.0 / max(ms * GRAPH_LAUNCHES, 1e-3)) + 1  # ~3 ms of replays
    clock.start()
    for _ in range(n_clock):
        g_small.replay()
    torch.cuda.synchronize()
    per = sorted(ev[2 + 2 * r].elapsed_time(ev[3 + 2 * r]) / GRAPH_LAUNCHES
                 for r in range(MEDIAN_REPLAYS))
    # Eager launches (host-bound for short kernels; reported for comparison).
    n_eager = min(steps, 64)
    ev[0].record()
    for i in range(n_eager):
        launch(i)
    ev[1].record()
    torch.cuda.synchronize()
    eager = ev[0].elapsed_time(ev[1]) / n_eager
    timing = {"graph_ms": round(ms, 6), "launches_timed": steps,
              "median_ms": round(statistics.median(per), 6),
              "p10_ms": round(per[len(per) // 10], 6),
              "p90_ms": round(per[(9 * len(per)) // 10], 6),
              "median_samples": MEDIAN_REPLAYS, "launches_per_sample": GRAPH_LAUNCHES,
              "eager_ms": round(eager, 6),
              "clock_mhz": clock.mhz()}
    if power:
        timing["power"] = board_power(g_small, torch)
    return ms, timing


class ClockSampler:
    """Shader clock while the GPU runs other work: ``neso_clock_sample`` puts
    one wave on a second stream that records (shader clock, 100 MHz reference
    clock) pairs every 2 us for 2 ms.  ``start()`` before enqueueing the work,
    ``mhz()`` after synchronising: the median over 20 us windows.  Under
    MFMA-heavy load the part lowers its clock below the 2.4 GHz that the
    published peak assumes."""

    def __init__(self, torch, samples=1000, gap_ticks=200):
        from neso_amd import _lib
        self.lib, self.n, self.gap = _lib.load(), samples, gap_ticks
        self.buf = torch.empty(2 * samples, dtype=torch.int64, device="cuda")
        self.side = torch.cuda.Stream()
        self.status = None

    def start(self):
        import ctypes
        self.status = self.lib.neso_clock_sample(ctypes.c_void_p(self.buf.data_ptr()), self.n,
                                                 self.gap, ctypes.c_void_p(self.side.cuda_stream))

    def mhz(self):
        if self.status != 0:
            return None
        s = self.buf.cpu().view(self.n, 2).tolist()
        w = 10
        return round(statistics.median((s[i + w][0] - s[i][0]) * 100.0 / (s[i + w][1] - s[i][1])
                                       for i in range(0, self.n - w, w)))


def board_power(graph, torch, seconds=1.0):
    """Median board power (W) from the amdgpu hwmon ``power1_input`` over the
    second half of ``seconds`` of back-to-back replays of ``graph``, with the
    power cap and the shader clock in that half; None where the sysfs
    entries are absent."""
    import glob
    import threading
    files = sorted(glob.glob("/sys/class/drm/card*/device/hwmon/hwmon*/power1_input"))
    if len(files) != 1:
        return None
    cap_file = files[0].replace("power1_input", "power1_cap")
    readings, stop = [], threading.Event()

    def poll():
        t0 = time.perf_counter()
        while not stop.is_set():
            try:
                readings.append((time.perf_counter() - t0, int(open(files[0]).read()) / 1e6))
            except (OSError, ValueError):
                pass
            time.sleep(0.01)

    clock = ClockSampler(torch)
    th = threading.Thread(target=poll)
    th.start()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        if clock.status is None and time.perf_counter() - t0 >= seconds / 2:
            clock.start()
        for _ in range(8):
            graph.replay()
        torch.cuda.synchronize()
    stop.set()
    th.join()
    late = [w for t, w in readings if t >= seconds / 2]
    if not late:
        return None
    try:
        cap = int(open(cap_file).read()) / 1e6
    except (OSError, ValueError):
        cap = None
    return {"board_power_w": round(statistics.median(late)), "power_cap_w": cap,
            "soak_clock_mhz": clock.mhz(),
            "source": "1 s of back-to-back replays: amdgpu hwmon power1_input, median over "
                      "the last half; shader clock sampled in the last half"}


def clock_note(tflops, timing):
    """The MFMA peak at the shader clock sampled during the workload, and the
    achieved rate against it (the published peak assumes 2.4 GHz)."""
    mhz = timing.get("clock_mhz")
    if not mhz:
        return None
    peak = MFMA_F16_PEAK_TFLOPS * mhz / 2400.0
    out = {"sampled_mhz": mhz, "peak_at_sampled_clock": round(peak, 1),
           "frac_at_sampled_clock": round(tflops / peak, 4)}
    if timing.get("power"):
        out.update(timing["power"])
    return out


def calibrate_copy(torch):
    """Plain 256 MiB device copy: bytes moved per launch and its time."""
    nbytes = 256 << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    ms, _ = time_case(lambda i: dst.copy_(src), 16, 3, torch)
    return {"metric": "device copy GB/s (read + write)", "bytes_read": nbytes,
            "bytes_written": nbytes, "ms_per_copy": round(ms, 6),
            "value": round(2 * nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s"}


def cpu_time(fn, reps=None):
    """Median seconds after one warm-up: of 5 runs, or of 3 when one run takes
    a second or more (the d = 128 config), as the CPU-baseline plan sets."""
    t0 = time.perf_counter()
    fn()
    if reps is None:
        reps = 5 if time.perf_counter() - t0 < 1.0 else 3
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def box_peak():
    """Dense fp16 MFMA peak of this box from rocminfo: compute units x max
    engine clock x 4096 FLOP/clk/CU (CDNA4), next to the spec-sheet peak.
    None when rocminfo is unavailable."""
    import re
    import subprocess
    try:
        out = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    for agent in out.split("Agent ")[1:]:
        if "gfx950" not in agent:
            continue
        cu = re.search(r"Compute Unit:\s+(\d+)", agent)
        mhz = re.search(r"Max Clock Freq\. \(MHz\):\s+(\d+)", agent)
        if cu and mhz:
            cus, clk = int(cu.group(1)), int(mhz.group(1))
            return {"compute_units": cus, "max_clock_mhz": clk,
                    "tflops": round(cus * clk * 1e6 * 4096 / 1e12, 1)}
    return None


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


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


# ---------------------------------------------------------------------------
# Workloads.  Each returns (launch(i), work per launch, unit kind, config,
# cpu_fn or None, extra dict); the work is FLOP ("flop") or bytes ("bytes").

def fa2_workload(neso_amd, torch, I, B, H, N, d, causal, want_cpu, f32=False):
    from oracle import attention as A  # FLOP formula and CPU baseline only
    q, k, v = (t.cuda() for t in I.fa2_inputs(B, H, N, d, seed=0))
    if f32:
        q, k, v = q.float(), k.float(), v.float()
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    scale = A.default_scale(d)
    # Synthetic inputs are far inside the fp16 range: no per-call range check.
    launch = lambda i: neso_amd.attention(q, k, v, causal=causal, out=out, check_range=False)
    cpu = None
    if want_cpu:
        qc, kc, vc = (t.cpu() for t in (q, k, v))
        cpu = lambda: A.attention(qc, kc, vc, scale, causal=causal)
    cfg = {"B": B, "H": H, "N": N, "d": d, "causal": causal}
    return launch, A.flops(B, H, N, d, causal), "flop", cfg, cpu


def relpos_workload(neso_amd, torch, I, want_cpu):
    from oracle import attention as A
    rc = I.RELPOS_CONFIG
    q, k, v, table = (t.cuda() for t in I.relpos_inputs(**rc, seed=0))
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    launch = lambda i: neso_amd.rel_pos_attention(q, k, v, table, out=out)
    cpu = None
    if want_cpu:
        qc, kc, vc, tc = (t.cpu() for t in (q, k, v, table))
        cpu = lambda: A.rel_pos_attention_table(qc, kc, vc, tc, A.default_scale(rc["d"]))
    return launch, 4.0 * rc["H"] * rc["N"] ** 2 * rc["d"], "flop", dict(rc), cpu


def relpos_precompute_workload(neso_amd, torch, I, want_cpu):
    """The dense-bias precompute at config 4's shape (H8 T1500 d64): Q_u and
    the fp16 [H][T][T] bias.  FLOP = 2 * H * T^2 * d (one d-long dot per
    output element); bytes = fp32 Q, K_rel, biases in + fp16 Q_u and bias
    out, 46.6 MB, which bound it (5.8 us at 8 TB/s)."""
    from oracle import attention as A
    rc = I.RELPOS_CONFIG
    h, t, d = rc["H"], rc["N"], rc["d"]
    g = torch.Generator().manual_seed(0)
    q, kr = torch.randn(h, t, d, generator=g), torch.randn(h, 2 * t - 1, d, generator=g)
    bu, bv = (torch.randn(h, d, generator=g) * 0.1 for _ in range(2))
    qd, krd, bud, bvd = (x.cuda() for x in (q, kr, bu, bv))
    q_u = torch.empty(h, t, d, dtype=torch.float16, device="cuda")
    rel = torch.empty(h, t, t, dtype=torch.float16, device="cuda")
    launch = lambda i: neso_amd.rel_pos_precompute(qd, krd, bud, bvd, t, d, h, d ** -0.5, q_u, rel,
                                                   check_range=False)
    cpu = None
    if want_cpu:
        qn, krn, bun, bvn = (x.numpy() for x in (q, kr, bu, bv))
        cpu = lambda: A.precompute_bias_and_qu(qn, krn, bun, bvn)
    nbytes = 4 * h * t * d + 4 * h * (2 * t - 1) * d + 8 * h * d + 2 * h * t * d + 2 * h * t * t
    cfg = {"H": h, "T": t, "d": d, "algorithmic_bytes": nbytes}
    return launch, 2.0 * h * t * t * d, "flop", cfg, cpu


def relpos_dense_workload(neso_amd, torch, I, T, want_cpu, nh=8, d=128):
    """The reference's own rel-pos bench (tests/test_rel_pos_fa2.py:377-426,
    configs :466-472): dense fp16 bias [nh][T][T], logits (QK^T + B) * scale,
    fp16 O, d = 128, nh = 8.  FLOP = 4 nh T^2 d as for BASELINE (the
    reference's own formula adds nh T^2 for the bias, :424)."""
    from neso_amd import _lib
    from oracle import attention as A
    g = torch.Generator().manual_seed(T)
    q, k, v = (torch.randn(nh, T, d, generator=g).half() for _ in range(3))
    bias = (torch.randn(nh, T, T, generator=g) * 2.0).half()
    qd, kd, vd, bd = (x.cuda() for x in (q, k, v, bias))
    o = torch.empty(nh, T, d, dtype=torch.float16, device="cuda")
    scale = d ** -0.5
    launch = lambda i: neso_amd.rel_pos_fa2_fwd(qd, kd, vd, bd, o, T, d, scale, T * d, T * T,
                                                num_heads=nh, head_dim=d,
                                                bias_mode=_lib.NESO_BIAS_DENSE_SCALED_F16)
    cpu = (lambda: A.rel_pos_attention_dense(q, k, v, bias, scale)) if want_cpu else None
    cfg = {"H": nh, "T": T, "d": d, "bias": "dense f16 [H][T][T]", "out": "f16"}
    return launch, 4.0 * nh * T * T * d, "flop", cfg, cpu


def fa2_io_workload(neso_amd, torch, N, d, want_cpu, f32=False):
    """The reference's hand-written FA2 bench (bench/bench_flash_attention.py
    :142-152, configs :498-508): one head, Q/K/V/O all fp16 (or fp32)."""
    from oracle import attention as A
    g = torch.Generator().manual_seed(N + d)
    dt = torch.float32 if f32 else torch.float16
    q, k, v = (torch.randn(N, d, generator=g).to(dt) for _ in range(3))
    qd, kd, vd = (x.cuda() for x in (q, k, v))
    o = torch.empty(N, d, dtype=dt, device="cuda")
    scale = d ** -0.5
    launch = lambda i: neso_amd.flash_attention_io_fwd(qd, kd, vd, o, N, d, scale,
                                                       check_range=False)
    cpu = (lambda: A.attention(q, k, v, scale)) if want_cpu else None
    cfg = {"B": 1, "H": 1, "N": N, "d": d, "io": "f32" if f32 else "f16"}
    return launch, 4.0 * N * N * d, "flop", cfg, cpu


def window_workload(neso_amd, torch, N, H, d, wl, wr, want_cpu):
    """The reference's sliding-window kernel (debug/fa2_correctness_legacy.py
    :92-102) at a larger shape: [seq][heads][d] fp16, fp16 O.  FLOP counts
    the visible (query, key) pairs, 4 d per pair."""
    from oracle import attention as A
    g = torch.Generator().manual_seed(N + wl)
    q, k, v = (torch.randn(N, H, d, generator=g).half() for _ in range(3))
    qd, kd, vd = (x.cuda() for x in (q, k, v))
    o = torch.empty(N, H, d, dtype=torch.float16, device="cuda")
    launch = lambda i: neso_amd.window_attention(qd, kd, vd, wl, wr, out=o)
    cpu = None
    if want_cpu:
        qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
        cpu = lambda: A.attention(qh, kh, vh, d ** -0.5, window=(wl, wr))
    i = torch.arange(N)
    pairs = int(((torch.minimum(i + wr, torch.tensor(N - 1)) - torch.clamp(i - wl, min=0)) + 1)
                .clamp(min=0).sum())
    cfg = {"N": N, "H": H, "d": d, "window_left": wl, "window_right": wr, "visible_pairs": pairs}
    return launch, 4.0 * H * pairs * d, "flop", cfg, cpu


def w4a16_workload(neso_amd, torch, I, M, want_cpu, rotate=ROTATE):
    from oracle import qmatmul as Q
    import numpy as np
    K, N = 4096, 11008
    x, codes, scales = I.qmatmul_inputs(M, K, N, seed=0)
    words = torch.from_numpy(Q.pack_int4(codes.numpy()))
    xs = x.cuda()
    ws = [words.cuda() for _ in range(rotate)]
    ss = [scales.cuda() for _ in range(rotate)]
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    launch = lambda i: neso_amd.w4a16_matmul(xs, ws[i % rotate], ss[i % rotate], y, M, N, K, K, N)
    cpu = None
    if want_cpu:
        xc = x.float()
        wdq = torch.from_numpy(Q.dequant_int4(words.numpy(), scales.numpy(), dtype=np.float32))

        def cpu():  # dequantise (numpy oracle) + fp32 matmul
            w = torch.from_numpy(Q.dequant_int4(words.numpy(), scales.numpy(), dtype=np.float32))
            return xc @ w.T
        cpu.matmul_only = lambda: xc @ wdq.T  # weights dequantised beforehand
    cfg = {"M": M, "K": K, "N": N, "group": 32, "zero": 8, "rotated_weight_copies": rotate}
    return launch, Q.algorithmic_bytes(M, N, K), "bytes", cfg, cpu


def w4a16_floor(neso_amd, torch, steps, warmup, rotate=ROTATE):
    """The streaming floor of the M=1 GEMV, timed like it: at the GEMV's own
    grid (from its launch plan), an empty kernel (dispatch and the kernel
    boundary alone) and a read-only stream of the same algorithmic bytes
    (16-byte non-temporal loads, four in flight per lane) over ``rotate``
    distinct buffers (more than the Infinity Cache holds), one per launch
    in turn.  Both through ``neso_stream_probe``."""
    from neso_amd import _lib
    K, N = 4096, 11008
    nbytes = K * N // 2 + (K // 32) * N * 2 + K * 2 + N * 2  # the GEMV's algorithmic bytes, M = 1
    nbytes -= nbytes % 16
    x = torch.zeros(1, K, dtype=torch.float16, device="cuda")
    w = torch.zeros(N, K // 8, dtype=torch.int32, device="cuda")
    sc = torch.zeros(N, K // 32, dtype=torch.float16, device="cuda")
    y = torch.empty(1, N, dtype=torch.float16, device="cuda")
    plan = neso_amd.launch_plan("w4a16_matmul", x, w, sc, y, 1, N, K, K, N)
    grid = int(plan[0]["grid"][0])
    del w, sc
    bufs = [torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device="cuda")
            for _ in range(rotate)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    lib = _lib.load()

    def probe(mode):
        def launch(i):
            st = torch.cuda.current_stream().cuda_stream
            _lib.check(lib.neso_stream_probe(bufs[i % rotate].data_ptr(), nbytes, grid, mode,
                                             0xFFFFFFFF, sink.data_ptr(), st))
        return launch
    ms_read, t_read = time_case(probe(1), steps, warmup, torch)
    ms_empty, t_empty = time_case(probe(0), steps, warmup, torch)
    del bufs
    return {"kernel": f"stream_read_kernel / stream_empty_kernel, grid {grid} x 256 "
                      f"(the GEMV's: {plan[0]['device_kernel']})",
            "bytes": nbytes, "rotated_buffers": rotate, "grid": grid,
            "stream_us": round(ms_read * 1e3, 3),
            "stream_gbs": round(nbytes / (ms_read * 1e-3) / 1e9, 1),
            "stream_median_us": round(t_read["median_ms"] * 1e3, 3),
            "empty_us": round(ms_empty * 1e3, 3),
            "empty_median_us": round(t_empty["median_ms"] * 1e3, 3)}


def w8a16_workload(neso_amd, torch, scaled, want_cpu, size=4096):
    m = n = k = size
    g = torch.Generator().manual_seed(0)
    a = torch.randn(m, k, generator=g).half()
    b = torch.randint(-128, 128, (k, n), generator=g, dtype=torch.int8)
    sc = (torch.rand(n, generator=g) * 0.1 + 0.001).half()
    ad, bd, sd = a.cuda(), b.cuda(), sc.cuda()
    c = torch.empty(m, n, dtype=torch.float32, device="cuda")
    if scaled:
        launch = lambda i: neso_amd.w8a16_scaled_matmul(ad, bd, c, sd, k, k, n, n, M=m, N=n)
    else:
        launch = lambda i: neso_amd.w8a16_matmul(ad, bd, c, k, k, n, n, M=m, N=n)
    cpu = None
    if want_cpu:
        af, bf, sf = a.float(), b.float(), sc.float()
        cpu = (lambda: (af @ bf) * sf) if scaled else (lambda: af @ bf)
    return launch, 2.0 * m * n * k, "flop", {"M": m, "N": n, "K": k}, cpu


def launched_kernels(launch):
    """The device kernels (with template arguments) and grids that one call of
    ``launch`` issues, from the library's launch plan (recorded, not run)."""
    import json as _json
    from neso_amd import _lib
    lib = _lib.load()
    _lib.check(lib.neso_plan_begin(0))
    try:
        launch(0)
    finally:
        plan = _json.loads(lib.neso_plan_end().decode())["launches"]
    return [f"{p['device_kernel']}<{','.join(str(x) for x in p['template_args'])}> grid "
            f"{p['grid']} x {p['threadgroup_size']}" for p in plan]


def run_case(workload, steps, warmup, torch, want_cpu, power=False):
    """Time one workload; returns a result row."""
    launch, work, kind, cfg, cpu = workload
    kernels = launched_kernels(launch)
    ms, timing = time_case(launch, steps, warmup, torch, power)
    row = dict(cfg)
    row["device_kernels"] = kernels
    row["us"] = round(ms * 1e3, 3)
    row["timing"] = timing
    if kind == "flop":
        tf = work / (ms * 1e-3) / 1e12
        row["tflops"] = round(tf, 3)
        row["mfma_frac"] = round(tf / MFMA_F16_PEAK_TFLOPS, 4)
        row["tflops_median"] = round(work / (timing["median_ms"] * 1e-3) / 1e12, 3)
    else:
        gbs = work / (ms * 1e-3) / 1e9
        row["gbs"] = round(gbs, 2)
        row["hbm_frac"] = round(gbs / HBM_PEAK_GBS, 4)
        row["gbs_median"] = round(work / (timing["median_ms"] * 1e-3) / 1e9, 2)
        row["algorithmic_bytes"] = work
    if want_cpu and cpu is not None:
        sec = cpu_time(cpu)
        row["cpu_seconds"] = round(sec, 5)
        if kind == "flop":
            row["cpu_tflops"] = round(work / sec / 1e12, 5)
        else:
            row["cpu_gbs"] = round(work / sec / 1e9, 4)
            if hasattr(cpu, "matmul_only"):
                row["cpu_matmul_only_gbs"] = round(work / cpu_time(cpu.matmul_only) / 1e9, 4)
        row["gpu_over_cpu"] = round(sec / (ms * 1e-3), 1)
    return row


def cases(neso_amd, torch, I, want_cpu):
    """name -> thunk building the workload (built lazily to bound memory)."""
    c = {
        "fa2_headline": lambda: fa2_workload(neso_amd, torch, I, 1, 16, 2048, 64, False, want_cpu),
        "fa2_config1": lambda: fa2_workload(neso_amd, torch, I, 1, 8, 128, 64, False, want_cpu),
        "fa2_d128": lambda: fa2_workload(neso_amd, torch, I, 2, 32, 4096, 128, True, want_cpu),
        "fa2_f32_qkv": lambda: fa2_workload(neso_amd, torch, I, 1, 16, 2048, 64, False, want_cpu,
                                            f32=True),
        "fa2_f32_qkv_d128": lambda: fa2_workload(neso_amd, torch, I, 1, 16, 2048, 128, False,
                                                 want_cpu, f32=True),
        "relpos": lambda: relpos_workload(neso_amd, torch, I, want_cpu),
        "relpos_precompute": lambda: relpos_precompute_workload(neso_amd, torch, I, want_cpu),
        "w8a16": lambda: w8a16_workload(neso_amd, torch, False, want_cpu),
        "w8a16_scaled": lambda: w8a16_workload(neso_amd, torch, True, want_cpu),
    }
    for cfg in I.FA2_SWEEP:
        name = f"fa2_n{cfg['N']}{'_causal' if cfg['causal'] else ''}"
        c[name] = (lambda cfg=cfg: fa2_workload(neso_amd, torch, I, cfg["B"], cfg["H"], cfg["N"],
                                                cfg["d"], cfg["causal"], want_cpu))
    for m in (1, 16, 256):
        c[f"w4a16_m{m}"] = lambda m=m: w4a16_workload(neso_amd, torch, I, m, want_cpu)
    # The reference's own benchmark configs (kernels it times itself).
    for t in REF_RELPOS_T:
        c[f"ref_relpos_dense_T{t}"] = lambda t=t: relpos_dense_workload(neso_amd, torch, I, t,
                                                                      want_cpu)
    for n, d in REF_FA2_IO:
        c[f"ref_fa2_io_f16_N{n}_d{d}"] = lambda n=n, d=d: fa2_io_workload(neso_amd, torch, n, d,
                                                                         want_cpu)
    for n, d in ((4096, 64), (4096, 128)):
        c[f"ref_fa2_io_f32_N{n}_d{d}"] = lambda n=n, d=d: fa2_io_workload(neso_amd, torch, n, d,
                                                                         want_cpu, f32=True)
    c["fa2_d32"] = lambda: fa2_workload(neso_amd, torch, I, 1, 16, 2048, 32, False, want_cpu)
    c["fa2_window"] = lambda: window_workload(neso_amd, torch, 4096, 16, 64, 256, 0, want_cpu)
    for size in (1024, 2048):
        c[f"w8a16_{size}"] = lambda size=size: w8a16_workload(neso_amd, torch, False, want_cpu,
                                                             size)
        c[f"w8a16_scaled_{size}"] = lambda size=size: w8a16_workload(neso_amd, torch, True,
                                                                    want_cpu, size)
    return c


REF_RELPOS_T = (128, 256, 384, 448, 512)  # tests/test_rel_pos_fa2.py:466-472
REF_FA2_IO = ((256, 64), (512, 64), (1024, 64), (2048, 64), (4096, 64), (512, 128), (1024, 128),
              (2048, 128), (4096, 128))  # bench/bench_flash_attention.py:498-508


SWEEP_ORDER = ["fa2_config1"] + [f"fa2_n{n}{s}" for n in (128, 256, 512, 1024, 2048)
                                 for s in ("", "_causal")] + [
    "fa2_d128", "relpos", "relpos_precompute", "fa2_f32_qkv", "fa2_f32_qkv_d128", "w8a16",
    "w8a16_scaled", "w4a16_m16", "w4a16_m256", "fa2_d32", "fa2_window"] + [
    f"ref_relpos_dense_T{t}" for t in REF_RELPOS_T] + [
    f"ref_fa2_io_f16_N{n}_d{d}" for n, d in REF_FA2_IO] + [
    "ref_fa2_io_f32_N4096_d64", "ref_fa2_io_f32_N4096_d128", "w8a16_1024", "w8a16_scaled_1024",
    "w8a16_2048", "w8a16_scaled_2048"]
KERNEL_OF = {  # device kernel each sweep row's time is dominated by (for readers)
    "fa2_f32_qkv": "fa2_fwd_kernel (F32IN: 3 fp16 MFMAs per product)",
    "fa2_f32_qkv_d128": "fa2_fwd_kernel (F32IN, 32-key blocks)",
    "relpos": "fa2_fast_kernel (BIAS: f32 table band in the score accumulator; QW = 2, KSPLIT = 4)",
    "relpos_precompute": "relpos_precompute_kernel (fp16 hi/lo MFMA; HBM-bound, hbm_frac)",
    "w8a16": "w8a16_gemm_kernel", "w8a16_scaled": "w8a16_gemm_kernel",
    "w4a16_m16": "w4a16_skinny_lds_kernel", "w4a16_m256": "w4a16_tile_gemm_kernel",
    "fa2_window": "neso_flash_attention_window_fwd (fast kernel, sliding window)",
    "w8a16_1024": "w8a16_gemm_kernel", "w8a16_scaled_1024": "w8a16_gemm_kernel",
    "w8a16_2048": "w8a16_gemm_kernel", "w8a16_scaled_2048": "w8a16_gemm_kernel",
    **{f"ref_relpos_dense_T{t}": "neso_rel_pos_fa2_fwd, NESO_BIAS_DENSE_SCALED_F16, fp16 O"
       for t in REF_RELPOS_T},
    **{f"ref_fa2_io_f16_N{n}_d{d}": "neso_flash_attention_io_fwd (fp16 io)" for n, d in REF_FA2_IO},
    "ref_fa2_io_f32_N4096_d64": "neso_flash_attention_io_fwd (fp32 io: F32IN kernel)",
    "ref_fa2_io_f32_N4096_d128": "neso_flash_attention_io_fwd (fp32 io: F32IN kernel)",
}


def main():
    global CLOCK_RAMP_S
    args = parse()
    CLOCK_RAMP_S = max(0.0, args.ramp)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU (one process, one "
                                   "device); --gpus must be 1", "n_gpus": args.gpus}))
        return 2
    # rocminfo runs as a child process before this process touches the GPU.
    peak_box = None if (args.case or args.calibrate_copy) else box_peak()
    import torch

    import neso_amd
    from oracle import inputs as I

    torch.manual_seed(0)
    if args.calibrate_copy:
        print(json.dumps(calibrate_copy(torch)), flush=True)
        return 0
    dev = torch.cuda.get_device_properties(0)
    log(f"device {dev.name} {dev.gcnArchName} CUs={dev.multi_processor_count}")
    want_cpu = not args.no_cpu
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    C = cases(neso_amd, torch, I, want_cpu and args.case is None)

    if args.case is not None:
        if args.case not in C:
            print(json.dumps({"error": f"unknown case {args.case!r}", "cases": sorted(C)}))
            return 2
        row = run_case(C[args.case](), args.steps, args.warmup, torch, False)
        print(json.dumps({"case": args.case, **row}), flush=True)
        return 0

    # ---- headline: FA2 forward, B1 H16 N2048 d64 non-causal ----
    head = run_case(C["fa2_headline"](), args.steps, args.warmup, torch, want_cpu, power=True)
    ms = head["us"] * 1e-3
    tflops = head["tflops"]
    log(f"fa2 headline {head['us']:.2f} us/launch {tflops:.1f} TFLOP/s "
        f"(median {head['timing']['median_ms'] * 1e3:.2f} us)")
    flop = 4.0 * 1 * 16 * 2048 ** 2 * 64
    result = {
        "metric": METRIC,
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "timing": head["timing"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "flash_attention_fwd B=1 H=16 N=2048 d=64 non-causal, "
                               "fp16 Q/K/V ~ N(0,1), fp32 accumulation and output",
                   "B": 1, "H": 16, "N": 2048, "d": 64, "causal": False},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic("fa2_headline"),
                     "kernel": "fa2_fast_kernel<64,false,false,2,false,false,4,false>",
                     "algorithmic_flop_per_launch": flop,
                     "peak_box": peak_box,
                     "clock": clock_note(tflops, head["timing"])},
    }
    if want_cpu:
        result["cpu_baseline"] = {
            "value": head["cpu_tflops"], "unit": "TFLOP/s", "cores": threads,
            "cpu_model": cpu_model(), "kind": "port",
            "sample": "oracle.attention (torch fp32 CPU, chunked rows) on the full headline "
                      "workload B1 H16 N2048 d64, median of 5 after 1 warm-up",
            "seconds_per_step": head["cpu_seconds"]}
        log(f"cpu baseline {head['cpu_seconds']:.3f} s/step")

    # ---- int4 qmatmul, M=1 (HBM-bound), rotated weights ----
    qm = run_case(C["w4a16_m1"](), args.steps, args.warmup, torch, want_cpu)
    gbs = qm["gbs"]
    result["qmatmul"] = {
        "metric": "int4 qmatmul HBM GB/s", "value": gbs, "unit": "GB/s",
        "ms_per_step": round(qm["us"] * 1e-3, 6), "timing": qm["timing"],
        "config": {"workload": f"w4a16_matmul M=1 K=4096 N=11008 group=32 zero=8, fp16 X, "
                               f"fp16 out, {ROTATE} rotated weight copies",
                   "M": 1, "K": 4096, "N": 11008},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic("w4a16_M1"),
                     "kernel": "w4a16_gemv_kernel<1,2,4,true>",
                     "algorithmic_bytes_per_launch": qm["algorithmic_bytes"]}}
    if want_cpu:
        result["qmatmul"]["cpu_baseline"] = {
            "value": qm["cpu_gbs"], "unit": "GB/s", "cores": threads, "cpu_model": cpu_model(),
            "kind": "port",
            "sample": "oracle dequant_int4 (numpy) + torch fp32 matmul on the full M=1 "
                      "workload, median of 5 after 1 warm-up; matmul_only_gbs with the "
                      "weights dequantised beforehand",
            "seconds_per_step": qm["cpu_seconds"],
            "matmul_only_gbs": qm.get("cpu_matmul_only_gbs")}
    floor = w4a16_floor(neso_amd, torch, args.steps, args.warmup)
    floor["gemv_minus_stream_us"] = round(qm["us"] - floor["stream_us"], 3)
    result["qmatmul"]["roofline"]["floor"] = floor
    log(f"qmm M=1 {gbs:.1f} GB/s; floor: stream {floor['stream_us']:.2f} us "
        f"({floor['stream_gbs']:.0f} GB/s), empty {floor['empty_us']:.2f} us")

    if not args.no_sweep:
        rows = []
        sweep_steps = max(32, min(args.steps, 64))
        for name in SWEEP_ORDER:
            row = run_case(C[name](), sweep_steps, 5, torch, want_cpu)
            row = {"case": name, **({"kernel": KERNEL_OF[name]} if name in KERNEL_OF else {}),
                   **row}
            if name.startswith("fa2_f32_qkv"):
                # Three fp16 MFMAs per product: the issued MFMA work is 3x
                # the useful FLOPs counted in tflops / mfma_frac.
                row["mfma_frac_issued"] = round(3 * row["mfma_frac"], 4)
            if name == "relpos_precompute":
                # HBM-bound: fp32 inputs in, fp16 Q_u and the T x T bias out.
                row["gbs"] = round(row["algorithmic_bytes"] / (row["us"] * 1e-6) / 1e9, 1)
                row["hbm_frac"] = round(row["gbs"] / HBM_PEAK_GBS, 4)
            if name.startswith("w4a16"):
                row["mfma_frac"] = round(2.0 * row["M"] * row["N"] * row["K"]
                                         / (row["us"] * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
            rows.append(row)
            torch.cuda.empty_cache()
            log(f"{name}: {row['us']:.2f} us")
        result["sweep"] = rows
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
