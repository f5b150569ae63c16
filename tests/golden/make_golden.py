#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ (inputs + expected outputs).

The reference holds no fixture files: its tests generate inputs from fixed
seeds and check against small pure-Python oracles.  This script reproduces
those generators exactly and evaluates the reference tests' own checking
procedures with plain Python loops in float64 (small sizes only), so the
fixtures are independent of ``oracle/`` (which is vectorised torch/numpy):

* fa2_kat.npz — macos/harness.rs:171-271: Q = K = 0, V[i] =
  ((i % 17) - 8) * 0.125, N = 64, d = 64; expected every row = column mean
  of fp16(V).
* fa2_ref_N{N}_d{d}.npz — tests/test_flash_attention.py:268-275 inputs
  (random.seed(42), gauss(0, 0.5)) and the expected rows 0 and N/2 computed
  as at :296-339.
* relpos_ref_T{T}_d{d}_nh{nh}.npz — tests/test_rel_pos_fa2.py:317-327
  inputs (np.random.seed(42)) and the direct Transformer-XL output computed
  as at :256-283 (loops over i, j).
* qmm_w8a16_*.npz / qmm_scaled_*.npz / qmm_w4i8_*.npz —
  tests/test_quantized_matmul.py:335-337, :379-381, :423-426 inputs and the
  f64 triple-loop outputs of :288-311.
* fa2_window_S{seq}_H{h}_d{d}_w{l}_{r}.npz — debug/fa2_correctness_legacy.py:68-79
  inputs (np.random.seed(42), randn * 0.5 as fp16) and the sliding-window
  reference of :53-64 (-1e9 outside [i - left, i + right]) in float64 loops.
* qmm_int4_kat.npz — hand-made packed int4 words with known nibble codes,
  group scales and one-hot activations, expected values from the format
  definition (code of column k = nibble k % 8 of word k // 8).

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import random
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def f16(x: float) -> float:
    return float(np.float16(x))


def fa2_kat(n: int = 64, d: int = 64) -> None:
    count = n * d
    v = [((i % 17) - 8.0) * 0.125 for i in range(count)]
    means = []
    for c in range(d):
        s = 0.0
        for r in range(n):
            s += f16(v[r * d + c])
        means.append(s / n)
    expected = [means[c] for _ in range(n) for c in range(d)]
    np.savez_compressed(HERE / "fa2_kat.npz", N=n, d=d,
                        q=np.zeros(count, np.float32), k=np.zeros(count, np.float32),
                        v=np.array(v, np.float32), expected=np.array(expected, np.float64),
                        tol=2e-3)


def fa2_ref_rows(n: int, d: int) -> None:
    rnd = random.Random(42)
    q = [rnd.gauss(0, 0.5) for _ in range(n * d)]
    k = [rnd.gauss(0, 0.5) for _ in range(n * d)]
    v = [rnd.gauss(0, 0.5) for _ in range(n * d)]
    scale = 1.0 / math.sqrt(d)
    rows = [0, n // 2]
    expected = []
    for row in rows:
        q_row = q[row * d:(row + 1) * d]
        scores = []
        for j in range(n):
            k_row = k[j * d:(j + 1) * d]
            scores.append(sum(q_row[kk] * k_row[kk] for kk in range(d)) * scale)
        mx = max(scores)
        ex = [math.exp(s - mx) for s in scores]
        tot = sum(ex)
        w = [e / tot for e in ex]
        o = [0.0] * d
        for j in range(n):
            v_row = v[j * d:(j + 1) * d]
            for kk in range(d):
                o[kk] += w[j] * v_row[kk]
        expected.append(o)
    np.savez_compressed(HERE / f"fa2_ref_N{n}_d{d}.npz", N=n, d=d, scale=scale,
                        q=np.array(q, np.float64), k=np.array(k, np.float64),
                        v=np.array(v, np.float64), rows=np.array(rows),
                        expected=np.array(expected, np.float64))


def fa2_window_ref(seq: int, heads: int, d: int, wl: int, wr: int) -> None:
    """debug/fa2_correctness_legacy.py:68-79 inputs (np.random.seed(42), randn * 0.5 as
    fp16, rows [seq][heads * d]) and the :53-64 reference evaluated with loops in float64."""
    rs = np.random.RandomState(42)
    kv = heads * d
    Q = (rs.randn(seq, kv) * 0.5).astype(np.float16)
    K = (rs.randn(seq, kv) * 0.5).astype(np.float16)
    V = (rs.randn(seq, kv) * 0.5).astype(np.float16)
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((seq, kv))
    Qd, Kd, Vd = (a.astype(np.float64) for a in (Q, K, V))
    for h in range(heads):
        c0 = h * d
        for i in range(seq):
            scores = []
            for j in range(seq):
                s = sum(Qd[i, c0 + c] * Kd[j, c0 + c] for c in range(d)) * scale
                scores.append(-1e9 if (j < i - wl or j > i + wr) else s)
            mx = max(scores)
            ex = [math.exp(x - mx) for x in scores]
            tot = sum(ex)
            for j in range(seq):
                w = ex[j] / tot
                if w:
                    for c in range(d):
                        out[i, c0 + c] += w * Vd[j, c0 + c]
    np.savez_compressed(HERE / f"fa2_window_S{seq}_H{heads}_d{d}_w{wl}_{wr}.npz", seq=seq,
                        heads=heads, d=d, window_left=wl, window_right=wr, scale=scale,
                        Q=Q, K=K, V=V, expected=out)


def relpos_ref(t: int, d: int, nh: int) -> None:
    rs = np.random.RandomState(42)
    Q = rs.randn(nh, t, d).astype(np.float32) * 0.5
    K = rs.randn(nh, t, d).astype(np.float32) * 0.5
    V = rs.randn(nh, t, d).astype(np.float32) * 0.5
    K_rel = rs.randn(nh, 2 * t - 1, d).astype(np.float32) * 0.5
    bias_u = rs.randn(nh, d).astype(np.float32) * 0.1
    bias_v = rs.randn(nh, d).astype(np.float32) * 0.1
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((nh, t, d))
    Qd, Kd, Vd, Rd = (a.astype(np.float64) for a in (Q, K, V, K_rel))
    for h in range(nh):
        for i in range(t):
            q_u = [Qd[h, i, c] + float(bias_u[h, c]) for c in range(d)]
            q_v = [Qd[h, i, c] + float(bias_v[h, c]) for c in range(d)]
            scores = []
            for j in range(t):
                content = sum(q_u[c] * Kd[h, j, c] for c in range(d))
                idx = t - 1 - i + j
                rel = sum(q_v[c] * Rd[h, idx, c] for c in range(d))
                scores.append((content + rel) * scale)
            mx = max(scores)
            ex = [math.exp(s - mx) for s in scores]
            tot = sum(ex)
            for j in range(t):
                wj = ex[j] / tot
                for c in range(d):
                    out[h, i, c] += wj * Vd[h, j, c]
    np.savez_compressed(HERE / f"relpos_ref_T{t}_d{d}_nh{nh}.npz", T=t, d=d, nh=nh, scale=scale,
                        Q=Q, K=K, V=V, K_rel=K_rel, bias_u=bias_u, bias_v=bias_v, expected=out)


def qmm_ref(kind: str, m: int, n: int, k: int) -> None:
    seed = {"w8a16": 42, "w4i8": 43, "scaled": 44}[kind]
    rnd = random.Random(seed)
    a = [rnd.gauss(0, 0.5) for _ in range(m * k)]
    lo, hi = (-8, 7) if kind == "w4i8" else (-128, 127)
    b = [rnd.randint(lo, hi) for _ in range(k * n)]
    scale = [rnd.uniform(0.001, 0.1) for _ in range(n)] if kind == "scaled" else None
    c = [0.0] * (m * n)
    for mm in range(m):
        for nn in range(n):
            acc = 0.0
            for kk in range(k):
                acc += float(a[mm * k + kk]) * float(b[kk * n + nn])
            c[mm * n + nn] = acc * (float(scale[nn]) if scale else 1.0)
    extra = {"scale": np.array(scale, np.float64)} if scale else {}
    np.savez_compressed(HERE / f"qmm_{kind}_{m}x{n}x{k}.npz", M=m, N=n, K=k,
                        a=np.array(a, np.float64), b=np.array(b, np.int8),
                        expected=np.array(c, np.float64), **extra)


def qmm_int4_kat() -> None:
    # N = 4 rows, K = 64 (two groups of 32).  Row r's words are chosen so that
    # every nibble position carries a distinct, known code.
    n_rows, k = 4, 64
    base_words = [0x76543210, 0xFEDCBA98, 0x89ABCDEF, 0x01234567]
    words = []
    codes = []
    for r in range(n_rows):
        row_w = []
        row_c = []
        for wi in range(k // 8):
            w = base_words[(r + wi) % 4] ^ (0x11111111 * ((r + 2 * wi) % 3))
            w &= 0xFFFFFFFF
            row_w.append(w)
            row_c.extend((w >> (4 * e)) & 0xF for e in range(8))
        words.append(row_w)
        codes.append(row_c)
    scales = [[0.0078125 * (1 + r + 2 * g) for g in range(k // 32)] for r in range(n_rows)]
    # One-hot activations: row m of X selects column m * 9 (spans nibbles and groups).
    picks = [0, 9, 18, 27, 36, 45, 54, 63]
    x = [[1.0 if kk == p else 0.0 for kk in range(k)] for p in picks]
    expected = [[(codes[r][p] - 8) * scales[r][p // 32] for r in range(n_rows)] for p in picks]
    w_arr = np.array(words, dtype=np.uint32).view(np.int32)
    np.savez_compressed(HERE / "qmm_int4_kat.npz", words=w_arr, codes=np.array(codes, np.uint8),
                        scales=np.array(scales, np.float64), x=np.array(x, np.float64),
                        picks=np.array(picks), expected=np.array(expected, np.float64),
                        group=32, zero=8)


def main() -> int:
    fa2_kat()
    for n, d in ((64, 32), (128, 64), (256, 64), (128, 128), (256, 128), (512, 128)):
        fa2_ref_rows(n, d)
    relpos_ref(32, 64, 2)
    relpos_ref(64, 64, 4)
    fa2_window_ref(64, 3, 64, 16, 0)
    fa2_window_ref(48, 2, 32, 5, 7)
    qmm_ref("w8a16", 32, 32, 32)
    qmm_ref("w8a16", 64, 64, 128)
    qmm_ref("w4i8", 64, 64, 64)
    qmm_ref("scaled", 64, 64, 64)
    qmm_int4_kat()
    return 0


if __name__ == "__main__":
    sys.exit(main())
