"""Seeded input generators (test infrastructure only).

Two families:

* BASELINE configs (repo BASELINE.json ``configs``): torch CPU generator with
  a fixed seed; Q/K/V ~ N(0, 1) fp16, rel-pos table ~ N(0, 0.5^2) f32,
  X ~ N(0, 1) fp16, int4 codes uniform in [0, 15], scales ~ U(0.005, 0.02).
* The reference tests' own generators, reproduced exactly:
  ``random.seed(42)`` + ``gauss(0, 0.5)`` for FA2
  (tests/test_flash_attention.py:268-275), ``np.random.seed(42)`` + randn *
  0.5 for rel-pos (tests/test_rel_pos_fa2.py:317-327), and
  ``random.seed(42/43/44)`` for the quantised matmuls
  (tests/test_quantized_matmul.py:335-337, :379-381, :423-426).
"""
from __future__ import annotations

import random

import numpy as np
import torch

# BASELINE.json configs, by name.
FA2_CONFIG1 = dict(B=1, H=8, N=128, d=64, causal=False)
FA2_SWEEP = [dict(B=1, H=16, N=n, d=64, causal=c) for n in (128, 256, 512, 1024, 2048)
             for c in (False, True)]
FA2_HEADLINE = dict(B=1, H=16, N=2048, d=64, causal=False)
FA2_D128 = dict(B=2, H=32, N=4096, d=128, causal=True)
RELPOS_CONFIG = dict(H=8, N=1500, d=64)
QMM_CONFIGS = [dict(M=m, K=4096, N=11008, group=32, zero=8) for m in (1, 16, 256)]


def fa2_inputs(B: int, H: int, N: int, d: int, seed: int = 0, **_):
    """Q, K, V fp16 [B, H, N, d] ~ N(0, 1) on the CPU."""
    g = torch.Generator().manual_seed(seed)
    shape = (B, H, N, d)
    q = torch.randn(shape, generator=g).to(torch.float16)
    k = torch.randn(shape, generator=g).to(torch.float16)
    v = torch.randn(shape, generator=g).to(torch.float16)
    return q, k, v


def relpos_inputs(H: int, N: int, d: int, seed: int = 0, **_):
    """Q, K, V fp16 [H, N, d] ~ N(0, 1) and table f32 [H, 2N-1] ~ N(0, 0.5^2)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((H, N, d), generator=g).to(torch.float16)
    k = torch.randn((H, N, d), generator=g).to(torch.float16)
    v = torch.randn((H, N, d), generator=g).to(torch.float16)
    table = (torch.randn((H, 2 * N - 1), generator=g) * 0.5).to(torch.float32)
    return q, k, v, table


def qmatmul_inputs(M: int, K: int, N: int, group: int = 32, seed: int = 0, **_):
    """X fp16 [M, K] ~ N(0,1); codes uint8 [N, K] ~ U{0..15}; scales fp16 [N, K/group] ~ U(.005,.02)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g).to(torch.float16)
    codes = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int64).to(torch.uint8)
    scales = (torch.rand((N, K // group), generator=g) * 0.015 + 0.005).to(torch.float16)
    return x, codes, scales


def reference_fa2_lists(N: int, d: int, seed: int = 42):
    """q, k, v python float lists exactly as tests/test_flash_attention.py:268-275."""
    rnd = random.Random(seed)
    q = [rnd.gauss(0, 0.5) for _ in range(N * d)]
    k = [rnd.gauss(0, 0.5) for _ in range(N * d)]
    v = [rnd.gauss(0, 0.5) for _ in range(N * d)]
    return q, k, v


def reference_relpos_arrays(T: int, d: int, nh: int, seed: int = 42):
    """Q, K, V, K_rel, bias_u, bias_v exactly as tests/test_rel_pos_fa2.py:317-327."""
    rs = np.random.RandomState(seed)
    Q = rs.randn(nh, T, d).astype(np.float32) * 0.5
    K = rs.randn(nh, T, d).astype(np.float32) * 0.5
    V = rs.randn(nh, T, d).astype(np.float32) * 0.5
    K_rel = rs.randn(nh, 2 * T - 1, d).astype(np.float32) * 0.5
    bias_u = rs.randn(nh, d).astype(np.float32) * 0.1
    bias_v = rs.randn(nh, d).astype(np.float32) * 0.1
    return Q, K, V, K_rel, bias_u, bias_v


def reference_quant_lists(M: int, N: int, K: int, kind: str):
    """A, B (and scale) lists exactly as the reference quantised-matmul tests.

    kind "w8a16": seed 42, B int8 in [-128, 127] (tests/test_quantized_matmul.py:335-337);
    kind "w4a16": seed 43, B in [-8, 7] (:379-381);
    kind "scaled": seed 44, B in [-128, 127], scale U(0.001, 0.1) (:423-426).
    """
    seed = {"w8a16": 42, "w4a16": 43, "scaled": 44}[kind]
    rnd = random.Random(seed)
    a = [rnd.gauss(0, 0.5) for _ in range(M * K)]
    lo, hi = (-8, 7) if kind == "w4a16" else (-128, 127)
    b = [rnd.randint(lo, hi) for _ in range(K * N)]
    scale = [rnd.uniform(0.001, 0.1) for _ in range(N)] if kind == "scaled" else None
    return a, b, scale
