"""Relative-position-bias FA2 parity on the GPU.

BASELINE semantics (table f32 [H, 2N-1], logits QK^T * scale + B[i-j+N-1],
fp32 output, max abs error <= 2e-3) at BASELINE config 4 and ragged sizes,
and the reference kernel's semantics (dense f16 [nh, T, T] bias,
(QK^T + B) * scale, fp16 output) at the reference test configs
(tests/test_rel_pos_fa2.py:434-441) with the reference's own inputs.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import neso_amd
from oracle import attention as A
from oracle import inputs as I

pytestmark = pytest.mark.gpu
TOL = 2e-3
DEV = "cuda:0"


def gpu_table(q, k, v, table, out_dtype=torch.float32):
    out = neso_amd.rel_pos_attention(q.to(DEV), k.to(DEV), v.to(DEV), table.to(DEV),
                                     out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu()


def test_baseline_config4(gpu):
    cfg = I.RELPOS_CONFIG
    q, k, v, table = I.relpos_inputs(**cfg, seed=0)
    out = gpu_table(q, k, v, table)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(cfg["d"]))
    err = (out - ref).abs().max().item()
    assert err <= TOL, err


@pytest.mark.parametrize("h,n,d", [(2, 1, 64), (3, 37, 64), (2, 129, 128), (4, 300, 32),
                                   (1, 1023, 64)])
def test_ragged(gpu, h, n, d):
    q, k, v, table = I.relpos_inputs(h, n, d, seed=n)
    out = gpu_table(q, k, v, table)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(d))
    assert (out - ref).abs().max().item() <= TOL


def test_constant_table_equals_plain_fa2(gpu):
    h, n, d = 8, 700, 64
    q, k, v, _ = I.relpos_inputs(h, n, d, seed=1)
    const = torch.full((h, 2 * n - 1), -1.25)
    rel = gpu_table(q, k, v, const)
    plain = neso_amd.attention(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    # Equal up to the fp16 rounding of P, which sees shifted logits.
    assert (rel - plain).abs().max().item() <= 2e-4


def test_spike_table_is_identity(gpu):
    h, n, d = 2, 257, 64
    q, k, v, _ = I.relpos_inputs(h, n, d, seed=2)
    spike = torch.zeros(h, 2 * n - 1)
    spike[:, n - 1] = 60.0
    out = gpu_table(q, k, v, spike)
    assert (out - v.float()).abs().max().item() <= TOL


def test_f16_output(gpu):
    h, n, d = 8, 1500, 64
    q, k, v, table = I.relpos_inputs(h, n, d, seed=4)
    out = gpu_table(q, k, v, table, out_dtype=torch.float16)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / 8).half().float()
    assert (out - ref).abs().max().item() <= TOL + 2e-3  # plus one fp16 ulp at |O| < 4


@pytest.mark.parametrize("t,d,nh", [(32, 64, 2), (64, 64, 4), (64, 128, 4), (128, 128, 8),
                                    (256, 128, 8), (448, 128, 8)])
def test_reference_mode(gpu, golden_dir, t, d, nh):
    """Reference kernel semantics on the reference test's inputs (:314-374)."""
    Q, K, V, K_rel, bu, bv = I.reference_relpos_arrays(t, d, nh)
    q_u, rel_bias = A.precompute_bias_and_qu(Q, K_rel, bu, bv)
    scale = 1 / math.sqrt(d)
    qd = torch.from_numpy(q_u).half().to(DEV)
    kd = torch.from_numpy(K).half().to(DEV)
    vd = torch.from_numpy(V).half().to(DEV)
    bd = torch.from_numpy(rel_bias).half().to(DEV)
    o = torch.empty(nh, t, d, dtype=torch.float16, device=DEV)
    neso_amd.rel_pos_fa2_fwd(qd, kd, vd, bd, o, t, d, scale, t * d, t * t, num_heads=nh,
                             bias_mode=neso_amd.NESO_BIAS_DENSE_SCALED_F16)
    torch.cuda.synchronize()
    out = o.float().cpu()
    # Against the oracle on the identical fp16 inputs.
    ref = A.rel_pos_attention_dense(qd.cpu(), kd.cpu(), vd.cpu(), bd.cpu(), scale)
    assert (out - ref).abs().max().item() <= TOL + 2e-3
    # Against the reference's own check (tolerance 0.1, :373), where a fixture exists.
    path = golden_dir / f"relpos_ref_T{t}_d{d}_nh{nh}.npz"
    direct = (np.load(path)["expected"] if path.exists()
              else A.reference_rel_pos_attention(Q, K, V, K_rel, bu, bv, scale))
    assert np.abs(out.numpy() - direct).max() < 0.1
