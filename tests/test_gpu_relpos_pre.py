"""The GPU rel-pos bias precompute against the oracle's restatement of the
reference's host precompute.

Reference: precompute_bias_and_qu, tests/test_rel_pos_fa2.py:286-311 (Q_u =
Q + bias_u; rel_bias[h, i, j] = (Q + bias_v)_i . K_rel[T - 1 - i + j],
float64 dot stored float32), whose outputs the reference test rounds to
fp16 for the kernel (:355-358).  Bars:

* Q_u: bit-exact with fp16(Q + bias_u) (one fp32 add, one rounding);
* rel_bias: every element written, and each within one fp16 ulp of
  fp16(oracle) plus (3d + 12) * 2^-24 * sum_k |(Q + v)_k K_rel_k|.  The GPU
  splits each fp32 factor into fp16 hi + lo and sums the 3d products
  hi.hi, hi.lo, lo.hi in fp32: 3d * 2^-24 is the classic bound of that
  fp32 sum, and 12 * 2^-24 per |q_k k_k| covers the dropped lo.lo term and
  the rounding of lo (each |lo - (x - hi)| <= 2^-22 |x|).  The bound matters
  only where the d products cancel to a value far below their size, e.g.
  5e-6 out of terms of 0.25.  Fewer than 1% of the elements may differ
  from fp16(oracle) at all: a lost lo term (about 2^-11 |q_k k_k| per
  product, up to half an fp16 ulp of the result) would change far more;
* end to end (GPU precompute, then the reference-signature kernel): the
  reference's own tolerance 0.1 against its direct Transformer-XL
  attention (golden fixtures where they exist), and the attention bar
  against the oracle on the same fp16 inputs.
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
DEV = "cuda:0"
REF_CONFIGS = [(32, 64, 2), (64, 64, 4), (64, 128, 4), (128, 128, 8), (256, 128, 8),
               (448, 128, 8)]


def _f16_ulp(x: torch.Tensor) -> torch.Tensor:
    a = x.abs().float().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def _gpu_pre(Q, K_rel, bu, bv):
    q_u, rel = neso_amd.precompute_bias_and_qu(*(torch.from_numpy(x).to(DEV)
                                                 for x in (Q, K_rel, bu, bv)))
    torch.cuda.synchronize()
    return q_u.cpu(), rel.cpu()


def _abs_dot(Q, K_rel, bv):
    """sum_k |(Q + bias_v)_ik K_rel[T-1-i+j]_k| per (h, i, j), float64."""
    nh, t, d = Q.shape
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    out = np.zeros((nh, t, t))
    for h in range(nh):
        qv = np.abs((Q[h] + bv[h]).astype(np.float64))
        out[h] = np.take_along_axis(qv @ np.abs(K_rel[h].astype(np.float64)).T, t - 1 - i + j,
                                    axis=1)
    return torch.from_numpy(out)


def _check_pre(Q, K_rel, bu, bv):
    q_u, rel = _gpu_pre(Q, K_rel, bu, bv)
    q_u_ref, rel_ref = A.precompute_bias_and_qu(Q, K_rel, bu, bv)
    assert torch.equal(q_u, torch.from_numpy(q_u_ref).half())
    rel_ref16 = torch.from_numpy(rel_ref).half()
    assert torch.isfinite(rel).all()
    diff = (rel.double() - rel_ref16.double()).abs()
    d = Q.shape[-1]
    bound = (_f16_ulp(torch.maximum(rel.float().abs(), rel_ref16.float().abs())).double()
             + (3 * d + 12) * 2.0 ** -24 * _abs_dot(Q, K_rel, bv))
    assert (diff <= bound).all(), (diff - bound).max().item()
    # Elements that round differently are rare (fp32 vs float64 accumulation).
    assert (diff > 0).double().mean().item() < 0.01
    return q_u, rel


@pytest.mark.parametrize("t,d,nh", REF_CONFIGS)
def test_reference_configs(gpu, t, d, nh):
    """The reference test's configs (:434-441) on its own seeded inputs (:317-327)."""
    Q, _, _, K_rel, bu, bv = I.reference_relpos_arrays(t, d, nh)
    _check_pre(Q, K_rel, bu, bv)


@pytest.mark.parametrize("t,d,nh", [(1, 64, 1), (2, 32, 3), (33, 64, 2), (100, 128, 1),
                                    (1500, 64, 2), (95, 64, 1), (129, 64, 1), (161, 128, 1),
                                    (200, 64, 1), (321, 64, 1)])
def test_ragged(gpu, t, d, nh):
    rs = np.random.RandomState(t + d)
    Q = rs.randn(nh, t, d).astype(np.float32)
    K_rel = rs.randn(nh, 2 * t - 1, d).astype(np.float32)
    bu, bv = (rs.randn(nh, d).astype(np.float32) * 0.1 for _ in range(2))
    _check_pre(Q, K_rel, bu, bv)


def test_fp16_range_checked(gpu):
    """Q + bias_v or K_rel elements at the fp16 limit (their hi part would
    be inf) are rejected before the launch; Q large but Q + bias_v within
    range is accepted."""
    rs = np.random.RandomState(4)
    t, d, nh = 40, 64, 2
    Q = rs.randn(nh, t, d).astype(np.float32)
    K_rel = rs.randn(nh, 2 * t - 1, d).astype(np.float32)
    bu, bv = (rs.randn(nh, d).astype(np.float32) * 0.1 for _ in range(2))
    bad = K_rel.copy()
    bad[1, 7, 3] = 7e4
    with pytest.raises(neso_amd.NesoArgumentError, match="K_rel: "):
        _gpu_pre(Q, bad, bu, bv)
    bad = Q.copy()
    bad[0, 5, 9] = -7e4
    with pytest.raises(neso_amd.NesoArgumentError, match="Q \\+ bias_v: "):
        _gpu_pre(bad, K_rel, bu, bv)
    Q2, bv2 = Q.copy(), bv.copy()
    Q2[0, :, 9] += 7e4
    bv2[0, 9] -= 7e4
    q_u, rel = _gpu_pre(Q2, K_rel, bu, bv2)
    assert torch.isfinite(rel).all()


def test_diagonal_structure(gpu):
    """K_rel row r one-hot on feature r % d, zero biases: rel_bias[i, j] is
    Q[i, (T - 1 - i + j) % d] exactly, which pins the relative index and its
    direction.  Q holds fp16 values, so its lo halves are 0 and the one
    nonzero product is exact."""
    t, d, nh = 70, 32, 2
    rs = np.random.RandomState(3)
    Q = rs.randn(nh, t, d).astype(np.float16).astype(np.float32)
    K_rel = np.zeros((nh, 2 * t - 1, d), np.float32)
    K_rel[:, np.arange(2 * t - 1), np.arange(2 * t - 1) % d] = 1.0
    z = np.zeros((nh, d), np.float32)
    _, rel = _gpu_pre(Q, K_rel, z, z)
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    want = np.take_along_axis(Q, np.broadcast_to((t - 1 - i + j) % d, (nh, t, t)), axis=2)
    assert torch.equal(rel, torch.from_numpy(want).half())


@pytest.mark.parametrize("t,d,nh", REF_CONFIGS)
def test_end_to_end_reference_mode(gpu, golden_dir, t, d, nh):
    """GPU precompute feeding the reference-signature rel-pos kernel (dense
    fp16 bias, (QK^T + B) * scale, fp16 output): the reference's tolerance
    0.1 (:373) against its direct attention, and the attention bar plus one
    fp16 ulp of O against the oracle on the same fp16 inputs."""
    Q, K, V, K_rel, bu, bv = I.reference_relpos_arrays(t, d, nh)
    scale = 1 / math.sqrt(d)
    q_u, rel = neso_amd.precompute_bias_and_qu(*(torch.from_numpy(x).to(DEV)
                                                 for x in (Q, K_rel, bu, bv)))
    kd, vd = (torch.from_numpy(x).half().to(DEV) for x in (K, V))
    o = torch.empty(nh, t, d, dtype=torch.float16, device=DEV)
    neso_amd.rel_pos_fa2_fwd(q_u, kd, vd, rel, o, t, d, scale, t * d, t * t, num_heads=nh,
                             bias_mode=neso_amd.NESO_BIAS_DENSE_SCALED_F16)
    torch.cuda.synchronize()
    out = o.float().cpu()
    ref = A.rel_pos_attention_dense(q_u.cpu(), kd.cpu(), vd.cpu(), rel.cpu(), scale)
    assert (out - ref).abs().max().item() <= 2e-3 + 2e-3
    path = golden_dir / f"relpos_ref_T{t}_d{d}_nh{nh}.npz"
    direct = (np.load(path)["expected"] if path.exists()
              else A.reference_rel_pos_attention(Q, K, V, K_rel, bu, bv, scale))
    assert np.abs(out.numpy() - direct).max() < 0.1
