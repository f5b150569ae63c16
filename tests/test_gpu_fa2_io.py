"""FA2 with O in the input type: the reference's hand-written kernel signature.

Reference: bench/bench_flash_attention.py:142-152, `flash_attention_fwd(Q, K,
V, O, N, d_head, scale)` with Q, K, V and O all of `io_type` (half or float,
:106), O row r at r * d_head (:361); correctness bar there 0.05 (half) /
0.01 (float) at :441.  Here:

* fp16 io: max abs error <= 2e-3 + the fp16 rounding of O (half an ulp,
  |O| * 2^-11) against the fp32 CPU oracle on the fp16 inputs;
* fp32 io: max abs error <= 5e-5 against the float64 oracle on the fp32
  inputs (the split-precision kernel).
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


def _f16_bar(ref):
    return 2e-3 + ref.abs() * 2.0 ** -11


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("n,bh", [(1, 1), (64, 1), (100, 3), (256, 1), (1000, 2), (2048, 16)])
def test_f16_io(gpu, d, n, bh):
    q, k, v = I.fa2_inputs(1, bh, n, d, seed=n + d)
    o = torch.empty((bh, n, d), dtype=torch.float16, device=DEV)
    scale = 1 / math.sqrt(d)
    # Reference positional order: Q, K, V, O, N, d_head, scale.
    neso_amd.launch("flash_attention_io_fwd", q.to(DEV), k.to(DEV), v.to(DEV), o, n, d, scale,
                    batch_heads=bh)
    torch.cuda.synchronize()
    ref = A.attention(q, k, v, scale)[0]
    out = o.float().cpu()
    assert torch.isfinite(out).all()
    assert ((out - ref).abs() <= _f16_bar(ref)).all(), (out - ref).abs().max().item()


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("n,bh", [(1, 1), (77, 2), (256, 1), (512, 4)])
def test_f32_io(gpu, d, n, bh):
    g = torch.Generator().manual_seed(n * d)
    q, k, v = (torch.randn((bh, n, d), generator=g) for _ in range(3))
    o = torch.full((bh, n, d), float("nan"), device=DEV)
    scale = 1 / math.sqrt(d)
    neso_amd.flash_attention_io_fwd(q.to(DEV), k.to(DEV), v.to(DEV), o, n, d, scale,
                                    batch_heads=bh)
    torch.cuda.synchronize()
    ref = A.attention(q, k, v, scale, dtype=torch.float64)
    err = (o.cpu().double() - ref).abs().max().item()
    assert err <= 5e-5, err


@pytest.mark.parametrize("n,d", [(128, 64), (256, 64), (128, 128), (256, 128), (512, 128)])
def test_reference_rows_f16_io(gpu, golden_dir, n, d):
    """Reference generator (tests/test_flash_attention.py:268-275) inputs as
    fp16 through the fp16-io kernel; rows 0 and N/2 against the fixture."""
    z = np.load(golden_dir / f"fa2_ref_N{n}_d{d}.npz")
    q, k, v = (torch.from_numpy(z[x].reshape(n, d)).half() for x in "qkv")
    o = torch.empty((n, d), dtype=torch.float16, device=DEV)
    neso_amd.flash_attention_io_fwd(q.to(DEV), k.to(DEV), v.to(DEV), o, n, d, float(z["scale"]))
    torch.cuda.synchronize()
    out = o.float().cpu()
    for r, exp in zip(z["rows"], z["expected"]):
        assert np.abs(out[r].numpy() - exp).max() < 0.05  # the reference's half tolerance
    ref = A.attention(q, k, v, float(z["scale"]))
    assert ((out - ref).abs() <= _f16_bar(ref)).all()


def test_io_errors(gpu):
    x = torch.zeros(64, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(TypeError):  # O must share Q's type
        neso_amd.flash_attention_io_fwd(x, x, x, x.float(), 64, 64, 0.125)
    with pytest.raises(ValueError, match="span"):
        neso_amd.flash_attention_io_fwd(x, x, x, x, 64, 64, 0.125, batch_heads=2)
    with pytest.raises(neso_amd.NesoArgumentError):
        neso_amd.flash_attention_io_fwd(x, x, x, x, 64, 48, 0.125, batch_heads=1)


def test_f32_io_range_rescaled(gpu):
    """fp32 io inputs outside the split's range are measured on the launch
    stream (data written there just before the call is what is measured)
    and rescaled by powers of two: V with an element at 7e4 and inputs of
    size 1e-5 both match the fp64 oracle to the fp32 bar relative to V's
    size; check_range=False skips the measurement."""
    n, d = 64, 64
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(n, d, generator=g).to(DEV) for _ in range(3))
    o = torch.empty(n, d, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        v[3, 2] = 7e4  # written on the launch stream, not the default one
    neso_amd.flash_attention_io_fwd(q, k, v, o, n, d, 0.125, stream=s)
    torch.cuda.synchronize()
    ref = A.attention(q.cpu()[None], k.cpu()[None], v.cpu()[None], 0.125, dtype=torch.float64)[0]
    assert (o.cpu().double() - ref).abs().max().item() <= 5e-5 * 7e4 / 4
    for x in (q, k, v):
        x.mul_(1e-5)
    neso_amd.flash_attention_io_fwd(q, k, v, o, n, d, 0.125)
    torch.cuda.synchronize()
    ref = A.attention(q.cpu()[None], k.cpu()[None], v.cpu()[None], 0.125, dtype=torch.float64)[0]
    assert (o.cpu().double() - ref).abs().max().item() <= 5e-5 * 1e-5 * 7e4 / 4
    neso_amd.flash_attention_io_fwd(q, k, v, o, n, d, 0.125, check_range=False)
    torch.cuda.synchronize()
