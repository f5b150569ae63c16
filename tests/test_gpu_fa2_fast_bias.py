"""The fast FA2 kernel with two query waves per key group and with the f32
bias table, against the CPU oracle.

``NESO_AMD_FA2_FAST=2`` forces the fast kernel, ``NESO_AMD_FA2_QW`` its
query waves per key group (2: 64-query workgroups with two K and two V LDS
slots per key group and the scores kept in registers for the slow path)
and ``NESO_AMD_FA2_KSPLIT`` its key groups (1, 2, and 4 with two query
waves).  The table form carries the bias band of each block in the initial
accumulator of the score MFMAs, in score units (t / |scale|): 32-key blocks
with four query waves, 64-key blocks (two bands per lane) with two.
Bar: max abs error <= 2e-3 against the fp32 CPU oracle
(tests/test_rel_pos_fa2.py:155-253 for the biased softmax).
"""
from __future__ import annotations

import math

import pytest
import torch

import neso_amd
from oracle import attention as A
from oracle import inputs as I

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-3


@pytest.fixture
def fast(monkeypatch):
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")

    def force(qw=None, ksplit=None):
        for name, val in (("NESO_AMD_FA2_QW", qw), ("NESO_AMD_FA2_KSPLIT", ksplit)):
            if val is None:
                monkeypatch.delenv(name, raising=False)
            else:
                monkeypatch.setenv(name, str(val))
    return force


def table_gpu(q, k, v, table, scale=None, out_dtype=torch.float32):
    out = neso_amd.rel_pos_attention(q.to(DEV), k.to(DEV), v.to(DEV), table.to(DEV),
                                     scale=scale, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu()


@pytest.mark.parametrize("ksplit", [None, 1, 2, 4])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 33, 64, 65, 127, 200, 1000])
def test_two_query_waves(gpu, fast, ksplit, causal, d, n):
    """64-query workgroups without a bias: ragged tails, one-row and
    exactly-one-block sequences, every key split."""
    fast(2, ksplit)
    q, k, v = I.fa2_inputs(1, 2, n, d, seed=n + d + (ksplit or 0))
    out = neso_amd.attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal).cpu()
    ref = A.attention(q, k, v, 1 / math.sqrt(d), causal=causal)
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("ksplit", [None, 2, 4])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n,wl,wr", [(7, 2, 1), (300, 100, 37), (300, 5, 290), (1500, 128, 128)])
def test_two_query_waves_windows(gpu, fast, ksplit, d, n, wl, wr):
    """Sliding windows on 64-query workgroups: blocks partly outside some
    query's window take the slow path on the scores kept in registers."""
    fast(2, ksplit)
    heads = 2
    q, k, v = (t[0].permute(1, 0, 2).contiguous() for t in I.fa2_inputs(1, heads, n, d, seed=n + d))
    out = neso_amd.window_attention(q.to(DEV), k.to(DEV), v.to(DEV), wl, wr,
                                    out_dtype=torch.float32).cpu()
    qh, kh, vh = (t.permute(1, 0, 2) for t in (q, k, v))
    ref = A.attention(qh, kh, vh, 1 / math.sqrt(d), window=(wl, wr)).permute(1, 0, 2)
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("qw,ksplit", [(2, None), (2, 1), (2, 2), (4, None), (4, 1), (4, 2)])
@pytest.mark.parametrize("h,n,d", [(8, 1500, 64), (2, 129, 128), (1, 1, 64), (3, 37, 64),
                                   (2, 31, 64), (2, 33, 128), (1, 1023, 64), (2, 2048, 128)])
def test_rel_pos_table(gpu, fast, qw, ksplit, h, n, d):
    fast(qw, ksplit)
    q, k, v, table = I.relpos_inputs(h, n, d, seed=n + h + qw)
    out = table_gpu(q, k, v, table)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(d))
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("path", ["fast-2-1", "fast-2-2", "fast-4-1", "fast-4-2", "generic"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [129, 161, 193, 225, 257, 289, 321, 385])
def test_rel_pos_table_entry_zero(gpu, monkeypatch, path, d, n):
    """Row 0 against key N-1 is the only pair that uses table entry 0.  Every
    key-block count and unrolled-step position of the group's last block:
    the band load of that entry must not read as zero (regression: its
    offset was once split into a wrapped negative register part plus an
    immediate, which the buffer range check rejects)."""
    if path == "generic":
        monkeypatch.setenv("NESO_AMD_FA2_FAST", "0")
    else:
        _, qw, ks = path.split("-")
        monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
        monkeypatch.setenv("NESO_AMD_FA2_QW", qw)
        monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", ks)
    q, k, v, table = I.relpos_inputs(2, n, d, seed=n + d)
    table[:, 0] = 3.0  # a large entry 0: dropping it moves row 0 by far more than the bar
    out = table_gpu(q, k, v, table)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(d))
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("qw", [2, 4])
def test_rel_pos_table_fp16_out(gpu, fast, qw):
    fast(qw)
    q, k, v, table = I.relpos_inputs(4, 300, 64, seed=9)
    out = table_gpu(q, k, v, table, out_dtype=torch.float16)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(64))
    assert (out - ref).abs().max().item() <= TOL + 2e-3


@pytest.mark.parametrize("qw,ksplit", [(2, None), (4, 2)])
def test_rel_pos_rescale_path(gpu, fast, qw, ksplit):
    """A table that grows by 0.05 per key of distance: every row's logits
    rise by ~1.6 (log2 units ~2.3) per 32-key block, so blocks past the
    lazy bound take the slow path (exact row max, O and l rescaled; with
    four query waves the scores are recomputed from LDS with the band
    again, with two the kept scores are reused)."""
    fast(qw, ksplit)
    h, n, d = 2, 1200, 64
    q, k, v, _ = I.relpos_inputs(h, n, d, seed=2)
    idx = torch.arange(2 * n - 1, dtype=torch.float32)
    table = (-(idx - (n - 1)) * 0.05).expand(h, -1).contiguous()  # = 0.05 (j - i)
    out = table_gpu(q, k, v, table)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(d))
    assert torch.isfinite(out).all()
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("scale", [-0.125, 0.01, 1e-30])
def test_rel_pos_scales(gpu, fast, scale):
    """A negative scale flips Q; the band is divided by |scale|.  Below a
    scale of 1e-20 t / |scale| could overflow, so the call takes the generic
    kernel (the result is then the bias-only softmax)."""
    fast(2)
    h, n, d = 2, 400, 64
    q, k, v, table = I.relpos_inputs(h, n, d, seed=7)
    out = table_gpu(q, k, v, table, scale=scale)
    ref = A.rel_pos_attention_table(q, k, v, table, scale)
    assert (out - ref).abs().max().item() <= TOL


def test_fast_and_generic_agree(gpu, monkeypatch):
    """Config 4 on both kernels (the generic one with its own choice of
    workgroup shape): two independent implementations of the biased
    softmax, both within the bar of the oracle and of each other."""
    cfg = I.RELPOS_CONFIG
    q, k, v, table = I.relpos_inputs(**cfg, seed=11)
    monkeypatch.delenv("NESO_AMD_FA2_QW", raising=False)
    monkeypatch.delenv("NESO_AMD_FA2_KSPLIT", raising=False)
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    a = table_gpu(q, k, v, table)
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "0")
    b = table_gpu(q, k, v, table)
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(cfg["d"]))
    assert (a - ref).abs().max().item() <= TOL
    assert (b - ref).abs().max().item() <= TOL
    assert (a - b).abs().max().item() <= TOL


def test_strided_rows(gpu, fast):
    """Row stride 96 > d = 64 and a head stride with a gap, through the
    reference-signature entry point with the table bias."""
    fast(2)
    h, n, d, stride = 3, 150, 64, 96
    q, k, v, table = I.relpos_inputs(h, n, d, seed=5)
    stride_h = n * stride + 32

    def pad(x):
        buf = torch.zeros(h * stride_h, dtype=x.dtype)
        for i in range(h):
            buf[i * stride_h:i * stride_h + n * stride].view(n, stride)[:, :d] = x[i]
        return buf.to(DEV)

    qp, kp, vp = pad(q), pad(k), pad(v)
    o = torch.zeros(h * stride_h, dtype=torch.float32, device=DEV)
    neso_amd.rel_pos_fa2_fwd(qp, kp, vp, table.to(DEV), o, n, stride, d ** -0.5, stride_h,
                             2 * n - 1, num_heads=h, head_dim=d,
                             bias_mode=neso_amd.NESO_BIAS_TABLE_F32)
    torch.cuda.synchronize()
    oc = o.cpu()
    out = torch.stack([oc[i * stride_h:i * stride_h + n * stride].view(n, stride)[:, :d]
                       for i in range(h)])
    ref = A.rel_pos_attention_table(q, k, v, table, d ** -0.5)
    assert (out - ref).abs().max().item() <= TOL
