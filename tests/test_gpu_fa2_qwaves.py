"""The generic FA2 kernel with 64-query workgroups (two query waves per key
group) against the CPU oracle.

``NESO_AMD_FA2_QW`` forces 2 or 4 query waves per key group (the library
picks 2 by itself when 128-query workgroups would leave compute units idle)
and ``NESO_AMD_FA2_KSPLIT`` the number of key groups; the fast kernel is
switched off.  Every mode of the generic kernel is covered: fp16 and f32
input, causal and windowed masks, the rel-pos table and the dense bias.
Bar: max abs error <= 2e-3 against the fp32 CPU oracle (f32 input: 5e-5).
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
def generic(monkeypatch):
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "0")

    def force(qw, ksplit=None):
        monkeypatch.setenv("NESO_AMD_FA2_QW", str(qw))
        if ksplit is None:
            monkeypatch.delenv("NESO_AMD_FA2_KSPLIT", raising=False)
        else:
            monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    return force


@pytest.mark.parametrize("ksplit", [None, 1, 2, 3, 4])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("n", [1, 33, 64, 65, 127, 200, 1000])
def test_fp16(gpu, generic, ksplit, causal, d, n):
    """Query blocks of 64 rows: ragged tails, one-row and exactly-one-block
    sequences, every key split (d = 128 falls back to two key groups where
    four do not fit the LDS)."""
    generic(2, ksplit)
    q, k, v = I.fa2_inputs(1, 2, n, d, seed=n + d + (ksplit or 0))
    out = neso_amd.attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal).cpu()
    ref = A.attention(q, k, v, 1 / math.sqrt(d), causal=causal)
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("ksplit", [1, 2])
def test_query_waves_agree(gpu, generic, ksplit):
    """Without a mask both workgroup shapes give each 32-query wave the same
    key blocks in the same order, so the results agree to the last bits."""
    q, k, v = I.fa2_inputs(1, 4, 777, 64, seed=5)
    generic(2, ksplit)
    a = neso_amd.attention(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    generic(4, ksplit)
    b = neso_amd.attention(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert (a - b).abs().max().item() <= 1e-6


@pytest.mark.parametrize("ksplit", [None, 2])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [32, 64])
@pytest.mark.parametrize("n", [1, 65, 300])
def test_f32_input(gpu, generic, ksplit, causal, d, n):
    generic(2, ksplit)
    g = torch.Generator().manual_seed(n + d)
    q, k, v = (torch.randn(1, 2, n, d, generator=g) for _ in range(3))
    out = neso_amd.attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal).cpu()
    ref = A.attention(q, k, v, 1 / math.sqrt(d), causal=causal)
    assert (out - ref).abs().max().item() <= 5e-5


@pytest.mark.parametrize("ksplit", [None, 2])
@pytest.mark.parametrize("n,wl,wr", [(7, 2, 1), (300, 100, 37), (300, 5, 290), (1500, 128, 128)])
def test_windows(gpu, generic, ksplit, n, wl, wr):
    generic(2, ksplit)
    heads, d = 2, 64
    q, k, v = (t[0].permute(1, 0, 2).contiguous() for t in I.fa2_inputs(1, heads, n, d, seed=n))
    out = neso_amd.window_attention(q.to(DEV), k.to(DEV), v.to(DEV), wl, wr,
                                    out_dtype=torch.float32).cpu()
    qh, kh, vh = (t.permute(1, 0, 2) for t in (q, k, v))
    ref = A.attention(qh, kh, vh, 1 / math.sqrt(d), window=(wl, wr)).permute(1, 0, 2)
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("ksplit", [None, 1, 3])
@pytest.mark.parametrize("h,n,d", [(8, 1500, 64), (2, 129, 128), (4, 300, 32), (1, 1, 64)])
def test_rel_pos_table(gpu, generic, ksplit, h, n, d):
    """The bias band of a 64-query block has 64 + 64 - 1 entries, one per
    thread of the 128-thread key group."""
    generic(2, ksplit)
    q, k, v, table = I.relpos_inputs(h, n, d, seed=n + h)
    out = neso_amd.rel_pos_attention(q.to(DEV), k.to(DEV), v.to(DEV), table.to(DEV)).cpu()
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(d))
    assert (out - ref).abs().max().item() <= TOL


def test_rel_pos_config4_default_dispatch(gpu, monkeypatch):
    """BASELINE config 4 with the library's own choice of workgroup shape."""
    monkeypatch.delenv("NESO_AMD_FA2_QW", raising=False)
    monkeypatch.delenv("NESO_AMD_FA2_KSPLIT", raising=False)
    cfg = I.RELPOS_CONFIG
    q, k, v, table = I.relpos_inputs(**cfg, seed=3)
    out = neso_amd.rel_pos_attention(q.to(DEV), k.to(DEV), v.to(DEV), table.to(DEV)).cpu()
    ref = A.rel_pos_attention_table(q, k, v, table, 1 / math.sqrt(cfg["d"]))
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("t,d,nh", [(64, 64, 4), (256, 128, 8)])
def test_dense_bias(gpu, generic, t, d, nh):
    generic(2)
    Q, K, V, K_rel, bu, bv = I.reference_relpos_arrays(t, d, nh)
    q_u, rel_bias = A.precompute_bias_and_qu(Q, K_rel, bu, bv)
    scale = 1 / math.sqrt(d)
    qd, kd, vd, bd = (torch.from_numpy(x).half().to(DEV) for x in (q_u, K, V, rel_bias))
    o = torch.empty(nh, t, d, dtype=torch.float16, device=DEV)
    neso_amd.rel_pos_fa2_fwd(qd, kd, vd, bd, o, t, d, scale, t * d, t * t, num_heads=nh,
                             bias_mode=neso_amd.NESO_BIAS_DENSE_SCALED_F16)
    torch.cuda.synchronize()
    ref = A.rel_pos_attention_dense(qd.cpu(), kd.cpu(), vd.cpu(), bd.cpu(), scale)
    assert (o.float().cpu() - ref).abs().max().item() <= TOL + 2e-3
