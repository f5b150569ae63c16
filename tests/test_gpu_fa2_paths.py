"""Both FA2 kernels for fp16 Q/K/V, and the fast kernel's rescale paths, vs the CPU oracle.

head_dim 64 and 128 without a bias run the fast kernel where it is the
faster one; ``NESO_AMD_FA2_FAST=2`` forces it wherever it applies and
``NESO_AMD_FA2_FAST=0`` forces the generic kernel.  Both must meet the
attention bar (max abs error <= 2e-3 against the fp32 CPU softmax(QK^T s) V)
for every key split, ragged and block-aligned lengths, causal or not.

The fast kernel bounds each block's P by the lane's row sum instead of
forming a row max (the running max is raised only when a block's fp16 P sum
exceeds 2^12).  The inputs below force that path: key blocks whose logits
jump far above the running max, fall far below it, or are huge throughout.
"""
from __future__ import annotations

import math

import pytest
import torch

import neso_amd
from oracle import attention as A
from oracle import inputs as I

pytestmark = pytest.mark.gpu
TOL = 2e-3


def run(q, k, v, causal=False, scale=None):
    dev = torch.device("cuda:0")
    out = neso_amd.attention(q.to(dev), k.to(dev), v.to(dev), causal=causal, scale=scale)
    torch.cuda.synchronize()
    return out.cpu()


def check(q, k, v, causal=False, scale=None, tol=TOL):
    s = 1 / math.sqrt(q.shape[-1]) if scale is None else scale
    out = run(q, k, v, causal, scale)
    ref = A.attention(q, k, v, s, causal=causal)
    assert torch.isfinite(out).all()
    err = (out - ref).abs().max().item()
    assert err <= tol, err
    return err


@pytest.mark.parametrize("path", ["fast", "generic"])
@pytest.mark.parametrize("ksplit", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 31, 32, 33, 63, 64, 65, 128, 192, 320, 1000])
def test_paths_and_splits(gpu, monkeypatch, path, ksplit, causal, d, n):
    """Key groups with equal and unequal block counts (odd block totals),
    single-block groups and tails shorter than a block (blocks are 64 keys
    at d = 64 and 32 keys at d = 128 in the fast kernel)."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2" if path == "fast" else "0")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    q, k, v = I.fa2_inputs(1, 2, n, d, seed=n + 7 * ksplit + d)
    check(q, k, v, causal)


def _stepped_keys(n, steps, seed, d=64, block=64):
    """K rows scaled by a factor that changes per key block."""
    q, k, v = I.fa2_inputs(1, 2, n, d, seed=seed)
    k = k.float()
    for b in range(0, n, block):
        k[:, :, b:b + block] *= steps[(b // block) % len(steps)]
    return q, k.half(), v


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("ksplit", [1, 2])
@pytest.mark.parametrize("causal", [False, True])
def test_running_max_jumps_up(gpu, monkeypatch, ksplit, causal, d):
    """Each later block's logits are far above the running max: P of the new
    block would overflow fp16 without the slow path's rescale."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    q, k, v = _stepped_keys(768, [0.5, 1.5, 3.0, 6.0, 9.0, 12.0], seed=31, d=d, block=128 // (d // 32))
    check(q, k, v, causal)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("ksplit", [1, 2])
def test_running_max_falls(gpu, monkeypatch, ksplit, d):
    """The first block holds the largest logits; later blocks contribute
    little and must not disturb the result (no rescale needed)."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    q, k, v = _stepped_keys(768, [12.0, 4.0, 1.0, 0.25, 0.0, 0.1], seed=32, d=d,
                            block=128 // (d // 32))
    check(q, k, v)


@pytest.mark.parametrize("d", [64, 128])
def test_alternating_magnitudes(gpu, monkeypatch, d):
    """Large and small logit blocks alternate: the running max rises in
    steps and the fast path's bound is exceeded repeatedly."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    q, k, v = _stepped_keys(1024, [0.2, 8.0, 0.2, 11.0, 0.2, 14.0, 0.2, 16.0], seed=33, d=d,
                            block=128 // (d // 32))
    check(q, k, v)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("scale", [4.0, -4.0, 1e-6])
def test_extreme_scales(gpu, monkeypatch, scale, d):
    """|scale * log2(e)| far above 1 (logits of hundreds) and nearly 0."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    q, k, v = I.fa2_inputs(1, 2, 256, d, seed=34)
    check(q, k, v, scale=scale)


def test_fast_equals_generic(gpu, monkeypatch):
    """The two kernels agree with each other on the headline shape (a check
    that does not depend on the oracle)."""
    q, k, v = I.fa2_inputs(1, 16, 2048, 64, seed=35)
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    fast = run(q, k, v)
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "0")
    generic = run(q, k, v)
    assert (fast - generic).abs().max().item() <= 1e-3


@pytest.mark.parametrize("ksplit", [1, 2])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 128, 129, 384, 1000, 1500])
def test_fast_paired_causal_blocks(gpu, monkeypatch, ksplit, d, n):
    """Fast kernel, causal, with paired query blocks (workgroup x takes
    blocks nqb-1-x and x; an odd middle block once)."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    monkeypatch.setenv("NESO_AMD_FA2_PAIR", "1")
    q, k, v = I.fa2_inputs(1, 3, n, d, seed=n + d + ksplit)
    check(q, k, v, causal=True)


@pytest.mark.parametrize("ksplit", [1, 2, 4])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 64, 65, 128, 129, 384, 1000, 1500, 2048])
def test_fast_paired_two_query_waves(gpu, monkeypatch, ksplit, d, n):
    """Paired query blocks on 64-query workgroups (two query waves per key
    group, two K and two V slots): workgroup x takes the 64-row blocks
    nqb-1-x and x, one pass each, with a barrier between the first pass's
    merge and the second pass's loads."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_QW", "2")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    monkeypatch.setenv("NESO_AMD_FA2_PAIR", "1")
    q, k, v = I.fa2_inputs(1, 3, n, d, seed=n + d + 5 * ksplit)
    check(q, k, v, causal=True)


@pytest.mark.parametrize("d", [64, 128])
def test_fast_paired_two_query_waves_rescale(gpu, monkeypatch, d):
    """The same with logits that jump between key blocks (the slow path on
    the kept scores) and with fp16 output through the window entry."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_QW", "2")
    monkeypatch.setenv("NESO_AMD_FA2_PAIR", "1")
    q, k, v = I.fa2_inputs(1, 2, 1000, d, seed=3 * d)
    k = k.float()
    for blk, f in enumerate([0.5, 3.0, 9.0, 1.0, 12.0, 2.0, 6.0, 0.25] * 2):
        k[:, :, 64 * blk:64 * blk + 64] *= f
    k = k.half()
    check(q, k, v, causal=True)
    n, dev = q.shape[-2], torch.device("cuda:0")
    qs, ks, vs = (t[0].permute(1, 0, 2).contiguous().to(dev) for t in (q, k, v))
    out = neso_amd.window_attention(qs, ks, vs, n, 0, out_dtype=torch.float16)
    out = out.float().cpu().permute(1, 0, 2)
    ref = A.attention(q[0], k[0], v[0], 1 / math.sqrt(d), causal=True)
    assert ((out - ref).abs() <= TOL + ref.abs() * 2.0 ** -11).all()


@pytest.mark.parametrize("ksplit", [1, 2, 3])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 129, 191, 384, 1000, 1500, 2048])
def test_fast_causal_halves(gpu, monkeypatch, ksplit, d, n):
    """Fast kernel, causal, 64-row halves: workgroup x takes the 64-row
    blocks x and n64-1-x (an odd middle block alone), each wave stops after
    its last visible block, and with two key groups the second group's
    waves take the slices two apart."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    monkeypatch.setenv("NESO_AMD_FA2_PAIR", "2")
    q, k, v = I.fa2_inputs(1, 3, n, d, seed=n + d + 7 * ksplit)
    check(q, k, v, causal=True)


@pytest.mark.parametrize("d", [64, 128])
def test_fast_causal_halves_rescale_and_f16(gpu, monkeypatch, d):
    """Halves with logits that jump between blocks (the slow path, per wave)
    and with fp16 output."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_PAIR", "2")
    q, k, v = I.fa2_inputs(1, 2, 1000, d, seed=d)
    k = k.float()
    for blk, f in enumerate([0.5, 3.0, 9.0, 1.0, 12.0, 2.0, 6.0, 0.25] * 2):
        k[:, :, 64 * blk:64 * blk + 64] *= f
    k = k.half()
    check(q, k, v, causal=True)
    # fp16 output through the window entry with (N, 0): full causal, so the
    # halves apply there too.
    n, dev = q.shape[-2], torch.device("cuda:0")
    qs, ks, vs = (t[0].permute(1, 0, 2).contiguous().to(dev) for t in (q, k, v))
    out = neso_amd.window_attention(qs, ks, vs, n, 0, out_dtype=torch.float16)
    out = out.float().cpu().permute(1, 0, 2)
    ref = A.attention(q[0], k[0], v[0], 1 / math.sqrt(d), causal=True)
    assert ((out - ref).abs() <= TOL + ref.abs() * 2.0 ** -11).all()


@pytest.mark.parametrize("n,wl,wr", [(300, 100, 37), (1500, 128, 128), (1000, 1000, 0)])
@pytest.mark.parametrize("pair,qw", [("1", "4"), ("2", "4"), ("1", "2"), ("2", "2")])
def test_fast_paired_windows(gpu, monkeypatch, n, wl, wr, pair, qw):
    """Windows with pairing forced: 64-row halves (2) apply only without a
    window and with four query waves, so a windowed call (or a two-query-wave
    one) falls back to whole blocks; paired blocks (1) take any window."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_PAIR", pair)
    monkeypatch.setenv("NESO_AMD_FA2_QW", qw)
    heads, d = 2, 64
    q, k, v = (t[0].permute(1, 0, 2).contiguous() for t in I.fa2_inputs(1, heads, n, d, seed=n))
    dev = torch.device("cuda:0")
    out = neso_amd.window_attention(q.to(dev), k.to(dev), v.to(dev), wl, wr,
                                    out_dtype=torch.float32).cpu()
    qh, kh, vh = (t.permute(1, 0, 2) for t in (q, k, v))
    ref = A.attention(qh, kh, vh, 1 / math.sqrt(d), window=(wl, wr)).permute(1, 0, 2)
    assert (out - ref).abs().max().item() <= TOL
