"""The pipelined fast FA2 kernel against its serialised debug build, bit for bit.

libneso_amd_serial.so is the same library with NESO_FA2_SERIAL_LDS: every
LDS phase of the fast kernel ends in a full wait (s_waitcnt vmcnt(0)) and a
workgroup barrier, so no LDS-DMA write overlaps an LDS read and no wave runs
ahead within a step.  The arithmetic is unchanged, so any difference from the
pipelined 4-slot ring (libneso_amd.so) would be a race in its slot
bookkeeping (the hazard the reference's barrier elision carries,
src/neso/backend/codegen/lowering.py:763-790).  Shapes: the headline, the
d = 128 causal config (reduced batch), ragged and windowed cases, and the
rescale path, each forced onto the fast kernel.
"""
from __future__ import annotations

import pytest
import torch

from neso_amd import _lib
from oracle import inputs as I

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def libs():
    return _lib.load(), _lib.load_variant(_lib.SERIAL_LIB_PATH)


def _run(lib, q, k, v, causal, wl=None, wr=None):
    b, h, n, d = q.shape
    o = torch.full(q.shape, float("nan"), device=DEV)
    if wl is None:
        st = lib.neso_flash_attention_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                          n, d, d, d ** -0.5, d, b * h, n * d, n * d, int(causal),
                                          None)
    else:
        st = lib.neso_flash_attention_window_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                 o.data_ptr(), n, n * d, d, d ** -0.5, wl, wr,
                                                 b * h, d, _lib.NESO_OUT_F32, None)
    assert st == _lib.NESO_OK
    torch.cuda.synchronize()
    return o.cpu()


@pytest.mark.parametrize("b,h,n,d,causal", [
    (1, 16, 2048, 64, False),   # the headline
    (1, 4, 4096, 128, True),    # config 3's shape per head (B=2, H=32 in the bench)
    (1, 16, 2048, 64, True),
    (1, 3, 1000, 64, False),
    (2, 2, 777, 128, True),
    (1, 2, 65, 64, False),
])
def test_pipelined_equals_serialised(gpu, libs, monkeypatch, b, h, n, d, causal):
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    q, k, v = (t.to(DEV) for t in I.fa2_inputs(b, h, n, d, seed=n + d))
    fast, serial = (_run(lib, q, k, v, causal) for lib in libs)
    assert torch.isfinite(fast).all()
    assert torch.equal(fast, serial)


@pytest.mark.parametrize("ksplit", [1, 2])
def test_rescale_path_equal(gpu, libs, monkeypatch, ksplit):
    """Key blocks whose logits jump, so the slow path re-reads a block's K."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    q, k, v = I.fa2_inputs(1, 2, 768, 64, seed=31)
    k = k.float()
    for blk, f in enumerate([0.5, 1.5, 3.0, 6.0, 9.0, 12.0] * 2):
        k[:, :, 64 * blk:64 * blk + 64] *= f
    q, k, v = (t.half().to(DEV) for t in (q, k, v))
    fast, serial = (_run(lib, q, k, v, False) for lib in libs)
    assert torch.equal(fast, serial)


def test_window_equal(gpu, libs, monkeypatch):
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    q, k, v = (t.to(DEV) for t in I.fa2_inputs(1, 4, 1500, 64, seed=4))
    fast, serial = (_run(lib, q, k, v, True, wl=300, wr=40) for lib in libs)
    assert torch.equal(fast, serial)


@pytest.mark.parametrize("d,causal", [(64, False), (64, True), (128, False)])
def test_two_query_waves_equal(gpu, libs, monkeypatch, d, causal):
    """64-query workgroups, four key groups of two waves (d = 128: two)."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_QW", "2")
    q, k, v = (t.to(DEV) for t in I.fa2_inputs(1, 3, 1000, d, seed=d))
    fast, serial = (_run(lib, q, k, v, causal) for lib in libs)
    assert torch.isfinite(fast).all()
    assert torch.equal(fast, serial)


@pytest.mark.parametrize("d,ksplit", [(64, 4), (128, 4), (128, 2)])
def test_paired_two_query_waves_equal(gpu, libs, monkeypatch, d, ksplit):
    """Paired causal blocks on 64-query workgroups: the second pass's loads
    reuse the slots the first pass's merge read."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_QW", "2")
    monkeypatch.setenv("NESO_AMD_FA2_PAIR", "1")
    monkeypatch.setenv("NESO_AMD_FA2_KSPLIT", str(ksplit))
    q, k, v = (t.to(DEV) for t in I.fa2_inputs(1, 3, 1000, d, seed=d + ksplit))
    fast, serial = (_run(lib, q, k, v, True) for lib in libs)
    assert torch.isfinite(fast).all()
    assert torch.equal(fast, serial)


def _run_table(lib, q, k, v, table):
    h, n, d = q.shape
    o = torch.full(q.shape, float("nan"), device=DEV)
    st = lib.neso_rel_pos_fa2_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(),
                                  o.data_ptr(), n, d, d ** -0.5, n * d, 2 * n - 1, h, d,
                                  _lib.NESO_BIAS_TABLE_F32, _lib.NESO_OUT_F32, None)
    assert st == _lib.NESO_OK
    torch.cuda.synchronize()
    return o.cpu()


@pytest.mark.parametrize("qw", [2, 4])
def test_rel_pos_table_equal(gpu, libs, monkeypatch, qw):
    """The bias band's wave-private slots: BASELINE config 4 on the fast
    kernel with either workgroup shape."""
    monkeypatch.setenv("NESO_AMD_FA2_FAST", "2")
    monkeypatch.setenv("NESO_AMD_FA2_QW", str(qw))
    cfg = I.RELPOS_CONFIG
    q, k, v, table = (t.to(DEV) for t in I.relpos_inputs(**cfg, seed=1))
    fast, serial = (_run_table(lib, q, k, v, table) for lib in libs)
    assert torch.isfinite(fast).all()
    assert torch.equal(fast, serial)
