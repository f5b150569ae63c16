"""The shader-clock sampler (neso_clock_sample) on the GPU: pairs of
(shader clock, 100 MHz reference clock) one gap apart, from which the bench
reports the clock a workload ran at."""
from __future__ import annotations

import ctypes

import pytest
import torch

from neso_amd import _lib

pytestmark = pytest.mark.gpu


def test_idle_clock_is_plausible(gpu):
    lib = _lib.load()
    n, gap = 200, 100  # one pair per microsecond
    buf = torch.zeros(2 * n, dtype=torch.int64, device="cuda:0")
    st = lib.neso_clock_sample(ctypes.c_void_p(buf.data_ptr()), n, gap,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.NESO_OK, lib.neso_last_error()
    torch.cuda.synchronize()
    s = buf.cpu().view(n, 2)
    dt, dr = (s[1:, 0] - s[:-1, 0]).double(), (s[1:, 1] - s[:-1, 1]).double()
    assert (dr >= gap).all() and (dt > 0).all()
    mhz = (s[-1, 0] - s[0, 0]).item() / ((s[-1, 1] - s[0, 1]).item() / 100.0)
    assert 50.0 < mhz < 5000.0, mhz
