"""The streaming-floor probe (`neso_stream_probe`, a measurement aid that
bench.py times beside the int4 GEMV): the read kernel must read every byte
it is given (the XOR of the buffer reaches the sink when it is the key, and
the sink is untouched otherwise), and the empty kernel must run at the
requested grid."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from neso_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4096, 1), (25392640, 768), (1 << 20, 17),
                                         (16 * 16 * 256 * 3, 3)])
def test_stream_read_covers_every_byte(gpu, nbytes, grid):
    lib = _lib.load()
    g = torch.Generator().manual_seed(nbytes + grid)
    host = torch.randint(-(1 << 31), (1 << 31) - 1, (nbytes // 4,), generator=g, dtype=torch.int64)
    host = host.to(torch.int32)
    buf = host.to(DEV)
    xor = int(np.bitwise_xor.reduce(host.numpy().view(np.uint32)))
    sink = torch.zeros(4, dtype=torch.int32, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.neso_stream_probe(buf.data_ptr(), nbytes, grid, 1, (xor + 1) & 0xFFFFFFFF,
                                 sink.data_ptr(), st) == _lib.NESO_OK
    torch.cuda.synchronize()
    assert int(sink[0]) == 0
    assert lib.neso_stream_probe(buf.data_ptr(), nbytes, grid, 1, xor, sink.data_ptr(),
                                 st) == _lib.NESO_OK
    torch.cuda.synchronize()
    assert int(sink[0]) & 0xFFFFFFFF == xor
    assert lib.neso_stream_probe(None, 0, grid, 0, 0, None, st) == _lib.NESO_OK
    torch.cuda.synchronize()
