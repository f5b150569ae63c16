"""The streaming-floor probe (`neso_stream_probe`, a measurement aid that
bench.py times beside the int4 GEMV): the read kernel must read every byte
it is given, lane t of T taking pieces t, t + T, ... (mode 2 writes each
lane's XOR, which must equal the host's per-lane XOR of those pieces), the
timed form must store only when a lane's XOR is the key, and the empty
kernel must run at the requested grid."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from neso_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def lane_xors(words: np.ndarray, grid: int) -> np.ndarray:
    """XOR of the 16-byte pieces lane t reads (t, t + T, ...), zeros past the end."""
    T = grid * 256
    pieces = np.bitwise_xor.reduce(words.reshape(-1, 4), axis=1)
    per = -(-pieces.size // T)
    padded = np.zeros(per * T, dtype=np.uint32)
    padded[:pieces.size] = pieces
    return np.bitwise_xor.reduce(padded.reshape(per, T), axis=0)


@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4096, 1), (25392640, 768), (1 << 20, 17),
                                         (16 * 16 * 256 * 3, 3), (16 * 1000 + 48, 2)])
def test_stream_read_covers_every_byte(gpu, nbytes, grid):
    lib = _lib.load()
    g = torch.Generator().manual_seed(nbytes + grid)
    host = torch.randint(-(1 << 31), (1 << 31) - 1, (nbytes // 4,), generator=g, dtype=torch.int64)
    host = host.to(torch.int32)
    buf = host.to(DEV)
    expect = lane_xors(host.numpy().view(np.uint32), grid)
    st = torch.cuda.current_stream().cuda_stream

    sink = torch.zeros(grid * 256, dtype=torch.int32, device=DEV)
    assert lib.neso_stream_probe(buf.data_ptr(), nbytes, grid, 2, 0, sink.data_ptr(),
                                 st) == _lib.NESO_OK
    torch.cuda.synchronize()
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), expect)

    # Timed form: a key no lane reaches leaves the sink alone; lane 0's XOR lands in sink[0].
    miss = next(k for k in range(1, 1 << 20) if k not in set(expect.tolist()))
    sink.fill_(-7)
    assert lib.neso_stream_probe(buf.data_ptr(), nbytes, grid, 1, miss, sink.data_ptr(),
                                 st) == _lib.NESO_OK
    torch.cuda.synchronize()
    assert int(sink[0]) == -7
    assert lib.neso_stream_probe(buf.data_ptr(), nbytes, grid, 1, int(expect[0]),
                                 sink.data_ptr(), st) == _lib.NESO_OK
    torch.cuda.synchronize()
    assert int(sink[0]) & 0xFFFFFFFF == int(expect[0])
    assert lib.neso_stream_probe(None, 0, grid, 0, 0, None, st) == _lib.NESO_OK
    torch.cuda.synchronize()
