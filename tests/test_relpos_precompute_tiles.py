"""CPU walk of the rel-pos precompute kernel's work assignment.

neso_amd/csrc/relpos_pre.hip: workgroup (x, y = head, z) covers query rows
128 x .. 128 x + 127, one 32-row block per wave, and relative-position tiles
r0 = rlo + 32 t for t in [8 z, 8 z + 8) of its row group; a wave computes a
tile only if its rows use it, and element (a, c) of a tile goes to
rel_bias[iw + a][r0 + c - (T - 1) + iw + a] when that lies in [0, T)^2.
The grid is (cdiv(T, 128), heads, cdiv(ntiles_max, 8)).  This restates that
arithmetic on the CPU and requires every output element to be written
exactly once (a gap would leave garbage, a double write is wasted work),
and every K_rel row read to exist.
"""
from __future__ import annotations

import numpy as np
import pytest


def _cdiv(a, b):
    return -(-a // b)


def _walk(T, rows_used=None):
    """Write counts per output element; rows_used(i0, T) is the last query
    row a row group's tile range is sized for (the kernel: min(i0 + 127, T - 1))."""
    rows_used = rows_used or (lambda i0, T: min(i0 + 127, T - 1))
    count = np.zeros((T, T), np.int32)
    ntiles_max = (T - 1 + min(127, T - 1)) // 32 + 1
    for x in range(_cdiv(T, 128)):
        i0 = 128 * x
        ilast = rows_used(i0, T)
        rlo = T - 1 - ilast
        ntiles = (2 * T - 2 - i0 - rlo) // 32 + 1
        assert rlo >= 0
        for z in range(_cdiv(ntiles_max, 8)):
            t0, t1 = 8 * z, min(ntiles, 8 * z + 8)
            for w in range(4):
                iw = i0 + 32 * w
                if iw >= T:
                    continue
                w_rlo, w_rhi = T - 1 - min(iw + 31, T - 1), 2 * T - 2 - iw
                for t in range(t0, t1):
                    r0 = rlo + 32 * t
                    if r0 > w_rhi or r0 + 31 < w_rlo:
                        continue
                    ia = iw + np.arange(32)[:, None]
                    j = r0 + np.arange(32)[None, :] - (T - 1) + ia
                    ok = (ia < T) & (j >= 0) & (j < T)
                    np.add.at(count, (np.broadcast_to(ia, ok.shape)[ok], j[ok]), 1)
                    # Rows of K_rel the tile reads (clamped to 2T - 2 in the kernel):
                    # the unclamped ones that feed stored elements must exist.
                    used_r = (r0 + np.arange(32))[ok.any(axis=0)]
                    assert used_r.max(initial=0) <= 2 * T - 2
    return count


@pytest.mark.parametrize("T", [1, 2, 17, 31, 32, 33, 64, 100, 127, 128, 129, 255, 256, 448,
                               1000, 1500])
def test_every_element_written_once(T):
    assert (_walk(T) == 1).all()


def test_planted_row_range_mistake_fails():
    """Sizing the tile range for one 32-row block instead of the workgroup's
    128 rows (a plausible slip from the one-block-per-workgroup layout)
    leaves the later blocks' far positions unwritten."""
    assert not (_walk(300, rows_used=lambda i0, T: min(i0 + 31, T - 1)) == 1).all()

