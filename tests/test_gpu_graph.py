"""Launches captured in a HIP graph replay to the eager results.

The bench replays graphs of launches, and callers with launch-bound loops
capture them the same way.  Every entry point enqueues exactly one kernel
and records no memset, so each replay must reproduce the eager output bit
for bit.  Between replays the test runs other eager work on the same
buffers' stream and synchronises.
"""
from __future__ import annotations

import pytest
import torch

import neso_amd
from oracle import inputs as I
from oracle import qmatmul as Q

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _replays_match(launch, outputs, clobber):
    launch()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outputs]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    for rep in range(4):
        clobber()                      # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outputs, eager):
            assert torch.equal(o, e), f"replay {rep} differs"


def test_graph_fa2_and_relpos(gpu):
    q, k, v = (t.to(DEV) for t in I.fa2_inputs(1, 4, 300, 64, seed=21))
    o = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    rq, rk, rv, table = (t.to(DEV) for t in I.relpos_inputs(3, 200, 64, seed=22))
    ro = torch.empty(rq.shape, dtype=torch.float32, device=DEV)

    def launch():
        neso_amd.attention(q, k, v, causal=True, out=o)
        neso_amd.rel_pos_attention(rq, rk, rv, table, out=ro)

    def clobber():
        o.fill_(float("nan"))
        ro.fill_(-1.0)
        neso_amd.attention(k, q, v, out=torch.empty_like(o))

    _replays_match(launch, [o, ro], clobber)


@pytest.mark.parametrize("m", [1, 3, 40])
def test_graph_w4a16(gpu, m):
    x, codes, scales = I.qmatmul_inputs(m, 1024, 700, seed=23 + m)
    w = torch.from_numpy(Q.pack_int4(codes.numpy())).to(DEV)
    xs, ss = x.to(DEV), scales.to(DEV)
    y = torch.empty(m, 700, dtype=torch.float16, device=DEV)

    def launch():
        neso_amd.w4a16_matmul(xs, w, ss, y, m, 700, 1024, 1024, 700)

    def clobber():
        y.fill_(3.0)

    _replays_match(launch, [y], clobber)
