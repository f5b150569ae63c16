"""The native C++ harness (neso_amd/harness/neso_harness.cpp) on the GPU:
the C ABI driven with no Python in the process, the role of the
reference's kernel harness (macos/harness.rs:201-366).

`test` runs closed-form known answers through the C entry points (FA2 with
Q = K = 0 gives the column mean of V at tolerance 2e-3, the reference
harness's own check; int4 one-hot X gives (code - 8) * scale exactly; a
rejected head_dim sets NESO_EUNSUPPORTED).  `bench` runs the reference
harness's N sweep with a median of 20 HIP-event-timed launches.
"""
from __future__ import annotations

import re
import subprocess

import pytest

from neso_amd import build as B

pytestmark = pytest.mark.gpu


def _run(mode):
    if not B.HARNESS_PATH.exists():
        pytest.fail("neso_harness is not built (run __graft_entry__.build())")
    return subprocess.run([str(B.HARNESS_PATH), mode], capture_output=True, text=True,
                          timeout=120)


def test_harness_known_answers(gpu):
    r = _run("test")
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASSED" in r.stdout
    assert r.stdout.count("PASS ") == 6


def test_harness_bench_sweep(gpu):
    r = _run("bench")
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    rates = re.findall(r"N=\s*(\d+) d=64 heads=\s*(\d+)\s+([\d.]+) ms\s+([\d.]+) GFLOP/s", r.stdout)
    assert [(int(n), int(h)) for n, h, _, _ in rates] == [
        (128, 1), (256, 1), (512, 1), (1024, 1), (2048, 1), (2048, 16)]
    assert all(float(ms) > 0 for _, _, ms, _ in rates)
