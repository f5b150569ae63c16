"""Build recipe of the HIP library ``neso_amd/libneso_amd.so`` (gfx950 only).

Each ``csrc/*.hip`` translation unit is compiled by ``hipcc`` to an object in
``neso_amd/_build/`` and the objects are linked into one shared library next
to this file, which is what :mod:`neso_amd._lib` loads with ctypes.

Run ``python -m neso_amd.build`` (or ``__graft_entry__.build()``).  It
cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD_DIR = PKG / "_build"
LIB_PATH = PKG / "libneso_amd.so"
ARCH = "gfx950"

SOURCES = ["neso_abi.hip", "fa2_fwd.hip", "fa2_fast.hip", "relpos_pre.hip", "qmatmul.hip",
           "qmatmul_skinny.hip"]

# Per-source options on top of COMMON_FLAGS.  The skinny int4 kernel runs
# 3-4% faster without the scheduler's memory-operation clustering (M = 16:
# 9.25 -> 8.92 us); the GEMV in qmatmul.hip does not gain from it.
SOURCE_FLAGS = {"qmatmul_skinny.hip": ["-mllvm", "-misched-cluster=0"]}

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed FP32 (v_pk_*_f32) stays off: the compiler would otherwise form
    # it from ordinary float code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the softmax reads S and rescales O with
    # ordinary VALU ops, so AGPR placement would add v_accvgpr copies.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the neso_amd HIP library cannot be built")
    return exe


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    # The host pass warns that it does not know the packed-fp32 feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    lines = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if any(ln.strip() for ln in lines):
        sys.stderr.write("\n".join(lines) + "\n")


def build(extra_flags: list[str] | None = None, jobs: int | None = None) -> Path:
    """Compile every translation unit and link ``libneso_amd.so``; return its path."""
    extra = list(extra_flags or [])
    BUILD_DIR.mkdir(exist_ok=True)
    objs = [BUILD_DIR / (Path(s).stem + ".o") for s in SOURCES]
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, CSRC / s, o, extra + SOURCE_FLAGS.get(s, []))
                for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
