"""Build recipe of the HIP library ``neso_amd/libneso_amd.so`` (gfx950 only).

Each ``csrc/*.hip`` translation unit is compiled by ``hipcc`` to an object in
``neso_amd/_build/`` and the objects are linked into one shared library next
to this file, which is what :mod:`neso_amd._lib` loads with ctypes.

Run ``python -m neso_amd.build`` (or ``__graft_entry__.build()``).  It
cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD_DIR = PKG / "_build"
LIB_PATH = PKG / "libneso_amd.so"
SERIAL_LIB_PATH = PKG / "libneso_amd_serial.so"
HARNESS_SRC = PKG / "harness" / "neso_harness.cpp"
HARNESS_PATH = PKG / "neso_harness"
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


# The hipcc on which the fast FA2 kernel's LDS-DMA inline asm (M0 written
# behind the compiler's back, fa2_tiles.h: lds_dma16) was last verified on
# the GPU.  Every build also checks the property itself in the generated
# assembly (m0_check); a different version only adds a note.
VERIFIED_HIPCC = "7.2.26015"

# Opcodes that read or write M0 without naming it (GFX9 family): relative
# moves, messages, GWS, append/consume, thread-indexed LDS access and
# LDS-DMA loads.
_M0_IMPLICIT = ("movrel", "s_sendmsg", "ds_gws", "ds_append", "ds_consume", "ds_ordered_count",
                "_addtid", "global_load_lds", "s_ttracedata")


def m0_check(asm: str) -> list[str]:
    """Problems with M0 use in a device assembly listing (empty: none).

    The only instructions allowed to touch M0 are the kernels' own LDS-DMA
    sequences: an inline-asm block of exactly ``s_mov_b32 m0, sN``,
    ``s_nop 0``, ``buffer_load_dwordx4 vN, s[..], 0 offen lds``.  Anything
    else that names M0 or uses it implicitly, inside or outside such a
    block, is reported.
    """
    import re
    problems = []
    lines = [ln.split(";", 1)[0].strip() if not ln.strip().startswith(";;#ASM") else ln.strip()
             for ln in asm.splitlines()]
    i = 0
    while i < len(lines):
        ln = lines[i]
        if ln == ";;#ASMSTART":
            j = i + 1
            body = []
            while j < len(lines) and lines[j] != ";;#ASMEND":
                if lines[j]:
                    body.append(lines[j])
                j += 1
            if any(re.search(r"\bm0\b", b) or " lds" in b for b in body):
                ok = (len(body) == 3 and re.fullmatch(r"s_mov_b32 m0, s\d+", body[0])
                      and body[1] == "s_nop 0"
                      and re.fullmatch(r"buffer_load_dwordx4 v\d+, s\[\d+:\d+\], 0 offen lds",
                                       body[2]))
                if not ok:
                    problems.append("unexpected inline-asm block: " + " | ".join(body))
            i = j + 1
            continue
        if ln and not ln.startswith((".", ";")) and not ln.endswith(":"):
            op = ln.split()[0]
            if re.search(r"\bm0\b", ln) or any(t in op for t in _M0_IMPLICIT) or ln.endswith(" lds"):
                problems.append("compiler-generated M0 use: " + ln)
        i += 1
    return problems


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the neso_amd HIP library cannot be built")
    return exe


_DIAG = re.compile(r"^(?:\S+:\d+:\d+: )?(warning|error|note): ")
_INCLUDED = "In file included from"


def _filter_diagnostics(text: str) -> tuple[list[str], int]:
    """Split compiler output into diagnostic blocks and drop the expected ones.

    Dropped: the host pass's warning that it does not know the packed-fp32
    feature, and the "clobber list contains reserved registers: m0" warning
    of the LDS-DMA asm, which the M0 check of the device assembly covers
    (returned as a count).  Returns (kept blocks, M0 warnings dropped).
    """
    blocks: list[list[str]] = []
    cur: list[str] = []
    for ln in text.splitlines():
        if re.match(r"^\d+ warnings? generated", ln):
            continue
        m = _DIAG.match(ln)
        after_include = bool(cur) and cur[-1].startswith(_INCLUDED)
        starts = ((ln.startswith(_INCLUDED) or (m and m.group(1) != "note")) and not after_include)
        if starts and cur:
            blocks.append(cur)
            cur = []
        cur.append(ln)
    if cur:
        blocks.append(cur)
    kept, m0 = [], 0
    for b in blocks:
        t = "\n".join(b)
        if "'-packed-fp32-ops' is not a recognized feature" in t:
            continue
        if "clobber list contains reserved registers: m0" in t:
            m0 += 1
            continue
        if t.strip():
            kept.append(t)
    return kept, m0


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    kept, m0 = _filter_diagnostics(res.stdout + res.stderr)
    if kept:
        sys.stderr.write("\n".join(kept) + "\n")
    if m0:
        sys.stderr.write(f"neso_amd build: {src.name}: {m0} expected warnings that the LDS-DMA asm "
                         f"clobbers the reserved M0 register (the M0 check of the assembly covers them)\n")


def _device_asm(src: Path, extra: list[str]) -> str:
    tag = "_serial" if "-DNESO_FA2_SERIAL_LDS" in extra else ""
    out = BUILD_DIR / (src.stem + tag + ".gfx950.s")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "--offload-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src.name}:\n{res.stdout}{res.stderr}")
    text = out.read_text()
    out.unlink()
    return text


def _link(objs: list[Path], path: Path) -> None:
    tmp = path.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, path)


def hipcc_version() -> str:
    res = subprocess.run([hipcc(), "--version"], capture_output=True, text=True)
    for ln in res.stdout.splitlines():
        if ln.startswith("HIP version:"):
            return ln.split(":", 1)[1].strip()
    return "unknown"


def build(extra_flags: list[str] | None = None, jobs: int | None = None) -> Path:
    """Compile every translation unit and link ``libneso_amd.so``; return its path.

    Also links ``libneso_amd_serial.so``, the same library whose fast FA2
    kernel ends every LDS phase in a full wait and barrier
    (NESO_FA2_SERIAL_LDS), which the GPU tests compare bit for bit with the
    pipelined build.  The fast kernel's LDS-DMA asm is checked in the
    generated assembly; if the check fails, both libraries are built without
    the fast kernel (NESO_FA2_FAST_DISABLED) and a warning is printed.
    """
    extra = list(extra_flags or [])
    BUILD_DIR.mkdir(exist_ok=True)
    objs = [BUILD_DIR / (Path(s).stem + ".o") for s in SOURCES]
    serial_obj = BUILD_DIR / "fa2_fast_serial.o"
    jobs = jobs or min(len(SOURCES) + 2, os.cpu_count() or 1)
    fast_flags = extra + SOURCE_FLAGS.get("fa2_fast.hip", [])
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        # Both builds of the fast kernel are checked: the serialised one
        # carries the same LDS-DMA asm.
        asm = ex.submit(_device_asm, CSRC / "fa2_fast.hip", fast_flags)
        asm_serial = ex.submit(_device_asm, CSRC / "fa2_fast.hip",
                               fast_flags + ["-DNESO_FA2_SERIAL_LDS"])
        futs = [ex.submit(_compile, CSRC / s, o, extra + SOURCE_FLAGS.get(s, []))
                for s, o in zip(SOURCES, objs)]
        futs.append(ex.submit(_compile, CSRC / "fa2_fast.hip", serial_obj,
                              extra + ["-DNESO_FA2_SERIAL_LDS"]))
        for f in futs:
            f.result()
        problems = m0_check(asm.result()) + m0_check(asm_serial.result())
    if problems:
        sys.stderr.write("neso_amd build: the fast FA2 kernel's LDS-DMA M0 assumption does not "
                         "hold for this compiler; building without the fast kernel:\n  "
                         + "\n  ".join(problems[:10]) + "\n")
        fast = CSRC / "fa2_fast.hip"
        _compile(fast, objs[SOURCES.index("fa2_fast.hip")], extra + ["-DNESO_FA2_FAST_DISABLED"])
        _compile(fast, serial_obj, extra + ["-DNESO_FA2_FAST_DISABLED"])
    ver = hipcc_version()
    if not ver.startswith(VERIFIED_HIPCC):
        sys.stderr.write(f"neso_amd build: hipcc {ver}; the fast FA2 kernel was last verified on "
                         f"the GPU with {VERIFIED_HIPCC} (its assembly check passed: "
                         f"{not problems})\n")
    _link(objs, LIB_PATH)
    _link([serial_obj if s == "fa2_fast.hip" else o for s, o in zip(SOURCES, objs)],
          SERIAL_LIB_PATH)
    build_harness()
    return LIB_PATH


def build_harness() -> Path:
    """The native C++ harness (known answers and a timing sweep through the
    C ABI, no Python), linked against the library beside it."""
    cmd = [hipcc(), "-O2", "-std=c++17", "-Wall", f"-I{PKG.parent / 'include'}",
           str(HARNESS_SRC), f"-L{PKG}", "-lneso_amd", "-Wl,-rpath,$ORIGIN",
           "-o", str(HARNESS_PATH)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"harness build failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    kept, _ = _filter_diagnostics(res.stdout + res.stderr)
    if kept:
        sys.stderr.write("\n".join(kept) + "\n")
    return HARNESS_PATH


if __name__ == "__main__":
    print(build())
