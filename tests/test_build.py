"""Build-time guards that run without a GPU.

The fast FA2 kernel loads K/V tiles with inline-asm LDS-DMA instructions
that set M0 behind the compiler's back (neso_amd/csrc/fa2_tiles.h,
lds_dma16).  neso_amd/build.py checks every build's generated assembly so
that no compiler-generated instruction uses M0 in that translation unit;
these tests pin the checker itself with planted listings, and check that
the debug build (every LDS phase serialised) exports the same entry points.
"""
from __future__ import annotations

import subprocess

from neso_amd import _lib
from neso_amd import build as B

OURS = (";;#ASMSTART\n\ts_mov_b32 m0, s2\n\ts_nop 0\n"
        "\tbuffer_load_dwordx4 v178, s[92:95], 0 offen lds\n;;#ASMEND\n")


def test_m0_check_accepts_the_dma_sequence():
    asm = "kernel:\n\tv_add_f32 v1, v2, v3\n" + OURS * 3 + "\ts_endpgm\n"
    assert B.m0_check(asm) == []


def test_m0_check_rejects_compiler_m0_use():
    for bad in ("\ts_mov_b32 m0, -1\n",                          # compiler writes M0
                "\tv_movrels_b32 v1, v2\n",                      # implicit M0 read
                "\ts_sendmsg sendmsg(MSG_INTERRUPT)\n",
                "\tds_append v1\n",
                "\tbuffer_load_dword v1, s[4:7], 0 offen lds\n",  # compiler-made LDS-DMA
                "\tv_readlane_b32 s0, v1, m0\n"):
        assert B.m0_check(OURS + bad), bad


def test_m0_check_rejects_altered_asm_block():
    altered = OURS.replace("\ts_nop 0\n", "")                   # missing wait state
    assert B.m0_check(altered)
    extra = OURS.replace("\ts_nop 0\n", "\ts_nop 0\n\ts_add_u32 s2, s2, 4\n")
    assert B.m0_check(extra)


def test_serial_build_exports_every_entry_point():
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.SERIAL_LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    assert set(_lib.SIGNATURES) <= exported
    lib = _lib.load_variant(_lib.SERIAL_LIB_PATH)
    assert lib.neso_abi_version() == _lib.load().neso_abi_version()


def test_build_output_filter_drops_only_expected_warnings():
    """The M0-clobber warnings of the LDS-DMA asm are counted, not printed
    (the assembly check above covers them); other diagnostics stay."""
    text = "\n".join([
        "In file included from a/fa2_fast.hip:37:",
        "a/fa2_tiles.h:117:7: warning: inline asm clobber list contains reserved registers: m0"
        " [-Winline-asm]",
        "  117 |       \"s_mov_b32 m0, %0\\n\\t\"",
        "      |       ^",
        "a/fa2_tiles.h:117:7: note: Reserved registers on the clobber list may not be preserved",
        "a/qmatmul.hip:10:3: warning: unused variable 'x' [-Wunused-variable]",
        "   10 |   int x;",
        "warning: feature flag '-packed-fp32-ops' is not a recognized feature for this target",
        "2 warnings generated when compiling for gfx950.",
    ])
    kept, m0 = B._filter_diagnostics(text)
    assert m0 == 1
    assert len(kept) == 1 and "unused variable" in kept[0]


def test_harness_usage_without_gpu():
    """The native harness loads the library and answers usage errors
    without touching a GPU (exit status 2)."""
    import pytest
    if not B.HARNESS_PATH.exists():
        pytest.skip("neso_harness not built")
    r = subprocess.run([str(B.HARNESS_PATH)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
