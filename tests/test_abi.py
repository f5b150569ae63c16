"""C-ABI checks that run without a GPU.

The library must load, export every function include/neso_amd.h declares
(and nothing the Python binding expects must be missing), publish a
manifest that agrees with the header, and reject invalid arguments with
NESO_EINVAL / NESO_EUNSUPPORTED before touching HIP (no compute call is
made here: each call either fails validation or is an empty no-op).
"""
from __future__ import annotations

import ctypes
import json
import re
import subprocess
from pathlib import Path

import pytest
import torch

import neso_amd
from neso_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "neso_amd.h"
A16 = 0x10000  # an aligned fake device address: never dereferenced here


def header_functions() -> dict[str, int]:
    """name -> parameter count for every function declared in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^[\w ]+?\*?\s*(neso_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_binding_agree():
    funcs = header_functions()
    assert funcs, "no declarations parsed from the header"
    assert set(funcs) == set(_lib.SIGNATURES)
    for name, n in funcs.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    for name in header_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None


def test_manifest_matches_header(lib):
    man = json.loads(lib.neso_kernel_manifest().decode())
    assert man["abi_version"] == lib.neso_abi_version() == 2
    funcs = header_functions()
    for k in man["kernels"]:
        # The reference's AOT metadata fields (src/neso/aot_compile.py:108-117).
        assert {"kernel_name", "params", "constants", "threadgroup_size", "num_warps",
                "grid"} <= set(k), k.get("kernel_name")
        assert k["kernel_name"] in funcs
        assert len(k["params"]) == funcs[k["kernel_name"]], k["kernel_name"]
        assert [p["index"] for p in k["params"]] == list(range(len(k["params"])))
        for v in k["variants"]:
            assert {"device_kernel", "template_params", "threadgroup_size", "num_warps",
                    "grid", "constants"} <= set(v)
            assert len(v["grid"]) == 3
    kernels = {k["kernel_name"] for k in man["kernels"]}
    assert kernels == {n for n in funcs if n.endswith(("_fwd", "_matmul", "_precompute"))}


def _cdiv(a, b):
    return -(-a // b)


def _eval(expr, env):
    """A manifest geometry expression (Python syntax, the manifest's own text)."""
    return eval(expr, {"__builtins__": {}}, {**env, "cdiv": _cdiv})


def _plan(lib, fn, args, cus):
    assert lib.neso_plan_begin(cus) == _lib.NESO_OK
    try:
        status = fn(*args)
    finally:
        plan = json.loads(lib.neso_plan_end().decode())
    return status, plan["launches"]


_P = A16
PLAN_CASES = [
    # (entry point, positional args, size variables)
    ("neso_flash_attention_fwd", [_P] * 4 + [2048, 64, 64, 0.125, 64, 16, 2048 * 64, 2048 * 64, 0],
     dict(N=2048, batch_heads=16)),
    ("neso_flash_attention_fwd", [_P] * 4 + [128, 64, 64, 0.125, 64, 8, 128 * 64, 128 * 64, 0],
     dict(N=128, batch_heads=8)),
    ("neso_flash_attention_fwd", [_P] * 4 + [1024, 64, 64, 0.125, 64, 16, 1024 * 64, 1024 * 64, 1],
     dict(N=1024, batch_heads=16)),
    ("neso_flash_attention_fwd", [_P] * 4 + [512, 64, 64, 0.125, 64, 16, 512 * 64, 512 * 64, 1],
     dict(N=512, batch_heads=16)),
    ("neso_flash_attention_fwd", [_P] * 4 + [4096, 128, 128, 0.08, 128, 8, 4096 * 128, 4096 * 128, 1],
     dict(N=4096, batch_heads=8)),
    ("neso_flash_attention_fwd", [_P] * 4 + [4096, 128, 128, 0.08, 128, 64, 4096 * 128, 4096 * 128, 1],
     dict(N=4096, batch_heads=64)),
    ("neso_flash_attention_fwd", [_P] * 4 + [2048, 64, 64, 0.125, 64, 4, 2048 * 64, 2048 * 64, 1],
     dict(N=2048, batch_heads=4)),
    ("neso_flash_attention_fwd", [_P] * 4 + [300, 32, 32, 0.17, 32, 3, 300 * 32, 300 * 32, 0],
     dict(N=300, batch_heads=3)),
    ("neso_flash_attention_fwd", [_P] * 4 + [1024, 128, 128, 0.08, 128, 16, 1024 * 128, 1024 * 128, 0],
     dict(N=1024, batch_heads=16)),
    ("neso_flash_attention_fwd", [_P] * 4 + [1500, 64, 64, 0.125, 64, 8, 1500 * 64, 1500 * 64, 0],
     dict(N=1500, batch_heads=8)),
    ("neso_flash_attention_f32_fwd", [_P] * 4 + [512, 128, 128, 0.08, 128, 2, 512 * 128, 512 * 128, 0],
     dict(N=512, batch_heads=2)),
    ("neso_flash_attention_f32_fwd", [_P] * 4 + [2048, 64, 64, 0.125, 64, 8, 2048 * 64, 2048 * 64, 1],
     dict(N=2048, batch_heads=8)),
    ("neso_flash_attention_io_fwd", [_P] * 4 + [1000, 128, 0.08, 0, 2], dict(N=1000, batch_heads=2)),
    ("neso_flash_attention_io_fwd", [_P] * 4 + [256, 64, 0.125, 1, 1], dict(N=256, batch_heads=1)),
    ("neso_flash_attention_window_fwd", [_P] * 4 + [400, 64, 192, 0.125, 5, 7, 3, 64, 1],
     dict(N=400, batch_heads=3)),
    ("neso_rel_pos_fa2_fwd", [_P] * 5 + [1500, 64, 0.125, 1500 * 64, 2999, 8, 64, 1, 1],
     dict(N=1500, batch_heads=8)),
    ("neso_rel_pos_fa2_fwd", [_P] * 5 + [64, 64, 0.125, 64 * 64, 64 * 64, 4, 64, 0, 0],
     dict(N=64, batch_heads=4)),
    ("neso_rel_pos_fa2_fwd", [_P] * 5 + [8192, 64, 0.125, 8192 * 64, 16383, 16, 64, 1, 1],
     dict(N=8192, batch_heads=16)),
    ("neso_rel_pos_precompute", [_P] * 4 + [1500, 64, 8, 0.125, _P, _P], dict(T=1500, nh=8)),
    ("neso_rel_pos_precompute", [_P] * 4 + [33, 128, 3, 0.1, _P, _P], dict(T=33, nh=3)),
    ("neso_rel_pos_precompute", [_P] * 4 + [10, 32, 2, 0.1, _P, _P], dict(T=10, nh=2)),
    ("neso_rel_pos_precompute", [_P] * 4 + [4096, 64, 1, 0.1, _P, _P], dict(T=4096, nh=1)),
    # X row stride 2^23: the tiled kernels' 32-bit buffer offsets would
    # overflow, so the fallback kernel is chosen.
    ("neso_w4a16_matmul", [_P] * 4 + [100, 11008, 4096, 1 << 23, 11008, 32, 8],
     dict(M=100, N=11008, K=4096)),
] + [
    ("neso_w4a16_matmul", [_P] * 4 + [m, 11008, k, k, 11008, g, 8], dict(M=m, N=11008, K=k))
    for m, k, g in ((1, 4096, 32), (2, 4096, 32), (1, 8192, 128), (3, 4096, 32), (16, 4096, 32),
                    (16, 5120, 32), (48, 4096, 64), (128, 4096, 32), (256, 4096, 32),
                    (1000, 4096, 32))
] + [
    ("neso_w8a16_matmul", [_P] * 3 + [4096, 4096, 4096, 4096, 4096, 4096],
     dict(M=4096, N=4096, K=4096)),
    ("neso_w8a16_scaled_matmul", [_P] * 4 + [100, 100, 100, 100, 64, 100],
     dict(M=64, N=100, K=100)),
]


@pytest.mark.parametrize("cus", [256, 80])
@pytest.mark.parametrize("case", range(len(PLAN_CASES)))
def test_manifest_geometry_matches_launches(lib, case, cus):
    """The launch each entry point chooses (recorded, not issued) is one of
    its manifest variants, with the threadgroup size, warp count and grid
    that the variant's formulas give for the call's sizes."""
    name, args, sizes = PLAN_CASES[case]
    man = {k["kernel_name"]: k for k in json.loads(lib.neso_kernel_manifest().decode())["kernels"]}
    status, launches = _plan(lib, getattr(lib, name), args + [None], cus)
    assert status == _lib.NESO_OK, lib.neso_last_error()
    assert len(launches) == 1, launches
    rec = launches[0]
    entry = man[name]
    variants = {v["device_kernel"]: v for v in entry["variants"]}
    assert rec["device_kernel"] in variants, (name, rec)
    v = variants[rec["device_kernel"]]
    assert len(v["template_params"]) == len(rec["template_args"])
    env = dict(zip(v["template_params"], rec["template_args"]), cus=cus, **sizes)
    assert _eval(v["threadgroup_size"], env) == rec["threadgroup_size"]
    assert _eval(v["num_warps"], env) == rec["num_warps"]
    assert [_eval(g, env) for g in v["grid"]] == rec["grid"], (v["grid"], rec)


# (entry point, args, expected kernel, expected template arguments by name)
CHOICE_CASES = [
    # 96 workgroups of 128 queries fill under half of 256
    # CUs, so the biased fast kernel runs 64-query workgroups, 4 key groups.
    ("neso_rel_pos_fa2_fwd", [_P] * 5 + [1500, 64, 0.125, 1500 * 64, 2999, 8, 64, 1, 1],
     "fa2_fast_kernel", dict(D=64, QW=2, KSPLIT=4, BIAS=2)),
    # A larger biased grid: 128-query workgroups.
    ("neso_rel_pos_fa2_fwd", [_P] * 5 + [8192, 64, 0.125, 8192 * 64, 16383, 16, 64, 1, 1],
     "fa2_fast_kernel", dict(QW=4, KSPLIT=1, BIAS=1)),
    # A scale whose reciprocal could overflow the band: generic kernel.
    ("neso_rel_pos_fa2_fwd", [_P] * 5 + [1500, 64, 1e-30, 1500 * 64, 2999, 8, 64, 1, 1],
     "fa2_fwd_kernel", dict(BIAS=1)),
    # The dense f16 bias has no fast kernel.
    ("neso_rel_pos_fa2_fwd", [_P] * 5 + [1500, 64, 0.125, 1500 * 64, 1500 * 1500, 8, 64, 0, 0],
     "fa2_fwd_kernel", dict(BIAS=2)),
    # The headline: 128-query workgroups, two key groups.
    ("neso_flash_attention_fwd", [_P] * 4 + [2048, 64, 64, 0.125, 64, 16, 2048 * 64, 2048 * 64, 0],
     "fa2_fast_kernel", dict(QW=4, KSPLIT=2, PAIR=0, HALVES=0, BIAS=0)),
    # Small grids from N = 512: two query waves; four key groups while the
    # 64-query workgroups fit the CUs and N >= 1024.
    ("neso_flash_attention_fwd", [_P] * 4 + [1500, 64, 64, 0.125, 64, 8, 1500 * 64, 1500 * 64, 0],
     "fa2_fast_kernel", dict(QW=2, KSPLIT=4)),
    ("neso_flash_attention_fwd", [_P] * 4 + [1024, 128, 128, 0.08, 128, 16, 1024 * 128, 1024 * 128, 0],
     "fa2_fast_kernel", dict(QW=2, KSPLIT=4)),
    ("neso_flash_attention_fwd", [_P] * 4 + [512, 64, 64, 0.125, 64, 8, 512 * 64, 512 * 64, 0],
     "fa2_fast_kernel", dict(QW=2, KSPLIT=2)),
    ("neso_flash_attention_fwd", [_P] * 4 + [2048, 64, 64, 0.125, 64, 4, 2048 * 64, 2048 * 64, 1],
     "fa2_fast_kernel", dict(QW=2, KSPLIT=4, CAUSAL=1, HALVES=0)),
    # Causal, one workgroup per CU: 64-row halves on four query waves.
    ("neso_flash_attention_fwd", [_P] * 4 + [2048, 64, 64, 0.125, 64, 16, 2048 * 64, 2048 * 64, 1],
     "fa2_fast_kernel", dict(QW=4, HALVES=1)),
    # head_dim 128, causal, one round of paired 64-row blocks from N = 2048:
    # paired blocks on two query waves with four key groups.
    ("neso_flash_attention_fwd", [_P] * 4 + [4096, 128, 128, 0.08, 128, 8, 4096 * 128, 4096 * 128, 1],
     "fa2_fast_kernel", dict(D=128, QW=2, KSPLIT=4, PAIR=1, HALVES=0)),
    ("neso_flash_attention_fwd", [_P] * 4 + [2048, 128, 128, 0.08, 128, 16, 2048 * 128, 2048 * 128, 1],
     "fa2_fast_kernel", dict(D=128, QW=2, KSPLIT=4, PAIR=1)),
    # Below N = 2048, or with more pairs than CUs: as before.
    ("neso_flash_attention_fwd", [_P] * 4 + [1024, 128, 128, 0.08, 128, 32, 1024 * 128, 1024 * 128, 1],
     "fa2_fast_kernel", dict(D=128, QW=4, HALVES=1)),
    ("neso_flash_attention_fwd", [_P] * 4 + [4096, 128, 128, 0.08, 128, 64, 4096 * 128, 4096 * 128, 1],
     "fa2_fast_kernel", dict(D=128, QW=4, PAIR=1)),
    # W8A16: 256 x 256 tiles once they give every CU a workgroup.
    ("neso_w8a16_matmul", [_P] * 3 + [4096, 4096, 4096, 4096, 4096, 4096],
     "w8a16_gemm_kernel", dict(T=256)),
    ("neso_w8a16_matmul", [_P] * 3 + [520, 520, 3000, 3000, 1000, 3000],
     "w8a16_gemm_kernel", dict(T=128)),
    # Short rows: the fast kernel with 128-query workgroups (N < 512).
    ("neso_flash_attention_fwd", [_P] * 4 + [128, 64, 64, 0.125, 64, 8, 128 * 64, 128 * 64, 0],
     "fa2_fast_kernel", dict(QW=4)),
]


@pytest.mark.parametrize("case", range(len(CHOICE_CASES)))
def test_fa2_kernel_choice(lib, case):
    """The launcher's kernel and workgroup shape for shapes whose choice was
    measured, on a 256-CU device."""
    name, args, kernel, want = CHOICE_CASES[case]
    man = {k["kernel_name"]: k for k in json.loads(lib.neso_kernel_manifest().decode())["kernels"]}
    status, launches = _plan(lib, getattr(lib, name), args + [None], 256)
    assert status == _lib.NESO_OK, lib.neso_last_error()
    (rec,) = launches
    assert rec["device_kernel"] == kernel, rec
    params = {v["device_kernel"]: v["template_params"] for v in man[name]["variants"]}[kernel]
    got = dict(zip(params, rec["template_args"]))
    assert {k: got[k] for k in want} == want, got


def test_plan_records_nothing_on_rejected_calls(lib):
    status, launches = _plan(lib, lib.neso_flash_attention_fwd,
                             [A16] * 4 + [128, 64, 64, 0.125, 96, 1, 0, 0, 0, None], 256)
    assert status == _lib.NESO_EUNSUPPORTED and launches == []
    assert lib.neso_plan_begin(-1) == _lib.NESO_EINVAL


def test_clock_sample_arguments(lib):
    """The clock sampler rejects bad buffers and counts before any HIP call,
    and launches exactly one 64-thread wave."""
    for args in ([None, 8, 100], [A16 + 4, 8, 100], [A16, 0, 100], [A16, 8, 0],
                 [A16, (1 << 20) + 1, 100], [A16, 8, (1 << 20) + 1], [A16, 1 << 20, 1025]):
        assert lib.neso_clock_sample(*args, None) == _lib.NESO_EINVAL, args
    status, launches = _plan(lib, lib.neso_clock_sample, [A16, 1 << 20, 1024, None], 256)
    assert status == _lib.NESO_OK
    assert [(k["device_kernel"], k["grid"], k["threadgroup_size"]) for k in launches] == [
        ("clock_sample_kernel", [1, 1, 1], 64)]


def test_stream_probe_arguments(lib):
    """The streaming-floor probe validates before any launch."""
    for args in ((A16, 1024, 0, 1), (A16, 1024, 1 << 21, 1), (A16, 1024, 4, 3), (None, 1024, 4, 2),
                 (A16 + 8, 1024, 4, 1), (A16, 1000, 4, 1), (A16, 0, 4, 1),
                 (A16, 16 * 16 * 256 * 4 + 16, 4, 1)):  # 17 pieces per thread
        assert lib.neso_stream_probe(args[0], args[1], args[2], args[3], 0, A16, None) \
            == _lib.NESO_EINVAL, args
    assert lib.neso_stream_probe(A16, 1024, 4, 1, 0, None, None) == _lib.NESO_EINVAL


def test_status_strings(lib):
    for code in (_lib.NESO_OK, _lib.NESO_EINVAL, _lib.NESO_EUNSUPPORTED, _lib.NESO_ELAUNCH):
        assert lib.neso_status_string(code).startswith(b"NESO_")


def fa2(lib, **kw):
    args = dict(Q=A16, K=A16, V=A16, O=A16, N=128, stride_qo=64, stride_kv=64, scale=0.125,
                head_dim=64, batch_heads=1, stride_bh_qo=0, stride_bh_kv=0, causal=0, stream=None)
    args.update(kw)
    return lib.neso_flash_attention_fwd(*args.values())


@pytest.mark.parametrize("kw,status", [
    (dict(Q=None), _lib.NESO_EINVAL),
    (dict(O=None), _lib.NESO_EINVAL),
    (dict(N=-1), _lib.NESO_EINVAL),
    (dict(head_dim=96, stride_qo=96, stride_kv=96), _lib.NESO_EUNSUPPORTED),
    (dict(stride_qo=32), _lib.NESO_EINVAL),
    (dict(stride_kv=68), _lib.NESO_EINVAL),
    (dict(K=A16 + 2), _lib.NESO_EINVAL),
    (dict(scale=float("nan")), _lib.NESO_EINVAL),
    (dict(causal=2), _lib.NESO_EINVAL),
    (dict(stride_bh_kv=12), _lib.NESO_EINVAL),
    (dict(N=0), _lib.NESO_OK),
    (dict(batch_heads=0), _lib.NESO_OK),
])
def test_fa2_validation(lib, kw, status):
    assert fa2(lib, **kw) == status
    if status != _lib.NESO_OK:
        assert lib.neso_last_error()


def fa2_f32(lib, **kw):
    args = dict(Q=A16, K=A16, V=A16, O=A16, N=0, stride_qo=64, stride_kv=64, scale=0.125,
                head_dim=64, batch_heads=1, stride_bh_qo=0, stride_bh_kv=0, causal=0, stream=None)
    args.update(kw)
    return lib.neso_flash_attention_f32_fwd(*args.values())


@pytest.mark.parametrize("kw,status", [
    (dict(head_dim=128, stride_qo=128, stride_kv=128), _lib.NESO_OK),
    (dict(head_dim=96, stride_qo=96, stride_kv=96), _lib.NESO_EUNSUPPORTED),
    (dict(stride_qo=66), _lib.NESO_EINVAL),          # f32 rows need multiples of 4
    (dict(stride_qo=68, stride_kv=68), _lib.NESO_OK),  # ... not of 8
    (dict(stride_bh_kv=6), _lib.NESO_EINVAL),
    (dict(V=A16 + 4), _lib.NESO_EINVAL),
    (dict(stride_qo=1 << 24), _lib.NESO_EUNSUPPORTED),  # 128-row block exceeds 32-bit offsets
    (dict(head_dim=32, stride_qo=32, stride_kv=32), _lib.NESO_OK),
])
def test_fa2_f32_validation(lib, kw, status):
    assert fa2_f32(lib, **kw) == status


def fa2_io(lib, **kw):
    args = dict(Q=A16, K=A16, V=A16, O=A16, N=0, d_head=64, scale=0.125, io_dtype=0,
                batch_heads=1, stream=None)
    args.update(kw)
    return lib.neso_flash_attention_io_fwd(*args.values())


@pytest.mark.parametrize("kw,status", [
    (dict(), _lib.NESO_OK),
    (dict(io_dtype=1), _lib.NESO_OK),
    (dict(io_dtype=2), _lib.NESO_EINVAL),
    (dict(O=None), _lib.NESO_EINVAL),
    (dict(d_head=96), _lib.NESO_EUNSUPPORTED),
    (dict(d_head=128, io_dtype=1), _lib.NESO_OK),
    (dict(O=A16 + 8), _lib.NESO_EINVAL),
    (dict(N=-3), _lib.NESO_EINVAL),
    (dict(batch_heads=-1), _lib.NESO_EINVAL),
])
def test_fa2_io_validation(lib, kw, status):
    assert fa2_io(lib, **kw) == status


def relpre(lib, **kw):
    args = dict(Q=A16, K_rel=A16, bias_u=A16, bias_v=A16, T=0, d=64, nh=1, scale=0.125,
                Q_u=A16, rel_bias=A16, stream=None)
    args.update(kw)
    return lib.neso_rel_pos_precompute(*args.values())


@pytest.mark.parametrize("kw,status", [
    (dict(), _lib.NESO_OK),
    (dict(Q=None), _lib.NESO_EINVAL),
    (dict(rel_bias=None), _lib.NESO_EINVAL),
    (dict(d=48), _lib.NESO_EUNSUPPORTED),
    (dict(T=-1), _lib.NESO_EINVAL),
    (dict(K_rel=A16 + 4), _lib.NESO_EINVAL),
    (dict(rel_bias=A16 + 2), _lib.NESO_OK),  # fp16 output: 2-byte alignment
    (dict(T=50000, nh=1), _lib.NESO_EUNSUPPORTED),  # T * T past 2^31
])
def test_relpos_precompute_validation(lib, kw, status):
    assert relpre(lib, **kw) == status


def relpos(lib, **kw):
    args = dict(Q=A16, K=A16, V=A16, bias=A16, O=A16, T=0, stride=64, scale=0.125, stride_h=0,
                bias_stride_h=0, num_heads=1, head_dim=64, bias_mode=1, out_dtype=1, stream=None)
    args.update(kw)
    return lib.neso_rel_pos_fa2_fwd(*args.values())


@pytest.mark.parametrize("kw,status", [
    (dict(bias=None), _lib.NESO_EINVAL),
    (dict(bias_mode=7), _lib.NESO_EINVAL),
    (dict(out_dtype=3), _lib.NESO_EINVAL),
    (dict(bias=A16 + 2), _lib.NESO_EINVAL),  # f32 table must be 4-byte aligned
    (dict(bias=A16 + 2, bias_mode=0), _lib.NESO_OK),
    (dict(head_dim=48, stride=48), _lib.NESO_EUNSUPPORTED),
    (dict(), _lib.NESO_OK),
])
def test_relpos_validation(lib, kw, status):
    assert relpos(lib, **kw) == status


def w4(lib, **kw):
    args = dict(X=A16, W=A16, S=A16, Y=A16, M=0, N=11008, K=4096, ldx=4096, ldy=11008,
                group=32, zero=8, stream=None)
    args.update(kw)
    return lib.neso_w4a16_matmul(*args.values())


@pytest.mark.parametrize("kw,status", [
    (dict(W=None), _lib.NESO_EINVAL),
    (dict(K=4100, ldx=4104), _lib.NESO_EINVAL),
    (dict(group=48), _lib.NESO_EINVAL),
    (dict(group=96), _lib.NESO_EINVAL),  # does not divide K=4096
    (dict(zero=16), _lib.NESO_EINVAL),
    (dict(zero=-1), _lib.NESO_EINVAL),
    (dict(ldx=4000), _lib.NESO_EINVAL),
    (dict(ldx=4100), _lib.NESO_EINVAL),
    (dict(ldy=100), _lib.NESO_EINVAL),
    (dict(X=A16 + 8), _lib.NESO_EINVAL),
    (dict(M=-1), _lib.NESO_EINVAL),
    (dict(), _lib.NESO_OK),
    (dict(group=128), _lib.NESO_OK),
])
def test_w4a16_validation(lib, kw, status):
    assert w4(lib, **kw) == status


@pytest.mark.parametrize("scaled", [False, True])
def test_w8a16_validation(lib, scaled):
    fn = lib.neso_w8a16_scaled_matmul if scaled else lib.neso_w8a16_matmul
    extra = [A16] if scaled else []
    good = [A16, A16, A16, *extra, 64, 64, 64, 64, 0, 64, None]
    assert fn(*good) == _lib.NESO_OK
    bad = list(good)
    bad[0] = None
    assert fn(*bad) == _lib.NESO_EINVAL
    bad = list(good)
    bad[-5] = 32  # stride_bk < N
    assert fn(*bad) == _lib.NESO_EINVAL
    if scaled:
        bad = list(good)
        bad[3] = None
        assert fn(*bad) == _lib.NESO_EINVAL
    # K = 0 with a non-empty output is rejected before any launch (the
    # kernel's B extent would otherwise be negative); with M = 0 it is a no-op.
    bad = list(good)
    bad[-7], bad[-3] = 0, 64  # K = 0, M = 64
    assert fn(*bad) == _lib.NESO_EINVAL
    assert b"K=0" in lib.neso_last_error()
    bad[-3] = 0
    assert fn(*bad) == _lib.NESO_OK


def test_qmatmul_4gib_extents_rejected(lib):
    """The int4 and W8A16 kernels address X / Y / A / B with 32-bit buffer
    offsets: a call whose byte extent reaches 2^32 is rejected before any
    launch (it would otherwise wrap and read zeros past the wrapped end).
    Extents just below the limit pass validation (M = 0: no launch)."""
    # int4: X spans (M-1) * ldx + K halves; 2^31 halves is 4 GiB.
    m = (1 << 31) // 4096 + 1
    assert w4(lib, M=m, ldx=4096, ldy=11008) == _lib.NESO_EINVAL
    assert b"4 GiB" in lib.neso_last_error()
    assert w4(lib, M=2, ldx=(1 << 31) - 8) == _lib.NESO_EINVAL
    assert w4(lib, M=2, N=64, ldy=(1 << 31) - 1, ldx=4096) == _lib.NESO_EINVAL
    assert w4(lib, M=0, ldx=(1 << 31) - 8) == _lib.NESO_OK
    for scaled in (False, True):
        fn = lib.neso_w8a16_scaled_matmul if scaled else lib.neso_w8a16_matmul
        extra = [A16] if scaled else []
        # B int8 [K][N]: (K - 1) * ldb + N bytes; ldb = 2^23 with K = 513 is 4 GiB + N.
        args = [A16, A16, A16, *extra, 513, 513, 1 << 23, 64, 64, 64, None]
        assert fn(*args) == _lib.NESO_EINVAL
        assert b"4 GiB" in lib.neso_last_error()
        # A fp16 [M][K]: 2^31 halves.
        args = [A16, A16, A16, *extra, 64, 1 << 26, 64, 64, 33, 64, None]
        assert fn(*args) == _lib.NESO_EINVAL


def test_python_wrappers_raise():
    with pytest.raises(ValueError, match="no CPU path"):
        neso_amd.attention(*(torch.zeros(1, 1, 8, 64, dtype=torch.float16) for _ in range(3)))
    with pytest.raises(neso_amd.NesoArgumentError):
        neso_amd.flash_attention_fwd(A16, A16, A16, A16, 128, 64, 64, 0.125, head_dim=80)
    with pytest.raises(ValueError):
        neso_amd.flash_attention_fwd(A16, A16, A16, A16, -5, 64, 64, 0.125, head_dim=64)
    with pytest.raises(ValueError, match="unknown kernel"):
        neso_amd.launch("vector_add")
    with pytest.raises(TypeError):
        neso_amd.w4a16_matmul("x", A16, A16, A16, 1, 1, 32, 32, 1)
    err = neso_amd.NesoArgumentError(1, "x")
    assert isinstance(err, RuntimeError) and isinstance(err, ValueError)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libneso_amd.so")
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.load()


def test_ctypes_signatures_are_c_types():
    for name, (res, args) in _lib.SIGNATURES.items():
        for a in args:
            assert issubclass(a, ctypes._SimpleCData), (name, a)


def test_tensor_wrappers_validate_before_launch():
    """Shape, dtype and extent errors raise ValueError before the ABI is called
    (CPU tensors here: the shape message must come first, not "no CPU path")."""
    f16 = torch.float16
    x = torch.zeros(2, 64, dtype=f16)
    w = torch.zeros(16, 8, dtype=torch.int32)
    s = torch.zeros(16, 2, dtype=f16)
    neso_amd_err = "w_packed must be"
    with pytest.raises(ValueError, match=neso_amd_err):
        neso_amd.w4a16_linear(x, torch.zeros(16, 4, dtype=torch.int32), s)
    with pytest.raises(ValueError, match="scales must be"):
        # scales made for group 128 passed with the default group 32
        neso_amd.w4a16_linear(x, w, torch.zeros(16, 1, dtype=f16))
    with pytest.raises(ValueError, match="group_size"):
        neso_amd.w4a16_linear(x, w, s, group_size=48)
    with pytest.raises(ValueError, match="out must be"):
        neso_amd.w4a16_linear(x, w, s, out=torch.zeros(2, 8, dtype=f16))
    q = torch.zeros(2, 16, 64, dtype=f16)
    table = torch.zeros(2, 31, dtype=torch.float32)
    with pytest.raises(ValueError, match="must match q"):
        neso_amd.rel_pos_attention(q, torch.zeros(2, 8, 64, dtype=f16), q, table)
    with pytest.raises(ValueError, match="table must be"):
        neso_amd.rel_pos_attention(q, q, q, torch.zeros(2, 30, dtype=torch.float32))
    with pytest.raises(ValueError, match="fp32"):
        neso_amd.rel_pos_attention(q, q, q, table.double())
    with pytest.raises(ValueError, match="out must be"):
        neso_amd.attention(q, q, q, out=torch.zeros(2, 16, 64, dtype=f16))
    # Reference-order launchers: a tensor shorter than the declared extent.
    with pytest.raises(ValueError, match="span"):
        neso_amd.flash_attention_fwd(q, q, q, torch.zeros(2, 16, 64), 16, 64, 64, 0.125,
                                     batch_heads=3, stride_bh_qo=1024, stride_bh_kv=1024)
    with pytest.raises(ValueError, match="span"):
        neso_amd.w4a16_matmul(x, w, s, torch.zeros(1, 16, dtype=f16), 2, 16, 64, 64, 16)
    with pytest.raises(ValueError, match="span"):
        neso_amd.w8a16_matmul(x, torch.zeros(64, 8, dtype=torch.int8),
                              torch.zeros(2, 16), 64, 64, 16, 16, M=2, N=16)
    with pytest.raises(ValueError, match="span"):
        neso_amd.rel_pos_fa2_fwd(q, q, q, torch.zeros(2, 16, 15, dtype=f16), q, 16, 64, 0.125,
                                 1024, 256, num_heads=2)


def test_python_manifest_and_plan():
    man = neso_amd.manifest()
    assert {k["kernel_name"] for k in man["kernels"]} >= {"neso_flash_attention_fwd",
                                                          "neso_w4a16_matmul"}
    plan = neso_amd.launch_plan("w4a16_matmul", A16, A16, A16, A16, 1, 11008, 4096, 4096, 11008,
                                cu_count=256)
    assert [p["device_kernel"] for p in plan] == ["w4a16_gemv_kernel"]
