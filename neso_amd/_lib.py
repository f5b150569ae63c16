"""ctypes binding of ``libneso_amd.so`` (the C ABI declared in include/neso_amd.h).

There is no fallback: if the shared library is missing or does not export an
entry point, loading raises.  ``import torch`` happens first so that torch's
HIP runtime (same soname, libamdhip64.so.7) is the one the library binds to,
which keeps torch streams and the library's launches in one runtime.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library shares)

LIB_PATH = Path(__file__).resolve().parent / "libneso_amd.so"
SERIAL_LIB_PATH = Path(__file__).resolve().parent / "libneso_amd_serial.so"

NESO_OK = 0
NESO_EINVAL = 1
NESO_EUNSUPPORTED = 2
NESO_ELAUNCH = 3

NESO_BIAS_DENSE_SCALED_F16 = 0
NESO_BIAS_TABLE_F32 = 1
NESO_OUT_F16 = 0
NESO_OUT_F32 = 1
NESO_IO_F16 = 0
NESO_IO_F32 = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/neso_amd.h line by line.
SIGNATURES = {
    "neso_abi_version": (ctypes.c_int, []),
    "neso_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "neso_last_error": (ctypes.c_char_p, []),
    "neso_kernel_manifest": (ctypes.c_char_p, []),
    "neso_plan_begin": (ctypes.c_int, [_i32]),
    "neso_plan_end": (ctypes.c_char_p, []),
    "neso_clock_sample": (ctypes.c_int, [_p, _i32, _i32, _p]),
    "neso_stream_probe": (ctypes.c_int, [_p, _i64, _i32, _i32, ctypes.c_uint32, _p, _p]),
    "neso_flash_attention_fwd": (
        ctypes.c_int,
        [_p, _p, _p, _p, _i32, _i32, _i32, _f32, _i32, _i32, _i64, _i64, _i32, _p],
    ),
    "neso_flash_attention_f32_fwd": (
        ctypes.c_int,
        [_p, _p, _p, _p, _i32, _i32, _i32, _f32, _i32, _i32, _i64, _i64, _i32, _p],
    ),
    "neso_flash_attention_io_fwd": (
        ctypes.c_int,
        [_p, _p, _p, _p, _i32, _i32, _f32, _i32, _i32, _p],
    ),
    "neso_flash_attention_window_fwd": (
        ctypes.c_int,
        [_p, _p, _p, _p, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _i32, _i32, _p],
    ),
    "neso_rel_pos_fa2_fwd": (
        ctypes.c_int,
        [_p, _p, _p, _p, _p, _i32, _i32, _f32, _i32, _i32, _i32, _i32, _i32, _i32, _p],
    ),
    "neso_rel_pos_precompute": (
        ctypes.c_int,
        [_p, _p, _p, _p, _i32, _i32, _i32, _f32, _p, _p, _p],
    ),
    "neso_w4a16_matmul": (
        ctypes.c_int,
        [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p],
    ),
    "neso_w8a16_matmul": (
        ctypes.c_int,
        [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p],
    ),
    "neso_w8a16_scaled_matmul": (
        ctypes.c_int,
        [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NesoError(RuntimeError):
    """A C-ABI call returned a non-OK status."""

    def __init__(self, status: int, detail: str):
        self.status = status
        super().__init__(detail)


class NesoArgumentError(NesoError, ValueError):
    """NESO_EINVAL / NESO_EUNSUPPORTED: the arguments were rejected before launch."""


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is missing or incomplete."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m neso_amd.build` "
                "(there is no CPU fallback)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if the symbol is not exported
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def load_variant(path: Path) -> ctypes.CDLL:
    """Load another build of the library (e.g. libneso_amd_serial.so, the
    debug build whose fast FA2 kernel serialises every LDS phase) with the
    same signatures; for tests that compare builds."""
    if not Path(path).exists():
        raise ImportError(f"{path} is missing: build it with `python -m neso_amd.build`")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def check(status: int) -> None:
    """Raise the Python exception that matches a non-OK status."""
    if status == NESO_OK:
        return
    lib = load()
    detail = (lib.neso_last_error() or b"").decode() or lib.neso_status_string(status).decode()
    if status in (NESO_EINVAL, NESO_EUNSUPPORTED):
        raise NesoArgumentError(status, detail)
    raise NesoError(status, detail)
