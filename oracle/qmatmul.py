"""CPU restatement of the weight-only quantised matmuls (test infrastructure only).

W8A16: tests/test_quantized_matmul.py:288-311 (f64 triple-loop references of
``w8a16_matmul``, ``w4a16`` stored as i8, and ``w8a16_scaled_matmul`` with
the per-channel scale applied after accumulation, :250-260).

W4A16 int4/group format (no reference kernel packs int4 -
tests/test_quantized_matmul.py:170-178 keeps one value per int8):
code(n, k) = nibble (k % 8) of W[n, k // 8], low nibble first;
dequant = (code - zero) * S[n, k // group]; Y = X dequant(W)^T.
"""
from __future__ import annotations

import numpy as np


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """uint8 codes [N, K] in [0, 15] -> int32 words [N, K/8], low nibble first."""
    c = np.asarray(codes, dtype=np.uint32)
    n, k = c.shape
    assert k % 8 == 0
    c = c.reshape(n, k // 8, 8)
    words = np.zeros((n, k // 8), np.uint32)
    for e in range(8):
        words |= c[:, :, e] << np.uint32(4 * e)
    return words.view(np.int32)


def unpack_int4(words: np.ndarray) -> np.ndarray:
    """int32 words [N, K/8] -> uint8 codes [N, K]."""
    w = np.ascontiguousarray(words).view(np.uint32)
    n, kw = w.shape
    out = np.empty((n, kw, 8), np.uint8)
    for e in range(8):
        out[:, :, e] = (w >> np.uint32(4 * e)) & np.uint32(0xF)
    return out.reshape(n, kw * 8)


def dequant_int4(words: np.ndarray, scales: np.ndarray, group: int = 32, zero: int = 8,
                 dtype=np.float64) -> np.ndarray:
    """Dense dequantised weights [N, K]: (code - zero) * scale[n, k // group]."""
    codes = unpack_int4(words).astype(dtype)
    s = np.asarray(scales).astype(dtype)
    s_full = np.repeat(s, group, axis=1)
    return (codes - zero) * s_full


def w4a16_matmul(x: np.ndarray, words: np.ndarray, scales: np.ndarray, group: int = 32,
                 zero: int = 8, dtype=np.float64) -> np.ndarray:
    """Y[M, N] = X[M, K] dequant(W)^T accumulated in ``dtype`` (float64 by default).

    X is taken at its given precision (fp16 values upcast exactly).  The
    kernel's fp16 output rounding is left to the caller.
    """
    w = dequant_int4(words, scales, group, zero, dtype)
    return np.asarray(x).astype(dtype) @ w.T


def w8a16_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C = A @ f16(B) with B int8 [K, N], f64 accumulation (tests/test_quantized_matmul.py:288-297)."""
    return np.asarray(a, np.float64) @ np.asarray(b, np.float64)


def w8a16_scaled_matmul(a: np.ndarray, b: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """C = (A @ f16(B)) * scale[n] (tests/test_quantized_matmul.py:306-311)."""
    return w8a16_matmul(a, b) * np.asarray(scale, np.float64)[None, :]


def rel_err(out: np.ndarray, ref: np.ndarray) -> float:
    """max|out - ref| / max|ref| (tests/test_quantized_matmul.py:354-358)."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    den = float(np.max(np.abs(ref))) if ref.size else 0.0
    num = float(np.max(np.abs(out - ref))) if ref.size else 0.0
    return num / (den or 1.0)


def algorithmic_bytes(m: int, n: int, k: int, group: int = 32) -> int:
    """HBM bytes of one W4A16 call: packed W + scales + X + Y (BASELINE formula)."""
    return k * n // 2 + (k // group) * n * 2 + m * k * 2 + m * n * 2


def flops(m: int, n: int, k: int) -> float:
    return 2.0 * m * n * k
