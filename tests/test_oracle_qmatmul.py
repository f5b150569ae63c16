"""Pins the quantised-matmul oracle (oracle/qmatmul.py) on the CPU.

Checks: the reference tests' seeded vectors and f64 triple-loop results
(golden fixtures), a hand-made int4 known-answer fixture whose one-hot
activations read single codes (pins nibble order and scale indexing),
closed forms (all codes = zero point -> 0; constant codes), a brute-force
pure-Python evaluation on tiny shapes, linearity, and planted mistakes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import neso_amd.packing as P
from oracle import inputs as I
from oracle import qmatmul as Q


def test_pack_unpack_known_words():
    words = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32).view(np.int32)
    codes = Q.unpack_int4(words)
    assert codes.tolist() == [list(range(16))]
    assert np.array_equal(Q.pack_int4(codes), words)


def test_pack_roundtrip_random():
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, size=(13, 96), dtype=np.uint8)
    assert np.array_equal(Q.unpack_int4(Q.pack_int4(codes)), codes)


def test_host_packing_matches_oracle():
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, size=(7, 64), dtype=np.uint8)
    t = P.pack_int4(torch.from_numpy(codes))
    assert t.dtype == torch.int32
    assert np.array_equal(t.numpy(), Q.pack_int4(codes))
    assert np.array_equal(P.unpack_int4(t).numpy(), codes)


def test_int4_kat_fixture(golden_dir):
    z = np.load(golden_dir / "qmm_int4_kat.npz")
    assert np.array_equal(Q.unpack_int4(z["words"]), z["codes"])
    y = Q.w4a16_matmul(z["x"], z["words"], z["scales"], int(z["group"]), int(z["zero"]))
    assert np.array_equal(y, z["expected"])


def _brute(x, words, scales, group, zero):
    m, k = x.shape
    n = words.shape[0]
    w = words.view(np.uint32)
    y = np.zeros((m, n))
    for mm in range(m):
        for nn in range(n):
            acc = 0.0
            for kk in range(k):
                code = (int(w[nn, kk // 8]) >> (4 * (kk % 8))) & 0xF
                acc += float(x[mm, kk]) * (code - zero) * float(scales[nn, kk // group])
            y[mm, nn] = acc
    return y


@pytest.mark.parametrize("group,zero", [(32, 8), (64, 7), (32, 0)])
def test_matches_brute_force(group, zero):
    x, codes, scales = I.qmatmul_inputs(2, 128, 3, group=group, seed=group + zero)
    words = Q.pack_int4(codes.numpy())
    xs = x.numpy().astype(np.float64)
    ss = scales.numpy().astype(np.float64)
    np.testing.assert_allclose(Q.w4a16_matmul(xs, words, ss, group, zero),
                               _brute(xs, words, ss, group, zero), atol=1e-12, rtol=1e-12)


def test_closed_forms():
    x, _, scales = I.qmatmul_inputs(3, 64, 5, seed=2)
    xs = x.numpy().astype(np.float64)
    eights = Q.pack_int4(np.full((5, 64), 8, np.uint8))
    assert np.array_equal(Q.w4a16_matmul(xs, eights, scales.numpy()), np.zeros((3, 5)))
    c, s = 13, 0.0125
    const = Q.pack_int4(np.full((5, 64), c, np.uint8))
    y = Q.w4a16_matmul(xs, const, np.full((5, 2), s))
    np.testing.assert_allclose(y, (c - 8) * s * xs.sum(1, keepdims=True).repeat(5, 1),
                               rtol=1e-12)


def test_linearity():
    x1, codes, scales = I.qmatmul_inputs(2, 256, 9, seed=3)
    x2, _, _ = I.qmatmul_inputs(2, 256, 9, seed=4)
    w = Q.pack_int4(codes.numpy())
    a, b = x1.numpy().astype(np.float64), x2.numpy().astype(np.float64)
    s = scales.numpy()
    np.testing.assert_allclose(Q.w4a16_matmul(a + b, w, s),
                               Q.w4a16_matmul(a, w, s) + Q.w4a16_matmul(b, w, s), atol=1e-10)


@pytest.mark.parametrize("name", ["w8a16_32x32x32", "w8a16_64x64x128", "w4i8_64x64x64",
                                  "scaled_64x64x64"])
def test_w8a16_golden(golden_dir, name):
    z = np.load(golden_dir / f"qmm_{name}.npz")
    m, n, k = int(z["M"]), int(z["N"]), int(z["K"])
    kind = name.split("_")[0]
    a, b, scale = I.reference_quant_lists(m, n, k, {"w4i8": "w4a16"}.get(kind, kind))
    assert np.array_equal(np.array(a), z["a"]) and np.array_equal(np.array(b, np.int8), z["b"])
    A = z["a"].reshape(m, k)
    B = z["b"].reshape(k, n)
    if kind == "scaled":
        out = Q.w8a16_scaled_matmul(A, B, z["scale"])
    else:
        out = Q.w8a16_matmul(A, B)
    np.testing.assert_allclose(out.reshape(-1), z["expected"], rtol=1e-12, atol=1e-9)


def test_rel_err_metric():
    ref = np.array([1.0, -4.0, 2.0])
    assert Q.rel_err(ref + np.array([0.0, 0.04, 0.0]), ref) == pytest.approx(0.01)


def test_algorithmic_bytes_baseline():
    # M=1, K=4096, N=11008: K*N/2 + (K/32)*N*2 + M*K*2 + M*N*2 = 25,392,640 bytes.
    assert Q.algorithmic_bytes(1, 11008, 4096) == 25_392_640


# --- planted mistakes ------------------------------------------------------

def test_planted_high_nibble_first_is_caught(golden_dir):
    z = np.load(golden_dir / "qmm_int4_kat.npz")
    w = z["words"].view(np.uint32)
    # Mistake: read nibble 7 - (k % 8) instead of k % 8.
    wrong_codes = np.stack([(w >> np.uint32(4 * (7 - e))) & 0xF for e in range(8)], -1)
    wrong_codes = wrong_codes.reshape(w.shape[0], -1).astype(np.uint8)
    wrong = Q.w4a16_matmul(z["x"], Q.pack_int4(wrong_codes), z["scales"])
    assert not np.array_equal(wrong, z["expected"])


def test_planted_scale_index_is_caught(golden_dir):
    z = np.load(golden_dir / "qmm_int4_kat.npz")
    # Mistake: scales indexed by column k % groups instead of k // group.
    codes = Q.unpack_int4(z["words"]).astype(np.float64)
    s = z["scales"]
    k = codes.shape[1]
    wrong_w = (codes - 8) * s[:, np.arange(k) % s.shape[1]]
    wrong = z["x"] @ wrong_w.T
    assert not np.array_equal(wrong, z["expected"])
