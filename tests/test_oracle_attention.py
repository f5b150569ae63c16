"""Pins the attention oracle (oracle/attention.py) on the CPU.

Each oracle function is checked against something it was not derived from:
the reference tests' own seeded vectors and pure-Python row oracle (golden
fixtures), the harness known-answer test, torch's scaled_dot_product_attention
in float64 (an independent library routine), closed forms and invariants.
The last tests plant plausible mistakes in a copy of the oracle (bias index
direction, scale applied to the bias) and show the checks catch them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import inputs as I


def _sdpa64(q, k, v, scale, causal=False, mask=None):
    return F.scaled_dot_product_attention(q.double(), k.double(), v.double(), attn_mask=mask,
                                          is_causal=causal, scale=scale)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n,d", [(1, 32), (7, 64), (64, 64), (130, 128)])
def test_closed_form_matches_sdpa(n, d, causal):
    q, k, v = I.fa2_inputs(2, 3, n, d, seed=n + d)
    scale = 1 / math.sqrt(d)
    ref = _sdpa64(q, k, v, scale, causal=causal)
    out = A.attention(q, k, v, scale, causal=causal, dtype=torch.float64)
    assert torch.allclose(out, ref, atol=1e-10, rtol=0)


@pytest.mark.parametrize("causal,window", [(False, None), (True, None), (False, (9, 4))])
def test_query_rows_subset(causal, window):
    """query_rows gives exactly those rows of the full result (SDPA-checked
    above), with causal and window masks at the rows' own positions."""
    q, k, v = I.fa2_inputs(1, 3, 200, 64, seed=21)
    rows = torch.tensor([0, 1, 63, 64, 117, 198, 199])
    full = A.attention(q, k, v, 0.125, causal=causal, window=window, dtype=torch.float64)
    sub = A.attention(q, k, v, 0.125, causal=causal, window=window, dtype=torch.float64,
                      query_rows=rows)
    assert torch.equal(sub, full[..., rows, :])


@pytest.mark.parametrize("n,d", [(64, 32), (128, 64), (256, 64), (128, 128), (256, 128),
                                 (512, 128)])
def test_golden_reference_rows(golden_dir, n, d):
    """tests/test_flash_attention.py:268-275 inputs, :296-339 expected rows."""
    z = np.load(golden_dir / f"fa2_ref_N{n}_d{d}.npz")
    q = torch.from_numpy(z["q"].reshape(n, d))
    k = torch.from_numpy(z["k"].reshape(n, d))
    v = torch.from_numpy(z["v"].reshape(n, d))
    # The fixture's inputs are the reference generator's exact output.
    ql, kl, vl = I.reference_fa2_lists(n, d)
    assert np.array_equal(np.array(ql), z["q"]) and np.array_equal(np.array(vl), z["v"])
    out = A.attention(q, k, v, float(z["scale"]), dtype=torch.float64).numpy()
    for r, exp in zip(z["rows"], z["expected"]):
        np.testing.assert_allclose(out[r], exp, atol=1e-12, rtol=0)


def test_harness_kat(golden_dir):
    """macos/harness.rs:241-271: Q = K = 0 -> every row is the column mean of fp16(V)."""
    z = np.load(golden_dir / "fa2_kat.npz")
    n, d = int(z["N"]), int(z["d"])
    qv, kv, vv = A.kat_values(n, d)
    assert np.array_equal(vv, z["v"])
    v16 = torch.from_numpy(vv.reshape(n, d)).half()
    zeros = torch.zeros(n, d, dtype=torch.float16)
    out = A.attention(zeros, zeros, v16, 1 / 8, dtype=torch.float64).numpy()
    np.testing.assert_allclose(out.reshape(-1), z["expected"], atol=1e-12, rtol=0)
    np.testing.assert_allclose(A.kat_expected(n, d).reshape(-1), z["expected"], atol=1e-6)


def test_invariants():
    q, k, v = I.fa2_inputs(1, 2, 48, 64, seed=3)
    s = 0.125
    base = A.attention(q, k, v, s, dtype=torch.float64)
    # scale = 0 -> uniform weights -> column mean of V
    mean = v.double().mean(dim=-2, keepdim=True).expand_as(base)
    assert torch.allclose(A.attention(q, k, v, 0.0, dtype=torch.float64), mean, atol=1e-12)
    # N = 1 -> O = V
    o1 = A.attention(q[..., :1, :], k[..., :1, :], v[..., :1, :], s, dtype=torch.float64)
    assert torch.allclose(o1, v[..., :1, :].double(), atol=0)
    # causal row 0 = V[0]
    oc = A.attention(q, k, v, s, causal=True, dtype=torch.float64)
    assert torch.allclose(oc[..., 0, :], v[..., 0, :].double(), atol=0)
    # joint permutation of K/V rows leaves non-causal attention unchanged
    perm = torch.randperm(48, generator=torch.Generator().manual_seed(1))
    op = A.attention(q, k[..., perm, :], v[..., perm, :], s, dtype=torch.float64)
    assert torch.allclose(op, base, atol=1e-12)
    # a per-row constant added to the logits changes nothing (shift invariance)
    shift = torch.randn(1, 2, 48, 1, dtype=torch.float64).expand(1, 2, 48, 48)
    assert torch.allclose(A.attention(q, k, v, s, logit_bias=shift, dtype=torch.float64), base,
                          atol=1e-12)
    # every output lies in the per-column hull of V
    vmin = v.double().amin(dim=-2, keepdim=True)
    vmax = v.double().amax(dim=-2, keepdim=True)
    assert bool(((base >= vmin - 1e-12) & (base <= vmax + 1e-12)).all())


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n,bm,bn", [(64, 16, 32), (100, 16, 32), (96, 32, 64), (5, 8, 32)])
def test_online_loop_equals_closed_form(n, bm, bn, causal):
    """The blockwise recurrence (m, alpha, l, rescale) reproduces the closed form."""
    q, k, v = I.fa2_inputs(1, 1, n, 64, seed=n)
    q, k, v = (t[0, 0].float().numpy() for t in (q, k, v))
    ref = A.attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), 0.125,
                      causal=causal, dtype=torch.float64).numpy()
    exact = A.fa2_online(q, k, v, 0.125, block_m=bm, block_n=bn, p_fp16=False, causal=causal)
    np.testing.assert_allclose(exact, ref, atol=2e-6, rtol=0)
    trunc = A.fa2_online(q, k, v, 0.125, block_m=bm, block_n=bn, p_fp16=True, causal=causal)
    assert np.max(np.abs(trunc - ref)) < 2e-3


def test_table_to_dense_index():
    """B[h, i, j] = table[h, i - j + N - 1]."""
    n = 5
    table = torch.arange(2 * (2 * n - 1), dtype=torch.float32).reshape(2, 2 * n - 1)
    dense = A.rel_pos_table_to_dense(table, n)
    for h in range(2):
        for i in range(n):
            for j in range(n):
                assert dense[h, i, j] == table[h, i - j + n - 1]


def test_rel_pos_table_matches_sdpa_mask():
    h, n, d = 3, 37, 64
    q, k, v, table = I.relpos_inputs(h, n, d, seed=5)
    s = 1 / 8
    out = A.rel_pos_attention_table(q, k, v, table, s, dtype=torch.float64)
    dense = A.rel_pos_table_to_dense(table.double(), n)
    ref = _sdpa64(q, k, v, s, mask=dense)
    assert torch.allclose(out, ref, atol=1e-10)


def test_rel_pos_special_cases():
    h, n, d = 2, 40, 32
    q, k, v, _ = I.relpos_inputs(h, n, d, seed=9)
    s = 1 / math.sqrt(d)
    plain = A.attention(q, k, v, s, dtype=torch.float64)
    const = torch.full((h, 2 * n - 1), 0.7)
    assert torch.allclose(A.rel_pos_attention_table(q, k, v, const, s, dtype=torch.float64),
                          plain, atol=1e-12)
    zero = torch.zeros(h, 2 * n - 1)
    assert torch.allclose(A.rel_pos_attention_table(q, k, v, zero, s, dtype=torch.float64),
                          plain, atol=1e-12)
    spike = torch.zeros(h, 2 * n - 1)
    spike[:, n - 1] = 200.0  # offset i - j = 0: each query attends to itself
    diag = A.rel_pos_attention_table(q, k, v, spike, s, dtype=torch.float64)
    assert torch.allclose(diag, v.double(), atol=1e-6)


@pytest.mark.parametrize("t,d,nh", [(32, 64, 2), (64, 64, 4)])
def test_rel_pos_reference_mode_golden(golden_dir, t, d, nh):
    """tests/test_rel_pos_fa2.py: precompute (:286-311) + fused kernel semantics
    (QK^T + B) * scale (:196-206) reproduce the direct Transformer-XL output
    (:256-283) computed by plain loops in the fixture."""
    z = np.load(golden_dir / f"relpos_ref_T{t}_d{d}_nh{nh}.npz")
    arrs = I.reference_relpos_arrays(t, d, nh)
    for name, a in zip(("Q", "K", "V", "K_rel", "bias_u", "bias_v"), arrs):
        assert np.array_equal(a, z[name]), name
    Q, K, V, K_rel, bu, bv = arrs
    scale = float(z["scale"])
    direct = A.reference_rel_pos_attention(Q, K, V, K_rel, bu, bv, scale)
    np.testing.assert_allclose(direct, z["expected"], atol=1e-10)
    q_u, rel_bias = A.precompute_bias_and_qu(Q, K_rel, bu, bv)
    fused = A.rel_pos_attention_dense(torch.from_numpy(q_u), torch.from_numpy(K),
                                      torch.from_numpy(V), torch.from_numpy(rel_bias), scale,
                                      dtype=torch.float64).numpy()
    np.testing.assert_allclose(fused, z["expected"], atol=1e-5)


# --- planted mistakes: the checks above must catch them --------------------

def test_planted_bias_direction_is_caught():
    h, n, d = 2, 33, 64
    q, k, v, table = I.relpos_inputs(h, n, d, seed=11)
    s = 1 / 8
    j = torch.arange(n).unsqueeze(1)
    i = torch.arange(n).unsqueeze(0)
    wrong_dense = table.double()[:, (i - j + n - 1).reshape(-1)].reshape(h, n, n)  # j - i
    wrong = _sdpa64(q, k, v, s, mask=wrong_dense)
    ref = A.rel_pos_attention_table(q, k, v, table, s, dtype=torch.float64)
    assert (wrong - ref).abs().max() > 1e-2


def test_planted_bias_scaling_is_caught(golden_dir):
    z = np.load(golden_dir / "relpos_ref_T32_d64_nh2.npz")
    Q, K, V, K_rel, bu, bv = I.reference_relpos_arrays(32, 64, 2)
    q_u, rel_bias = A.precompute_bias_and_qu(Q, K_rel, bu, bv)
    scale = float(z["scale"])
    # Mistake: bias added after the scale instead of before it.
    wrong = A.attention(torch.from_numpy(q_u), torch.from_numpy(K), torch.from_numpy(V), scale,
                        logit_bias=torch.from_numpy(rel_bias), dtype=torch.float64).numpy()
    assert np.max(np.abs(wrong - z["expected"])) > 1e-2


def test_planted_missing_rescale_is_caught():
    q, k, v = (t[0, 0].float().numpy() for t in I.fa2_inputs(1, 1, 96, 64, seed=4))
    ref = A.attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), 0.5,
                      dtype=torch.float64).numpy()
    good = A.fa2_online(q, k, v, 0.5, p_fp16=False)
    # Mistake: forget alpha on the accumulator (l still rescaled).
    qb_out = np.zeros_like(q)
    for m0 in range(0, 96, 16):
        rows = slice(m0, m0 + 16)
        m_i = np.full(16, -np.inf, np.float32)
        l_i = np.zeros(16, np.float32)
        acc = np.zeros((16, 64), np.float32)
        for k0 in range(0, 96, 32):
            s = q[rows] @ k[k0:k0 + 32].T * 0.5
            m_new = np.maximum(m_i, s.max(1))
            alpha = np.exp(m_i - m_new)
            p = np.exp(s - m_new[:, None])
            l_i = l_i * alpha + p.sum(1)
            acc = acc + p @ v[k0:k0 + 32]
            m_i = m_new
        qb_out[rows] = acc / l_i[:, None]
    assert np.max(np.abs(good - ref)) < 1e-5
    assert np.max(np.abs(qb_out - ref)) > 1e-2


# ---- sliding window (debug/fa2_correctness_legacy.py:53-64) ----

@pytest.mark.parametrize("n,left,right", [(1, 0, 0), (37, 0, 0), (64, 16, 0), (100, 7, 23),
                                          (90, 200, 200), (90, 89, 0)])
def test_window_matches_sdpa_mask(n, left, right):
    q, k, v = (t[0] for t in I.fa2_inputs(1, 2, n, 64, seed=n + left))
    i = torch.arange(n).unsqueeze(1)
    j = torch.arange(n).unsqueeze(0)
    mask = torch.zeros(n, n, dtype=torch.float64)
    mask = mask.masked_fill((j < i - left) | (j > i + right), float("-inf"))
    ref = _sdpa64(q, k, v, 0.125, mask=mask)
    out = A.attention(q, k, v, 0.125, window=(left, right), dtype=torch.float64)
    assert torch.allclose(out, ref, atol=1e-12)


def test_window_special_cases():
    q, k, v = (t[0] for t in I.fa2_inputs(1, 3, 120, 32, seed=5))
    full = A.attention(q, k, v, 0.2, dtype=torch.float64)
    causal = A.attention(q, k, v, 0.2, causal=True, dtype=torch.float64)
    assert torch.equal(A.attention(q, k, v, 0.2, window=(120, 120), dtype=torch.float64), full)
    assert torch.equal(A.attention(q, k, v, 0.2, window=(500, 0), dtype=torch.float64), causal)
    # (0, 0): every query sees only its own key.
    diag = A.attention(q, k, v, 0.2, window=(0, 0), dtype=torch.float64)
    assert torch.allclose(diag, v.double(), atol=1e-15)


@pytest.mark.parametrize("name", ["fa2_window_S64_H3_d64_w16_0", "fa2_window_S48_H2_d32_w5_7"])
def test_window_golden(golden_dir, name):
    """Reference generator and reference formula (float64 loops) vs both oracle forms."""
    z = np.load(golden_dir / f"{name}.npz")
    seq, heads, d = int(z["seq"]), int(z["heads"]), int(z["d"])
    wl, wr, scale = int(z["window_left"]), int(z["window_right"]), float(z["scale"])
    for h in range(heads):
        cols = slice(h * d, (h + 1) * d)
        exp = z["expected"][:, cols]
        legacy = A.reference_window_attention(z["Q"][:, cols], z["K"][:, cols], z["V"][:, cols],
                                              scale, wl, wr)
        assert np.abs(legacy - exp).max() < 1e-5
        qt, kt, vt = (torch.from_numpy(z[x][:, cols].astype(np.float32)) for x in "QKV")
        out = A.attention(qt, kt, vt, scale, window=(wl, wr), dtype=torch.float64).numpy()
        assert np.abs(out - exp).max() < 1e-10


def test_planted_window_off_by_one_is_caught(golden_dir):
    z = np.load(golden_dir / "fa2_window_S64_H3_d64_w16_0.npz")
    cols = slice(0, 64)
    qt, kt, vt = (torch.from_numpy(z[x][:, cols].astype(np.float32)) for x in "QKV")
    wrong = A.attention(qt, kt, vt, float(z["scale"]), window=(17, 0), dtype=torch.float64)
    assert np.abs(wrong.numpy() - z["expected"][:, cols]).max() > 1e-3
