"""CPU restatement of the reference attention kernels (test infrastructure only).

Reference algorithm: the TTIR of ``flash_attention_fwd``
(/root/reference/tests/test_flash_attention.py:79-247) and of
``rel_pos_fa2_fwd`` (tests/test_rel_pos_fa2.py:80-253); the pure-Python row
oracle of tests/test_flash_attention.py:296-339; the numpy reference of
tests/test_rel_pos_fa2.py:256-311; the Q=K=0 known-answer test of
macos/harness.rs:171-271.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, *,
              causal: bool = False, logit_bias: torch.Tensor | None = None,
              window: tuple[int, int] | None = None,
              dtype: torch.dtype = torch.float32, chunk_rows: int = 1024,
              query_rows: torch.Tensor | None = None) -> torch.Tensor:
    """Closed form O = softmax(Q K^T * scale [+ logit_bias], mask) V on the CPU.

    Follows tests/test_flash_attention.py:296-339 (scores = q.k * scale, max
    subtraction, exp, normalise, weighted sum of V) vectorised over rows and
    over leading (batch, head) dimensions.  ``logit_bias`` [..., N, N] is
    added after scaling (BASELINE rel-pos semantics).  ``causal`` masks key j
    > query i, the window (inf, 0) of debug/fa2_correctness_legacy.py:53-64;
    ``window`` = (left, right) masks j < i - left and j > i + right (the
    masked logits get -inf here, -1e9 in the reference: identical results
    while every row keeps its diagonal, which non-negative windows do).
    Inputs are upcast to ``dtype``; rows are processed in chunks so the score
    matrix stays bounded.  Returns ``dtype`` [..., N, d], or, with
    ``query_rows`` (1-D indices), only those query rows [..., len, d]
    (masks use the rows' positions; for parity checks at full sizes).
    """
    q = q.to("cpu", dtype)
    k = k.to("cpu", dtype)
    v = v.to("cpu", dtype)
    n = q.shape[-2]
    rows_all = torch.arange(n) if query_rows is None else query_rows.to("cpu", torch.long)
    if query_rows is not None:
        q = q[..., rows_all, :]
        if logit_bias is not None:
            logit_bias = logit_bias[..., rows_all, :]
    nq = q.shape[-2]
    out = torch.empty(q.shape, dtype=dtype)
    kt = k.transpose(-1, -2)
    for r0 in range(0, nq, chunk_rows):
        r1 = min(nq, r0 + chunk_rows)
        s = torch.matmul(q[..., r0:r1, :], kt) * scale
        if logit_bias is not None:
            s = s + logit_bias[..., r0:r1, :].to(dtype)
        if causal or window is not None:
            rows = rows_all[r0:r1].unsqueeze(1)
            cols = torch.arange(n).unsqueeze(0)
            left, right = window if window is not None else (n, 0)
            s = s.masked_fill((cols > rows + right) | (cols < rows - left), float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        p = torch.exp(s - m)
        out[..., r0:r1, :] = torch.matmul(p, v) / p.sum(dim=-1, keepdim=True)
    return out


def fa2_online(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, *, block_m: int = 16,
               block_n: int = 32, p_fp16: bool = True, causal: bool = False,
               logit_bias: np.ndarray | None = None) -> np.ndarray:
    """Blockwise online-softmax loop of the reference TTIR, in numpy float32.

    One (batch, head) slice, q/k/v [N, d].  Per query block: m = -inf, l = 0,
    O = 0 (tests/test_flash_attention.py:165-167); per key block of
    ``block_n``: S = Q K^T (:178-182), S *= scale (:185-186),
    m' = max(m, rowmax S) (:189-196), alpha = exp(m - m') (:199-200),
    P = exp(S - m') (:203-206), l = l*alpha + rowsum P (:209-217),
    O = O*alpha + f16(P) V (:220-231, truncf at :140-145 when ``p_fp16``);
    finally O / max(l, 1e-6) (src/neso/backend/codegen/lowering.py:4352-4353).
    Keys past N and masked keys get -inf logits (tail / causal masking).
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    n, d = q.shape
    out = np.zeros((n, d), np.float32)
    for m0 in range(0, n, block_m):
        rows = np.arange(m0, min(n, m0 + block_m))
        qb = q[rows]
        m_i = np.full(len(rows), -np.inf, np.float32)
        l_i = np.zeros(len(rows), np.float32)
        acc = np.zeros((len(rows), d), np.float32)
        for k0 in range(0, n, block_n):
            cols = np.arange(k0, min(n, k0 + block_n))
            s = (qb @ k[cols].T).astype(np.float32) * np.float32(scale)
            if logit_bias is not None:
                s = s + logit_bias[np.ix_(rows, cols)].astype(np.float32)
            if causal:
                s = np.where(cols[None, :] > rows[:, None], -np.inf, s).astype(np.float32)
            m_new = np.maximum(m_i, s.max(axis=1))
            m_use = np.where(np.isneginf(m_new), 0.0, m_new).astype(np.float32)
            alpha = np.exp(m_i - m_use).astype(np.float32)
            p = np.exp(s - m_use[:, None]).astype(np.float32)
            l_i = l_i * alpha + p.sum(axis=1, dtype=np.float32)
            pv = p.astype(np.float16).astype(np.float32) if p_fp16 else p
            acc = acc * alpha[:, None] + pv @ v[cols]
            m_i = m_new
        out[rows] = acc / np.maximum(l_i, 1e-6)[:, None]
    return out


def reference_window_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float,
                               window_left: int, window_right: int) -> np.ndarray:
    """Sliding-window attention of one head, restating
    debug/fa2_correctness_legacy.py:53-64: float32 scores * sm_scale, keys
    j < i - window_left or j > i + window_right set to -1e9, softmax, @ V."""
    n = q.shape[0]
    scores = (q.astype(np.float32) @ k.astype(np.float32).T) * np.float32(sm_scale)
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    scores = np.where((j < i - window_left) | (j > i + window_right), np.float32(-1e9), scores)
    mx = scores.max(axis=1, keepdims=True)
    e = np.exp(scores - mx)
    return (e / e.sum(axis=1, keepdims=True)) @ v.astype(np.float32)


def rel_pos_table_to_dense(table: torch.Tensor, n: int) -> torch.Tensor:
    """Dense bias [H, N, N] with B[h, i, j] = table[h, i - j + N - 1]."""
    i = torch.arange(n).unsqueeze(1)
    j = torch.arange(n).unsqueeze(0)
    idx = (i - j + n - 1).reshape(-1)
    return table[:, idx].reshape(table.shape[0], n, n)


def rel_pos_attention_table(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            table: torch.Tensor, scale: float, *,
                            dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """BASELINE rel-pos FA2: softmax(Q K^T * scale + table[h, i - j + N - 1]) V, [H, N, d].

    The score structure is the reference kernel's (tests/test_rel_pos_fa2.py
    :196-206: content scores plus a per-head additive bias, then the online
    softmax of :209-240) with the bias given as a relative-offset table.
    """
    n = q.shape[-2]
    h = q.shape[0]
    out = torch.empty(q.shape, dtype=dtype)
    for hh in range(h):
        dense = rel_pos_table_to_dense(table[hh:hh + 1].to(dtype), n)[0]
        out[hh] = attention(q[hh], k[hh], v[hh], scale, logit_bias=dense, dtype=dtype)
    return out


def rel_pos_attention_dense(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            bias: torch.Tensor, scale: float, *,
                            dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Reference-kernel semantics: softmax((Q K^T + B) * scale) V with dense B [H, T, T].

    tests/test_rel_pos_fa2.py:196-206 (QK_plus_bias then * scale).  The
    kernel's fp16 output rounding (:242-246) is left to the caller.
    """
    qf = q.to("cpu", dtype)
    kf = k.to("cpu", dtype)
    b = bias.to("cpu", dtype)
    # (QK^T + B) * scale == QK^T * scale + B * scale
    return attention(qf, kf, v, scale, logit_bias=b * scale, dtype=dtype)


def reference_rel_pos_attention(q, k, v, k_rel, bias_u, bias_v, scale):
    """Transformer-XL relative attention computed directly (float64 numpy).

    Restates tests/test_rel_pos_fa2.py:256-283: content = (Q + u) K^T,
    rel[i, j] = (Q + v)_i . K_rel[T - 1 - i + j], scores = (content + rel) *
    scale, softmax, times V.  Shapes [nh, T, d], k_rel [nh, 2T-1, d],
    bias_u / bias_v [nh, d].
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    k_rel = np.asarray(k_rel, np.float64)
    nh, t, _ = q.shape
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    idx = t - 1 - i + j
    out = np.zeros_like(q)
    for h in range(nh):
        q_u = q[h] + bias_u[h]
        q_v = q[h] + bias_v[h]
        content = q_u @ k[h].T
        rel_all = q_v @ k_rel[h].T  # [T, 2T-1]: (Q+v)_i . K_rel[r]
        rel = np.take_along_axis(rel_all, idx, axis=1)
        s = (content + rel) * scale
        s = s - s.max(axis=-1, keepdims=True)
        e = np.exp(s)
        out[h] = (e / e.sum(axis=-1, keepdims=True)) @ v[h]
    return out


def precompute_bias_and_qu(q, k_rel, bias_u, bias_v):
    """Host precompute of the fused kernel's inputs (float32 numpy).

    Restates tests/test_rel_pos_fa2.py:286-311: Q_u = Q + bias_u and the
    UNSCALED dense bias rel_bias[h, i, j] = (Q + bias_v)_i . K_rel[T-1-i+j]
    (accumulated in float64, stored float32).  The kernel then computes
    (Q_u K^T + rel_bias) * scale.
    """
    q = np.asarray(q, np.float32)
    k_rel = np.asarray(k_rel, np.float32)
    bias_u = np.asarray(bias_u, np.float32)
    bias_v = np.asarray(bias_v, np.float32)
    nh, t, _ = q.shape
    q_u = q + bias_u[:, None, :]
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    idx = t - 1 - i + j
    rel_bias = np.zeros((nh, t, t), np.float32)
    for h in range(nh):
        q_v = (q[h] + bias_v[h]).astype(np.float64)
        rel_all = q_v @ k_rel[h].astype(np.float64).T
        rel_bias[h] = np.take_along_axis(rel_all, idx, axis=1).astype(np.float32)
    return q_u, rel_bias


def kat_values(n: int, d: int = 64):
    """Deterministic harness inputs of macos/harness.rs:171-183 (flattened [n*d] float32)."""
    i = np.arange(n * d)
    q = ((i % 29).astype(np.float32) - 14.0) * np.float32(0.01)
    k = ((i % 31).astype(np.float32) - 15.0) * np.float32(0.01)
    v = ((i % 17).astype(np.float32) - 8.0) * np.float32(0.125)
    return q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)


def kat_expected(n: int, d: int = 64) -> np.ndarray:
    """Known answer of macos/harness.rs:241-271: with Q = K = 0 every output
    row is the column mean of fp16(V) (uniform attention)."""
    _, _, v = kat_values(n, d)
    v16 = v.astype(np.float16).astype(np.float64).reshape(n, d)
    return np.broadcast_to(v16.mean(axis=0), (n, d)).astype(np.float32)


def flops(b: int, h: int, n: int, d: int, causal: bool) -> float:
    """Algorithmic FLOPs 4*B*H*N^2*d, halved for causal (BASELINE formula)."""
    f = 4.0 * b * h * n * n * d
    return f / 2 if causal else f


def default_scale(d: int) -> float:
    return 1.0 / math.sqrt(d)
