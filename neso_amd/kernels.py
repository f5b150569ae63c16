"""Host-side launchers with the reference kernels' names and positional order.

The reference launches hand-written TTIR kernels by name with positional
buffers, e.g. ``dispatch(pipe, (N // BM, 1, 1), threads, [Q, K, V, O, N,
stride_qo, stride_kv, scale])`` (tests/test_flash_attention.py:65-76,
:283-292).  Here each kernel is a Python function taking the same positional
arguments - device tensors (or raw device addresses) followed by the
scalars - that calls the C ABI of ``libneso_amd.so`` on the current HIP
stream.  The grid is derived by the library, so it is not an argument.

Errors follow the reference: invalid arguments raise
:class:`~neso_amd._lib.NesoArgumentError` (a ``ValueError`` and a
``RuntimeError``), launch failures raise :class:`~neso_amd._lib.NesoError`
(a ``RuntimeError``).  There is no CPU path: without the library, or
without a GPU, these functions raise.
"""
from __future__ import annotations

import contextlib

import math
from typing import Any

import torch

from . import _lib

__all__ = [
    "flash_attention_fwd",
    "flash_attention_io_fwd",
    "flash_attention_window_fwd",
    "rel_pos_fa2_fwd",
    "rel_pos_precompute",
    "precompute_bias_and_qu",
    "w4a16_matmul",
    "w8a16_matmul",
    "w8a16_scaled_matmul",
    "launch",
    "launch_plan",
    "manifest",
    "KERNELS",
    "attention",
    "rel_pos_attention",
    "window_attention",
    "w4a16_linear",
]


def _ptr(x: Any, name: str, dtype: torch.dtype | tuple[torch.dtype, ...] | None) -> int:
    """Device address of a tensor (dtype/device checked) or a raw integer address."""
    if x is None:
        return 0
    if isinstance(x, int):
        return x
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor or a device address, got {type(x)!r}")
    if x.device.type != "cuda":
        raise ValueError(f"{name}: tensor must be on the GPU (got {x.device}); there is no CPU path")
    if dtype is not None:
        allowed = dtype if isinstance(dtype, tuple) else (dtype,)
        if x.dtype not in allowed:
            raise TypeError(f"{name}: dtype {x.dtype} not in {allowed}")
    return x.data_ptr()


def _extent(x: Any, name: str, elems: int) -> None:
    """Raise ValueError if tensor ``x`` cannot hold ``elems`` elements from its
    first element on (the extent the declared sizes and strides imply).

    The kernels bound their loads by the declared sizes, not by the tensor,
    so a short tensor would be read or written past its allocation.  Raw
    integer addresses are the caller's responsibility.
    """
    if not isinstance(x, torch.Tensor) or elems <= 0:
        return
    avail = x.untyped_storage().nbytes() - x.storage_offset() * x.element_size()
    if elems * x.element_size() > avail:
        raise ValueError(f"{name}: the declared sizes and strides span {elems} elements but the "
                         f"tensor holds {avail // x.element_size()} from its first element")


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _stream(stream: Any, *tensors: Any) -> int:
    if stream is not None:
        return int(stream.cuda_stream) if hasattr(stream, "cuda_stream") else int(stream)
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.device.type == "cuda":
            return int(torch.cuda.current_stream(t.device).cuda_stream)
    return 0


def _on_stream(stream: int, device):
    """Context that makes ``stream`` (a raw HIP stream handle) torch's current
    stream, so that torch work in it is ordered with the launch."""
    if torch.cuda.current_stream(device).cuda_stream == stream:
        return contextlib.nullcontext()
    return torch.cuda.stream(torch.cuda.ExternalStream(stream, device=device))


# fp32 inputs of the split-precision kernels (fp16 hi + lo per element) keep
# fp32-class accuracy while their largest magnitude lies in this range: below
# it the lo parts (and the hi parts of small elements) fall into fp16
# subnormals, from 2^15 up the hi parts approach the fp16 limit (65504).
_SPLIT_RANGE = (2.0 ** -2, 2.0 ** 15)
_SPLIT_TOP = 14     # rescaled inputs get their largest |x| in [2^13, 2^14)
_QK_EXP_CAP = 50    # |exponent| of a Q or K rescale, so that the folded scale stays normal


def _split_exponents(inputs, stream: int) -> dict[str, int]:
    """Power-of-two exponents for the fp32 inputs of a split-precision call.

    ``inputs`` holds (tensor, name, view shape, view strides) for the
    elements the kernel reads.  One reduction per input and one
    synchronisation for all of them, on ``stream`` (the launch stream), so
    data written there before the call is what is measured.  Returns
    {name: k} for each input whose largest |x| lies outside _SPLIT_RANGE: k
    puts it in [2^13, 2^14), where the hi + lo split is exact to ~2^-22 of
    the largest element, instead of underflowing (tiny inputs) or
    overflowing (|x| >= 65504) in fp16.  Raises NesoArgumentError for
    infinite inputs; NaN inputs pass (they give NaN rows, as an fp32
    computation does).  Returns {} for raw addresses, host tensors
    (rejected at launch) and while the stream is being captured into a
    graph, where no synchronisation is possible."""
    views = [(t.as_strided(shape, strides), name) for t, name, shape, strides in inputs
             if isinstance(t, torch.Tensor) and t.device.type == "cuda"]
    if not views or torch.cuda.is_current_stream_capturing():
        return {}
    dev = views[0][0].device
    with _on_stream(stream, dev):
        if torch.cuda.is_current_stream_capturing():
            return {}
        maxima = torch.stack([v.abs().amax() for v, _ in views]).cpu()
    out = {}
    for (_, name), m in zip(views, maxima.tolist()):
        if math.isinf(m):
            raise _lib.NesoArgumentError(
                _lib.NESO_EINVAL, f"{name}: infinite element; fp32 inputs must be finite")
        if m != m or m == 0.0 or _SPLIT_RANGE[0] <= m < _SPLIT_RANGE[1]:
            continue
        out[name] = _SPLIT_TOP - math.frexp(m)[1]  # m in [2^(e-1), 2^e)
    return out


def _pow2_scaled(t: torch.Tensor, k: int, name: str, stream: int) -> torch.Tensor:
    """t * 2^k (exact: a power-of-two factor only moves exponents), same
    shape and layout as t, formed on the launch stream."""
    if not t.is_contiguous():
        raise _lib.NesoArgumentError(
            _lib.NESO_EINVAL, f"{name}: a non-contiguous fp32 input whose magnitude lies outside "
                              f"[2^-2, 2^15) cannot be rescaled for the fp16 hi + lo split")
    with _on_stream(stream, t.device):
        return t * (2.0 ** k)


def _rescale_split_inputs(Q, K, V, O, scale: float, inputs, stream: int, o_view):
    """Apply _split_exponents: Q, K, V replaced by power-of-two rescaled
    copies where needed, the Q and K factors folded into ``scale``.  Returns
    (Q, K, V, scale, post) where ``post()`` undoes V's factor on O's view
    after the launch (None when V is not rescaled; V is left alone when O
    is not a tensor, and then must lie below 65504)."""
    exps = _split_exponents(inputs, stream)
    if not exps:
        return Q, K, V, scale, None
    kq = max(-_QK_EXP_CAP, min(_QK_EXP_CAP, exps.get("Q", 0)))
    kk = max(-_QK_EXP_CAP, min(_QK_EXP_CAP, exps.get("K", 0)))
    kv = exps.get("V", 0)
    if kq:
        Q = _pow2_scaled(Q, kq, "Q", stream)
    if kk:
        K = _pow2_scaled(K, kk, "K", stream)
    post = None
    if kv and isinstance(O, torch.Tensor):
        V = _pow2_scaled(V, kv, "V", stream)

        def post():
            with _on_stream(stream, O.device):
                o_view().mul_(2.0 ** -kv)
    elif kv < 0:
        raise _lib.NesoArgumentError(
            _lib.NESO_EINVAL, "V: |x| reaches the fp16 limit (65504) of the hi + lo split and O "
                              "is a raw address, so the result cannot be rescaled")
    return Q, K, V, scale * 2.0 ** -(kq + kk), post


def flash_attention_fwd(Q, K, V, O, N: int, stride_qo: int, stride_kv: int, scale: float, *,
                        head_dim: int | None = None, batch_heads: int = 1,
                        stride_bh_qo: int = 0, stride_bh_kv: int = 0, causal: bool = False,
                        qkv_dtype: str | None = None, check_range: bool = True,
                        stream=None) -> None:
    """FA2 forward, O = softmax(Q K^T * scale) V.

    Positional arguments as the reference kernel (tests/test_flash_attention.py
    :149-153): Q, K, V [N, d] rows, O fp32 rows with row stride
    ``stride_qo``, N, stride_qo, stride_kv (elements), scale.  Keyword
    extensions: ``head_dim`` (inferred from ``Q.shape[-1]`` for tensors),
    ``batch_heads`` with ``stride_bh_qo`` / ``stride_bh_kv`` for B*H slices
    in one launch, and ``causal``.  ``qkv_dtype`` is 'f16' or 'f32' as in
    the reference's generator (:79-89); for tensors it follows Q's dtype.
    The fp32 kernel splits each element into fp16 hi + lo; with
    ``check_range`` (default) the largest |x| of each fp32 tensor is
    measured first (one device reduction per input and one synchronisation)
    and a tensor outside [2^-2, 2^15) is replaced by an exact power-of-two
    rescaled copy, its factor folded into ``scale`` (Q, K) or undone on O
    (V), so any finite magnitude keeps fp32-class accuracy.  Without it, or
    under graph capture, fp32 elements must lie below 65504 in magnitude.
    """
    if head_dim is None:
        if not isinstance(Q, torch.Tensor):
            raise ValueError("head_dim is required when Q is a raw address")
        head_dim = int(Q.shape[-1])
    if qkv_dtype is None:
        qkv_dtype = "f32" if isinstance(Q, torch.Tensor) and Q.dtype == torch.float32 else "f16"
    if qkv_dtype not in ("f16", "f32"):
        raise ValueError(f"qkv_dtype must be 'f16' or 'f32', got {qkv_dtype!r}")
    if N > 0 and batch_heads > 0:
        span_q = (batch_heads - 1) * stride_bh_qo + (N - 1) * stride_qo + head_dim
        span_kv = (batch_heads - 1) * stride_bh_kv + (N - 1) * stride_kv + head_dim
        for t, nm, sp in ((Q, "Q", span_q), (K, "K", span_kv), (V, "V", span_kv),
                          (O, "O", span_q)):
            _extent(t, nm, sp)
    post = None
    if qkv_dtype == "f32" and check_range and N > 0 and batch_heads > 0:
        st = _stream(stream, Q, O)
        Q, K, V, scale, post = _rescale_split_inputs(
            Q, K, V, O, scale,
            [(t, nm, (batch_heads, N, head_dim), (sb, sr, 1))
             for t, nm, sr, sb in ((Q, "Q", stride_qo, stride_bh_qo),
                                   (K, "K", stride_kv, stride_bh_kv),
                                   (V, "V", stride_kv, stride_bh_kv))
             if isinstance(t, torch.Tensor) and t.dtype == torch.float32], st,
            lambda: O.as_strided((batch_heads, N, head_dim), (stride_bh_qo, stride_qo, 1)))
    lib = _lib.load()
    dt = torch.float32 if qkv_dtype == "f32" else torch.float16
    fn = lib.neso_flash_attention_f32_fwd if qkv_dtype == "f32" else lib.neso_flash_attention_fwd
    st = fn(
        _ptr(Q, "Q", dt), _ptr(K, "K", dt), _ptr(V, "V", dt),
        _ptr(O, "O", torch.float32), int(N), int(stride_qo), int(stride_kv), float(scale),
        int(head_dim), int(batch_heads), int(stride_bh_qo), int(stride_bh_kv), int(bool(causal)),
        _stream(stream, Q, O))
    _lib.check(st)
    if post:
        post()


def flash_attention_io_fwd(Q, K, V, O, N: int, d_head: int, scale: float, *,
                           batch_heads: int = 1, io_dtype: str | None = None,
                           check_range: bool = True, stream=None) -> None:
    """FA2 forward with O in the input type, O = softmax(Q K^T * scale) V.

    Positional arguments as the hand-written reference kernel
    (bench/bench_flash_attention.py:142-152): Q, K, V, O [N, d_head] rows of
    one type (``io_type`` half or float there), N, d_head, scale.  Keyword
    extensions: ``batch_heads`` contiguous [batch_heads, N, d_head] slices in
    one launch; ``io_dtype`` 'f16' or 'f32' (inferred from Q for tensors).
    fp32 tensors are rescaled by powers of two where their magnitude needs
    it, as in :func:`flash_attention_fwd` (``check_range``; without it, or
    under graph capture, fp32 elements must lie below 65504 in magnitude).
    """
    if io_dtype is None:
        if not isinstance(Q, torch.Tensor):
            raise ValueError("io_dtype is required when Q is a raw address")
        io_dtype = "f32" if Q.dtype == torch.float32 else "f16"
    if io_dtype not in ("f16", "f32"):
        raise ValueError(f"io_dtype must be 'f16' or 'f32', got {io_dtype!r}")
    if N > 0 and batch_heads > 0:
        for t, nm in ((Q, "Q"), (K, "K"), (V, "V"), (O, "O")):
            _extent(t, nm, batch_heads * N * d_head)
    post = None
    if io_dtype == "f32" and check_range and N > 0 and batch_heads > 0:
        n_el = batch_heads * N * d_head
        Q, K, V, scale, post = _rescale_split_inputs(
            Q, K, V, O, scale,
            [(t, nm, (n_el,), (1,)) for t, nm in ((Q, "Q"), (K, "K"), (V, "V"))
             if isinstance(t, torch.Tensor) and t.dtype == torch.float32],
            _stream(stream, Q, O), lambda: O.view(-1)[:n_el])
    dt = torch.float32 if io_dtype == "f32" else torch.float16
    lib = _lib.load()
    st = lib.neso_flash_attention_io_fwd(
        _ptr(Q, "Q", dt), _ptr(K, "K", dt), _ptr(V, "V", dt), _ptr(O, "O", dt), int(N),
        int(d_head), float(scale), _lib.NESO_IO_F32 if io_dtype == "f32" else _lib.NESO_IO_F16,
        int(batch_heads), _stream(stream, Q, O))
    _lib.check(st)
    if post:
        post()


def flash_attention_window_fwd(Q, K, V, O, seq_len: int, stride_h: int, stride_m: int,
                               sm_scale: float, window_left: int, window_right: int, *,
                               num_heads: int, head_dim: int | None = None,
                               stream=None) -> None:
    """Sliding-window attention: key j is visible to query i iff
    i - window_left <= j <= i + window_right.

    Positional arguments as the windowed reference kernel
    (debug/fa2_correctness_legacy.py:92-102): Q, K, V fp16, O, seq_len,
    stride_h (elements between heads of one row), stride_m (elements
    between rows), sm_scale, window_left, window_right.  ``num_heads``
    replaces the reference's grid y.  The output dtype follows O (fp16 as in
    the reference, or fp32).
    """
    if head_dim is None:
        if not isinstance(Q, torch.Tensor):
            raise ValueError("head_dim is required when Q is a raw address")
        head_dim = int(Q.shape[-1])
    if isinstance(O, torch.Tensor):
        out_dtype = _lib.NESO_OUT_F32 if O.dtype == torch.float32 else _lib.NESO_OUT_F16
    else:
        out_dtype = _lib.NESO_OUT_F16
    if seq_len > 0 and num_heads > 0:
        span = (seq_len - 1) * stride_m + (num_heads - 1) * stride_h + head_dim
        for t, nm in ((Q, "Q"), (K, "K"), (V, "V"), (O, "O")):
            _extent(t, nm, span)
    lib = _lib.load()
    st = lib.neso_flash_attention_window_fwd(
        _ptr(Q, "Q", torch.float16), _ptr(K, "K", torch.float16), _ptr(V, "V", torch.float16),
        _ptr(O, "O", (torch.float16, torch.float32)), int(seq_len), int(stride_h), int(stride_m),
        float(sm_scale), int(window_left), int(window_right), int(num_heads), int(head_dim),
        int(out_dtype), _stream(stream, Q, O))
    _lib.check(st)


def rel_pos_fa2_fwd(Q, K, V, bias, O, T: int, stride: int, scale: float, stride_h: int,
                    bias_stride_h: int, *, num_heads: int, head_dim: int | None = None,
                    bias_mode: int = _lib.NESO_BIAS_DENSE_SCALED_F16, stream=None) -> None:
    """Relative-position-bias FA2.

    Positional arguments as the reference (tests/test_rel_pos_fa2.py:157-163):
    Q, K, V fp16 [nh, T, d], bias, O, T, stride, scale, stride_h,
    bias_stride_h.  ``num_heads`` replaces the reference's grid y.
    ``bias_mode`` selects NESO_BIAS_DENSE_SCALED_F16 (reference: f16
    [nh, T, T], logits (QK^T + B) * scale) or NESO_BIAS_TABLE_F32 (f32
    [nh, 2T-1], logits QK^T * scale + B[i - j + T - 1]).  The output dtype
    follows O (fp16 as in the reference, or fp32).
    """
    if head_dim is None:
        if not isinstance(Q, torch.Tensor):
            raise ValueError("head_dim is required when Q is a raw address")
        head_dim = int(Q.shape[-1])
    if isinstance(O, torch.Tensor):
        out_dtype = _lib.NESO_OUT_F32 if O.dtype == torch.float32 else _lib.NESO_OUT_F16
    else:
        out_dtype = _lib.NESO_OUT_F16
    bias_dtype = torch.float16 if bias_mode == _lib.NESO_BIAS_DENSE_SCALED_F16 else torch.float32
    if T > 0 and num_heads > 0:
        span = (num_heads - 1) * stride_h + (T - 1) * stride + head_dim
        for t, nm in ((Q, "Q"), (K, "K"), (V, "V"), (O, "O")):
            _extent(t, nm, span)
        per_head = T * T if bias_mode == _lib.NESO_BIAS_DENSE_SCALED_F16 else 2 * T - 1
        _extent(bias, "bias", (num_heads - 1) * bias_stride_h + per_head)
    lib = _lib.load()
    st = lib.neso_rel_pos_fa2_fwd(
        _ptr(Q, "Q", torch.float16), _ptr(K, "K", torch.float16), _ptr(V, "V", torch.float16),
        _ptr(bias, "bias", bias_dtype), _ptr(O, "O", (torch.float16, torch.float32)), int(T),
        int(stride), float(scale), int(stride_h), int(bias_stride_h), int(num_heads),
        int(head_dim), int(bias_mode), int(out_dtype), _stream(stream, Q, O))
    _lib.check(st)


def rel_pos_precompute(Q, K_rel, bias_u, bias_v, T: int, d: int, nh: int, scale: float, Q_u,
                       rel_bias, *, check_range: bool = True, stream=None) -> None:
    """Q_u = Q + bias_u and the unscaled dense rel_bias[h, i, j] = (Q + bias_v)_i .
    K_rel[T - 1 - i + j] on the GPU.

    Leading arguments as the reference's host precompute
    ``precompute_bias_and_qu(Q, K_rel, bias_u, bias_v, T, d, nh, scale)``
    (tests/test_rel_pos_fa2.py:286-311; ``scale`` unused, as there), then
    the two outputs it returns: Q_u fp16 [nh, T, d] and rel_bias fp16
    [nh, T, T], the inputs of :func:`rel_pos_fa2_fwd` in the dense mode.
    Q, K_rel, bias_u, bias_v are contiguous fp32 [nh, T, d], [nh, 2T-1, d],
    [nh, d], [nh, d].  The bias is formed from fp16 hi + lo splits of
    Q + bias_v and K_rel, so their elements must lie below 65504 in
    magnitude; ``check_range`` verifies that before the launch (device
    reductions and a synchronisation, skipped under graph capture).
    """
    if T > 0 and nh > 0:
        for t, nm, n in ((Q, "Q", nh * T * d), (K_rel, "K_rel", nh * (2 * T - 1) * d),
                         (bias_u, "bias_u", nh * d), (bias_v, "bias_v", nh * d),
                         (Q_u, "Q_u", nh * T * d), (rel_bias, "rel_bias", nh * T * T)):
            _extent(t, nm, n)
        if check_range and all(isinstance(x, torch.Tensor) and x.device.type == "cuda"
                               and x.dtype == torch.float32 for x in (Q, K_rel, bias_v)) \
                and not torch.cuda.is_current_stream_capturing():
            st = _stream(stream, Q, Q_u)
            with _on_stream(st, Q.device):
                qv = (Q.reshape(-1)[:nh * T * d].view(nh, T, d)
                      + bias_v.reshape(-1)[:nh * d].view(nh, 1, d))
                kr = K_rel.reshape(-1)[:nh * (2 * T - 1) * d]
                maxima = torch.stack([qv.abs().amax(), kr.abs().amax()]).cpu().tolist()
            for m, nm in zip(maxima, ("Q + bias_v", "K_rel")):
                if m >= 65504.0:
                    raise _lib.NesoArgumentError(
                        _lib.NESO_EINVAL, f"{nm}: |x| reaches {m:g}; the precompute needs "
                                          f"|Q + bias_v|, |K_rel| < 65504 (fp16 hi + lo split)")
    lib = _lib.load()
    f32, f16 = torch.float32, torch.float16
    st = lib.neso_rel_pos_precompute(
        _ptr(Q, "Q", f32), _ptr(K_rel, "K_rel", f32), _ptr(bias_u, "bias_u", f32),
        _ptr(bias_v, "bias_v", f32), int(T), int(d), int(nh), float(scale),
        _ptr(Q_u, "Q_u", f16), _ptr(rel_bias, "rel_bias", f16), _stream(stream, Q, Q_u))
    _lib.check(st)


def w4a16_matmul(X, W, scales, Y, M: int, N: int, K: int, stride_xm: int, stride_ym: int,
                 group_size: int = 32, zero_point: int = 8, *, stream=None) -> None:
    """Y[M, N] fp16 = X[M, K] fp16 @ dequant(W)^T, W int32 [N, K/8] (int4, low nibble first)."""
    if M > 0 and N > 0 and K > 0 and group_size > 0:
        _extent(X, "X", (M - 1) * stride_xm + K)
        _extent(W, "W", N * (K // 8))
        _extent(scales, "scales", N * (K // group_size))
        _extent(Y, "Y", (M - 1) * stride_ym + N)
    lib = _lib.load()
    st = lib.neso_w4a16_matmul(
        _ptr(X, "X", torch.float16), _ptr(W, "W", torch.int32), _ptr(scales, "scales", torch.float16),
        _ptr(Y, "Y", torch.float16), int(M), int(N), int(K), int(stride_xm), int(stride_ym),
        int(group_size), int(zero_point), _stream(stream, X, Y))
    _lib.check(st)


def _w8_extents(A, B, C, scale, K, stride_am, stride_bk, stride_cm, M, N) -> None:
    if M > 0 and N > 0 and K > 0:
        _extent(A, "A", (M - 1) * stride_am + K)
        _extent(B, "B", (K - 1) * stride_bk + N)
        _extent(C, "C", (M - 1) * stride_cm + N)
        _extent(scale, "scale", N)


def w8a16_matmul(A, B, C, K: int, stride_am: int, stride_bk: int, stride_cm: int, *, M: int,
                 N: int, stream=None) -> None:
    """C fp32 = A fp16 @ f16(B int8 [K, N]) (tests/test_quantized_matmul.py:77-80 order)."""
    _w8_extents(A, B, C, None, K, stride_am, stride_bk, stride_cm, M, N)
    lib = _lib.load()
    st = lib.neso_w8a16_matmul(
        _ptr(A, "A", torch.float16), _ptr(B, "B", torch.int8), _ptr(C, "C", torch.float32), int(K),
        int(stride_am), int(stride_bk), int(stride_cm), int(M), int(N), _stream(stream, A, C))
    _lib.check(st)


def w8a16_scaled_matmul(A, B, C, scale, K: int, stride_am: int, stride_bk: int, stride_cm: int,
                        *, M: int, N: int, stream=None) -> None:
    """C = (A @ f16(B)) * scale[n] (tests/test_quantized_matmul.py:189-192 order)."""
    _w8_extents(A, B, C, scale, K, stride_am, stride_bk, stride_cm, M, N)
    lib = _lib.load()
    st = lib.neso_w8a16_scaled_matmul(
        _ptr(A, "A", torch.float16), _ptr(B, "B", torch.int8), _ptr(C, "C", torch.float32),
        _ptr(scale, "scale", torch.float16), int(K), int(stride_am), int(stride_bk),
        int(stride_cm), int(M), int(N), _stream(stream, A, C))
    _lib.check(st)


KERNELS = {
    "flash_attention_fwd": flash_attention_fwd,
    "flash_attention_io_fwd": flash_attention_io_fwd,
    "flash_attention_window_fwd": flash_attention_window_fwd,
    "rel_pos_fa2_fwd": rel_pos_fa2_fwd,
    "rel_pos_precompute": rel_pos_precompute,
    "w4a16_matmul": w4a16_matmul,
    "w8a16_matmul": w8a16_matmul,
    "w8a16_scaled_matmul": w8a16_scaled_matmul,
}


def manifest() -> dict:
    """The library's kernel manifest (``neso_kernel_manifest``) as a dict: per
    entry point the reference's AOT fields (src/neso/aot_compile.py:108-117)
    and per device-kernel variant its launch geometry."""
    import json
    return json.loads(_lib.load().neso_kernel_manifest().decode())


def launch_plan(name: str, *args, cu_count: int = 0, **kwargs) -> list[dict]:
    """The kernel launches that ``launch(name, *args, **kwargs)`` would issue,
    recorded instead of issued (``neso_plan_begin`` / ``neso_plan_end``): each
    a dict with the device kernel, its template arguments, grid,
    threadgroup size and warp count.  Needs no GPU; ``cu_count`` stands in
    for the device's compute units (0: the current device's).  Tensors must
    still be given on the GPU or as raw device addresses."""
    import json
    lib = _lib.load()
    _lib.check(lib.neso_plan_begin(int(cu_count)))
    try:
        launch(name, *args, **kwargs)
    finally:
        plan = json.loads(lib.neso_plan_end().decode())
    return plan["launches"]


def launch(name: str, *args, **kwargs) -> None:
    """Launch a kernel by its reference name with positional arguments."""
    try:
        fn = KERNELS[name]
    except KeyError:
        raise ValueError(f"unknown kernel {name!r}; known: {sorted(KERNELS)}") from None
    fn(*args, **kwargs)


# ---------------------------------------------------------------------------
# Tensor-level conveniences over the launchers above.

def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False,
              scale: float | None = None, out: torch.Tensor | None = None,
              check_range: bool = True) -> torch.Tensor:
    """FA2 forward over [..., N, d] fp16 or fp32 tensors (contiguous, one
    dtype); returns fp32 [..., N, d].  ``check_range`` as in
    flash_attention_fwd (fp32 inputs only)."""
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v must have the same shape [..., N, d]")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError("q, k, v must be contiguous")
    if not q.dtype == k.dtype == v.dtype:
        raise TypeError("q, k, v must share one dtype")
    n, d = int(q.shape[-2]), int(q.shape[-1])
    bh = q.numel() // max(n * d, 1) if n * d else 0
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    _require(out.shape == q.shape and out.is_contiguous() and out.dtype == torch.float32,
             f"out must be a contiguous fp32 tensor of shape {tuple(q.shape)}")
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    flash_attention_fwd(q, k, v, out, n, d, d, scale, head_dim=d, batch_heads=bh,
                        stride_bh_qo=n * d, stride_bh_kv=n * d, causal=causal,
                        check_range=check_range)
    return out


def rel_pos_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, table: torch.Tensor, *,
                      scale: float | None = None, out_dtype: torch.dtype = torch.float32,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(Q K^T * scale + table[h, i - j + N - 1]) V for [H, N, d] fp16, table f32 [H, 2N-1]."""
    _require(q.dim() == 3, f"q must be [H, N, d], got {tuple(q.shape)}")
    _require(k.shape == q.shape and v.shape == q.shape,
             f"k {tuple(k.shape)} and v {tuple(v.shape)} must match q {tuple(q.shape)}")
    _require(q.is_contiguous() and k.is_contiguous() and v.is_contiguous(),
             "q, k, v must be contiguous")
    _require(q.dtype == k.dtype == v.dtype == torch.float16, "q, k, v must be fp16")
    h, n, d = (int(s) for s in q.shape)
    if table.shape != (h, 2 * n - 1):
        raise ValueError(f"table must be [H, 2N-1] = [{h}, {2 * n - 1}], got {tuple(table.shape)}")
    _require(table.is_contiguous() and table.dtype == torch.float32,
             "table must be a contiguous fp32 tensor")
    _require(out_dtype in (torch.float16, torch.float32), "out_dtype must be fp16 or fp32")
    if out is not None:
        _require(out.shape == q.shape and out.is_contiguous() and out.dtype == out_dtype,
                 f"out must be a contiguous {out_dtype} tensor of shape {tuple(q.shape)}")
    if out is None:
        out = torch.empty((h, n, d), dtype=out_dtype, device=q.device)
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    rel_pos_fa2_fwd(q, k, v, table, out, n, d, scale, n * d, 2 * n - 1, num_heads=h, head_dim=d,
                    bias_mode=_lib.NESO_BIAS_TABLE_F32)
    return out


def precompute_bias_and_qu(q: torch.Tensor, k_rel: torch.Tensor, bias_u: torch.Tensor,
                           bias_v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """GPU counterpart of the reference's ``precompute_bias_and_qu``
    (tests/test_rel_pos_fa2.py:286-311) on fp32 tensors q [nh, T, d],
    k_rel [nh, 2T-1, d], bias_u / bias_v [nh, d]; returns (Q_u fp16
    [nh, T, d], rel_bias fp16 [nh, T, T]) for :func:`rel_pos_fa2_fwd`."""
    _require(q.dim() == 3, f"q must be [nh, T, d], got {tuple(q.shape)}")
    nh, t, d = (int(x) for x in q.shape)
    _require(tuple(k_rel.shape) == (nh, 2 * t - 1, d),
             f"k_rel must be [nh, 2T-1, d] = [{nh}, {2 * t - 1}, {d}], got {tuple(k_rel.shape)}")
    for x, nm in ((bias_u, "bias_u"), (bias_v, "bias_v")):
        _require(tuple(x.shape) == (nh, d), f"{nm} must be [nh, d] = [{nh}, {d}]")
    for x, nm in ((q, "q"), (k_rel, "k_rel"), (bias_u, "bias_u"), (bias_v, "bias_v")):
        _require(x.is_contiguous() and x.dtype == torch.float32, f"{nm} must be contiguous fp32")
    q_u = torch.empty((nh, t, d), dtype=torch.float16, device=q.device)
    rel_bias = torch.empty((nh, t, t), dtype=torch.float16, device=q.device)
    rel_pos_precompute(q, k_rel, bias_u, bias_v, t, d, nh, 1.0 / math.sqrt(d), q_u, rel_bias)
    return q_u, rel_bias


def window_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window_left: int,
                     window_right: int, *, scale: float | None = None,
                     out_dtype: torch.dtype = torch.float16,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Sliding-window attention over fp16 [seq, heads, d] tensors (the
    reference's [seq][heads * d] rows); returns [seq, heads, d] in out_dtype."""
    if q.shape != k.shape or q.shape != v.shape or q.dim() != 3:
        raise ValueError("q, k, v must have the same shape [seq, heads, d]")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError("q, k, v must be contiguous")
    n, h, d = (int(x) for x in q.shape)
    if out is None:
        out = torch.empty((n, h, d), dtype=out_dtype, device=q.device)
    _require(out.shape == q.shape and out.is_contiguous()
             and out.dtype in (torch.float16, torch.float32),
             f"out must be a contiguous fp16 or fp32 tensor of shape {tuple(q.shape)}")
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    flash_attention_window_fwd(q, k, v, out, n, d, h * d, scale, window_left, window_right,
                               num_heads=h, head_dim=d)
    return out


def w4a16_linear(x: torch.Tensor, w_packed: torch.Tensor, scales: torch.Tensor, *,
                 group_size: int = 32, zero_point: int = 8,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """x [M, K] fp16 @ dequant(w_packed [N, K/8] int32, scales [N, K/group])^T -> fp16 [M, N]."""
    _require(x.dim() == 2 and x.stride(1) == 1, "x must be [M, K] with unit column stride")
    m, k = (int(s) for s in x.shape)
    _require(w_packed.dim() == 2 and w_packed.is_contiguous() and w_packed.dtype == torch.int32,
             "w_packed must be a contiguous int32 [N, K/8] tensor")
    n = int(w_packed.shape[0])
    _require(k % 8 == 0 and int(w_packed.shape[1]) == k // 8,
             f"w_packed must be [N, K/8] = [{n}, {k // 8}], got {tuple(w_packed.shape)}")
    _require(group_size > 0 and k % group_size == 0,
             f"group_size {group_size} must divide K = {k}")
    _require(scales.dim() == 2 and scales.is_contiguous() and scales.dtype == torch.float16
             and tuple(scales.shape) == (n, k // group_size),
             f"scales must be a contiguous fp16 [N, K/group] = [{n}, {k // group_size}] tensor, "
             f"got {tuple(scales.shape)} {scales.dtype}")
    if out is not None:
        _require(out.dim() == 2 and tuple(out.shape) == (m, n) and out.stride(1) == 1
                 and out.dtype == torch.float16,
                 f"out must be fp16 [M, N] = [{m}, {n}] with unit column stride")
    if out is None:
        out = torch.empty((m, n), dtype=torch.float16, device=x.device)
    w4a16_matmul(x, w_packed, scales, out, m, n, k, x.stride(0), out.stride(0), group_size,
                 zero_point)
    return out
