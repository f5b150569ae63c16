"""Quantised matmul parity on the GPU.

W4A16: rel error max|Y - ref| / max|ref| <= 1e-2 against
the float64 oracle at M in {1, 16, 256}, K = 4096, N = 11008, plus the int4
known-answer fixture (exact), ragged shapes, other group sizes / zero
points and closed forms.  W8A16 / scaled: the reference tests' inputs and
tolerance (tests/test_quantized_matmul.py:316-447, :531-580).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import neso_amd
from oracle import inputs as I
from oracle import qmatmul as Q

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def gpu_w4(x, words, scales, group=32, zero=8):
    y = neso_amd.w4a16_linear(x.to(DEV), torch.as_tensor(words).to(DEV), scales.to(DEV),
                              group_size=group, zero_point=zero)
    torch.cuda.synchronize()
    return y.cpu()


@pytest.mark.parametrize("cfg", I.QMM_CONFIGS, ids=lambda c: f"M{c['M']}")
def test_baseline_config5(gpu, cfg):
    x, codes, scales = I.qmatmul_inputs(**cfg, seed=0)
    words = Q.pack_int4(codes.numpy())
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy(),
                         dtype=np.float64 if cfg["M"] <= 16 else np.float32)
    err = Q.rel_err(y.float().numpy(), ref)
    assert err <= 1e-2, err
    assert err <= 2e-3, err  # fp16 output rounding is the only expected error


def test_int4_kat_exact(gpu, golden_dir):
    z = np.load(golden_dir / "qmm_int4_kat.npz")
    x = torch.from_numpy(z["x"]).half()
    s = torch.from_numpy(z["scales"]).half()
    for m in (1, 3, 8):  # GEMV and MFMA regimes
        y = gpu_w4(x[:m], z["words"], s)
        assert np.array_equal(y.float().numpy(), z["expected"][:m]), m


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 17, 33, 64, 100])
@pytest.mark.parametrize("n,k", [(1, 32), (7, 96), (100, 4096), (129, 256)])
def test_ragged(gpu, m, n, k):
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=m * n + k)
    words = Q.pack_int4(codes.numpy())
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("m", [3, 16])
@pytest.mark.parametrize("n,k", [(4100, 4096), (13000, 2048), (20000, 2048)])
def test_skinny_tiles_per_workgroup(gpu, m, n, k):
    """The X-in-LDS skinny kernel gives each workgroup T = ceil(tiles / CUs)
    16-row tiles, at most 4: N = 4100 / 13000 / 20000 take T = 2, 4 and 4
    with more workgroups than CUs on 256 CUs (N = 11008 takes T = 3 in the
    config-5 test).  Checked against the float64 oracle."""
    import json
    from neso_amd import _lib
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=m + n)
    words = Q.pack_int4(codes.numpy())
    lib = _lib.load()
    xd, wd, sd = x.to(DEV), torch.as_tensor(words).to(DEV), scales.to(DEV)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert lib.neso_plan_begin(cus) == _lib.NESO_OK
    try:
        assert lib.neso_w4a16_matmul(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), y.data_ptr(),
                                     m, n, k, k, n, 32, 8, None) == _lib.NESO_OK
    finally:
        plan = json.loads(lib.neso_plan_end().decode())["launches"]
    tiles = (n + 15) // 16
    t = min(4, -(-tiles // cus))
    assert [(p["device_kernel"], p["template_args"][1], p["grid"][0]) for p in plan] == [
        ("w4a16_skinny_lds_kernel", t, -(-tiles // t))], plan
    out = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy(), dtype=np.float64)
    assert Q.rel_err(out.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("m", [1, 3])
@pytest.mark.parametrize("k", [2048, 2080, 2112, 4064, 4096, 6144])
@pytest.mark.parametrize("n", [1, 65, 300])
def test_gemv_chunks_per_lane(gpu, m, k, n):
    """GEMV with one, two and four 32-code chunks per lane.  With two chunks
    and an even chunk count (K = 2112, 4096) the row's scales arrive as one
    4-byte load per lane and are handed between lanes; an odd count (2080,
    4064) keeps one 2-byte load per chunk.  Distinct per-(row, group) scales
    catch a scale delivered to the wrong lane."""
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=k + n + m)
    words = Q.pack_int4(codes.numpy())
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("gemv_max_m", ["0", "4"])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", [(300, 4096), (129, 2080)])
def test_small_m_both_regimes(gpu, monkeypatch, gemv_max_m, m, n, k):
    """M = 1..4 through the GEMV kernel (NESO_AMD_W4_GEMV_MAX_M = 4) and
    through the MFMA kernels (= 0); by default M <= 2 takes the GEMV."""
    monkeypatch.setenv("NESO_AMD_W4_GEMV_MAX_M", gemv_max_m)
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=m + n + k)
    words = Q.pack_int4(codes.numpy())
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("env,m,n,kernel,targs", [
    ({}, 32, 300, "w4a16_tile_gemm_kernel", [8, 1, 1]),
    ({}, 16, 300, "w4a16_skinny_lds_kernel", None),
    ({"NESO_AMD_W4_TILE_GEMM": "0"}, 24, 300, "w4a16_skinny_kernel", None),
    ({}, 32, 8192, "w4a16_tile_gemm_kernel", [8, 1, 1]),
    ({"NESO_AMD_W4_TILE_GEMM": "7"}, 64, 11008, "w4a16_tile_gemm_kernel", [8, 1, 1]),
    ({}, 33, 11008, "w4a16_tile_gemm_kernel", [4, 2, 2]),
    ({}, 33, 1000, "w4a16_tile_gemm_kernel", [8, 1, 1]),
    ({"NESO_AMD_W4_SKINNY_MAX_M": "64"}, 48, 300, "w4a16_skinny_kernel", None),
    ({"NESO_AMD_W4_SKINNY_MAX_M": "64"}, 64, 300, "w4a16_skinny_kernel", None),
    ({}, 64, 11008, "w4a16_tile_gemm_kernel", [4, 2, 2]),
    ({}, 64, 4096, "w4a16_tile_gemm_kernel", [8, 1, 1]),
    ({"NESO_AMD_W4_TILE_GEMM": "6"}, 24, 300, "w4a16_tile_gemm_kernel", [4, 2, 1]),
    ({"NESO_AMD_W4_TILE_GEMM": "0"}, 64, 300, "w4a16_gemm_kernel", None),
    ({"NESO_AMD_W4_TILE_GEMM": "3"}, 64, 300, "w4a16_tile_gemm_kernel", [2, 2, 4]),
    ({"NESO_AMD_W4_SKINNY_MAX_M": "16", "NESO_AMD_W4_TILE_GEMM": "6"}, 24, 300, "w4a16_tile_gemm_kernel", [4, 2, 1]),
    ({}, 96, 11008, "w4a16_tile_gemm_kernel", [4, 2, 4]),
    ({}, 128, 11008, "w4a16_tile_gemm_kernel", [4, 2, 4]),
    ({}, 128, 4096, "w4a16_tile_gemm_kernel", [4, 2, 1]),
    ({}, 129, 11008, "w4a16_tile_gemm_kernel", [2, 4, 4]),
    ({}, 256, 4096, "w4a16_tile_gemm_kernel", [4, 2, 2]),
    ({}, 256, 8192, "w4a16_tile_gemm_kernel", [4, 2, 4]),
    ({"NESO_AMD_W4_WIDE_TILE_MIN_M": "192"}, 160, 11008, "w4a16_tile_gemm_kernel", [2, 2, 4]),
    ({}, 160, 11008, "w4a16_tile_gemm_kernel", [2, 4, 4]),
    ({}, 1024, 4096, "w4a16_tile_gemm_kernel", [2, 4, 4]),
    ({}, 1200, 4096, "w4a16_tile_gemm_kernel", [1, 4, 4]),
    ({}, 128, 32768, "w4a16_tile_gemm_kernel", [2, 4, 4]),
    ({}, 100, 40960, "w4a16_tile_gemm_kernel", [2, 2, 4]),
    ({"NESO_AMD_W4_WIDE_TILE_MIN_M": "129"}, 128, 32768, "w4a16_tile_gemm_kernel", [2, 2, 4]),
])
def test_route_thresholds(gpu, monkeypatch, env, m, n, kernel, targs):
    """The kernels on each side of the skinny / tile GEMM threshold (M = 16
    / 17) and of the tile GEMM's tile shapes, for a 256-CU part: the finest
    of 32 x 32, 32 x 64, 64 x 64 and 128 x 64 tiles whose grid fits on the
    CUs, else 128 x 128 from M = 65 while those tiles fit (from M = 129
    with one K-group beyond), 128 x 64 with two K-groups for M = 65..128,
    64 x 64 from M = 33; the NESO_AMD_W4_SKINNY_MAX_M, NESO_AMD_W4_TILE_GEMM and
    NESO_AMD_W4_WIDE_TILE_MIN_M overrides, and the skinny and 128 x 64
    kernels with the tile GEMM turned off."""
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    k = 4096 if n <= 1000 else 256
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=m + n + k)
    words = Q.pack_int4(codes.numpy())
    xd, wd, sd = x.to(DEV), torch.as_tensor(words).to(DEV), scales.to(DEV)
    yd = torch.empty(m, n, dtype=torch.float16, device=DEV)
    plan = neso_amd.launch_plan("w4a16_matmul", xd, wd, sd, yd, m, n, k, k, n, 32, 8, cu_count=256)
    assert [p["device_kernel"] for p in plan] == [kernel], plan
    if targs is not None:
        assert plan[0]["template_args"] == targs, plan
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("env,m,n,kernel", [
    ({}, 16, 4096, "w4a16_tile_gemm_kernel"),
    ({}, 1, 1000, "w4a16_tile_gemm_kernel"),
    ({}, 3, 1000, "w4a16_tile_gemm_kernel"),
    ({}, 16, 11008, "w4a16_skinny_kernel"),
    ({"NESO_AMD_W4_SKINNY_MAX_M": "16"}, 16, 4096, "w4a16_skinny_kernel"),
    ({"NESO_AMD_W4_TILE_GEMM": "0"}, 8, 1000, "w4a16_skinny_kernel"),
])
def test_long_k_small_m_route(gpu, monkeypatch, env, m, n, kernel):
    """Up to M = 16 with K past the X-in-LDS kernel's limit (and the
    GEMV's, for M = 1): the 32 x 32 tile GEMM where its grid fits on a
    256-CU part, the split-K skinny kernel where it does not, when forced,
    or with the tile GEMM off."""
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    k = 11008
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=m + n)
    words = Q.pack_int4(codes.numpy())
    xd, wd, sd = x.to(DEV), torch.as_tensor(words).to(DEV), scales.to(DEV)
    yd = torch.empty(m, n, dtype=torch.float16, device=DEV)
    plan = neso_amd.launch_plan("w4a16_matmul", xd, wd, sd, yd, m, n, k, k, n, 32, 8, cu_count=256)
    assert [p["device_kernel"] for p in plan] == [kernel], plan
    if kernel == "w4a16_tile_gemm_kernel":
        assert plan[0]["template_args"] == [8, 1, 1], plan
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy(), dtype=np.float64)
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("m,targs", [(17, [4, 2, 1]), (32, [4, 2, 1]), (33, [4, 2, 2]), (64, [4, 2, 2]),
                                    (65, [4, 2, 4])])
def test_small_tile_route(gpu, m, targs):
    """N = 11008 gives the 32 x 64 tiles a grid that fills more than half
    the CUs, so M = 17..32 takes the tile GEMM; 33..64 takes 64 x 64 tiles
    and 65 up 128 x 64 ones."""
    n, k = 11008, 256
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=m)
    words = Q.pack_int4(codes.numpy())
    xd, wd, sd = x.to(DEV), torch.as_tensor(words).to(DEV), scales.to(DEV)
    yd = torch.empty(m, n, dtype=torch.float16, device=DEV)
    plan = neso_amd.launch_plan("w4a16_matmul", xd, wd, sd, yd, m, n, k, k, n, 32, 8, cu_count=256)
    assert [(p["device_kernel"], p["template_args"]) for p in plan] == [("w4a16_tile_gemm_kernel", targs)], plan
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("group,zero", [(64, 8), (128, 7), (32, 0), (4096, 15)])
@pytest.mark.parametrize("m", [1, 16])
def test_group_and_zero_point(gpu, group, zero, m):
    x, codes, scales = I.qmatmul_inputs(m, 4096, 300, group=group, seed=group + zero)
    words = Q.pack_int4(codes.numpy())
    y = gpu_w4(x, words, scales, group, zero)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy(), group, zero)
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("m", [1, 16, 256])
def test_zero_point_codes_give_zero(gpu, m):
    """Codes equal to the zero point dequantise to 0, so Y = 0.

    The MFMA regime subtracts the zero point per element (exact zeros).  The
    GEMV regime (M <= 2) folds it into a per-chunk correction computed from
    X, so it returns 0 up to fp32 rounding: |Y| <= 1e-3 here, against
    typical |Y| ~ 4 for these inputs with random codes.
    """
    x, _, scales = I.qmatmul_inputs(m, 4096, 512, seed=1)
    eights = Q.pack_int4(np.full((512, 4096), 8, np.uint8))
    y = gpu_w4(x, eights, scales)
    if m <= 2:
        assert y.float().abs().max().item() <= 1e-3
    else:
        assert torch.count_nonzero(y).item() == 0


@pytest.mark.parametrize("amp", [200.0, 1000.0])
@pytest.mark.parametrize("at_zero", [False, True], ids=["random_codes", "codes_at_zero"])
@pytest.mark.parametrize("m", [1, 2, 16])
def test_outlier_activations(gpu, amp, at_zero, m):
    """A few activation channels of size |x| = amp among N(0, 1) ones, as in
    LLM hidden states.  The GEMV (M <= 2) accumulates (1024 + c) x and
    (1024 + 16 c) x in fp32 and subtracts the zero point's share once per
    chunk, so an outlier's terms reach ~1264 |x| before they cancel.  With
    the outliers' codes at the zero point the cancellation is exact in real
    arithmetic and only rounding is left, the worst case for the fold.

    Bars: max|err| / max|ref| <= 2e-3, and per element half an fp16 ulp of
    max(|ref|, |Y|) plus 2^-20 * sum_g s_g * 1264 * sum_{k in g} |x_k| (the fp32 rounding
    of at most 16 accumulations per chunk sum, each term at most 1264 |x|).
    """
    k, n = 4096, 512
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=int(amp) + m)
    rs = np.random.RandomState(m)
    idx = rs.choice(k, 6, replace=False)
    x[:, idx] = torch.from_numpy(amp * np.sign(rs.randn(m, 6))).half()
    codes = codes.numpy()
    if at_zero:
        codes[:, idx] = 8
    words = Q.pack_int4(codes)
    y = gpu_w4(x, words, scales).double().numpy()
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy(), dtype=np.float64)
    assert Q.rel_err(y, ref) <= 2e-3
    ax = np.abs(x.double().numpy()).reshape(m, k // 32, 32).sum(-1)  # [M][groups]
    fold = 2.0 ** -20 * 1264 * ax @ scales.double().numpy().T      # [M][N]
    top = np.maximum(np.maximum(np.abs(ref), np.abs(y)), 2.0 ** -14)
    half_ulp = np.exp2(np.floor(np.log2(top)) - 11)
    assert (np.abs(y - ref) <= half_ulp + fold).all(), np.abs(y - ref).max()


@pytest.mark.parametrize("m,tile", [(3, None), (24, "6"), (48, None), (48, "0"), (200, None), (300, "1"),
                                    (300, "2"), (300, "3"), (300, "4"), (300, "5"), (300, "6"), (300, "7")])
def test_strided_output(gpu, monkeypatch, m, tile):
    """Row strides of X and Y wider than K and N on every regime (GEMV, the
    128 x 64 kernel, the tile GEMM in each of its forms): the padding
    columns of Y keep their contents."""
    if tile:
        monkeypatch.setenv("NESO_AMD_W4_TILE_GEMM", tile)
        monkeypatch.setenv("NESO_AMD_W4_SKINNY_MAX_M", "0")
    n, k = 200, 512
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=9)
    words = torch.from_numpy(Q.pack_int4(codes.numpy())).to(DEV)
    xp = torch.zeros(m, k + 64, dtype=torch.float16, device=DEV)
    xp[:, :k] = x.to(DEV)
    y = torch.full((m, n + 8), 5.0, dtype=torch.float16, device=DEV)
    neso_amd.w4a16_matmul(xp, words, scales.to(DEV), y, m, n, k, k + 64, n + 8)
    torch.cuda.synchronize()
    ref = Q.w4a16_matmul(x.numpy(), words.cpu().numpy(), scales.numpy())
    assert Q.rel_err(y[:, :n].float().cpu().numpy(), ref) <= 2e-3
    assert torch.all(y[:, n:].cpu() == 5.0)


def _w8(kind, m, n, k):
    a, b, scale = I.reference_quant_lists(m, n, k, kind)
    A_ = torch.tensor(a).reshape(m, k).half().to(DEV)
    B_ = torch.tensor(b, dtype=torch.int8).reshape(k, n).to(DEV)
    C_ = torch.empty(m, n, dtype=torch.float32, device=DEV)
    if scale is None:
        neso_amd.launch("w8a16_matmul", A_, B_, C_, k, k, n, n, M=m, N=n)
    else:
        S_ = torch.tensor(scale).half().to(DEV)
        neso_amd.launch("w8a16_scaled_matmul", A_, B_, C_, S_, k, k, n, n, M=m, N=n)
    torch.cuda.synchronize()
    return C_.cpu().numpy(), a, b, scale


@pytest.mark.parametrize("kind", ["w8a16", "w4a16", "scaled"])
@pytest.mark.parametrize("mnk", [(32, 32, 32), (64, 64, 64), (64, 64, 128), (128, 128, 128),
                                 (128, 128, 256), (256, 256, 256)])
def test_w8a16_reference_configs(gpu, golden_dir, kind, mnk):
    m, n, k = mnk
    c, a, b, scale = _w8(kind, m, n, k)
    A_ = np.array(a, np.float64).reshape(m, k)
    B_ = np.array(b, np.float64).reshape(k, n)
    ref = Q.w8a16_scaled_matmul(A_, B_, scale) if scale else Q.w8a16_matmul(A_, B_)
    assert Q.rel_err(c, ref) < 1e-2  # reference tolerance (:354-358)
    # Tighter: against the same product on the fp16-rounded activations.
    A16 = np.array(a, np.float16).astype(np.float64).reshape(m, k)
    s16 = np.array(scale, np.float16).astype(np.float64) if scale else None
    ref16 = Q.w8a16_scaled_matmul(A16, B_, s16) if scale else Q.w8a16_matmul(A16, B_)
    assert Q.rel_err(c, ref16) < 1e-4  # fp32 accumulation order only
    fixture = golden_dir / f"qmm_{ {'w4a16': 'w4i8'}.get(kind, kind)}_{m}x{n}x{k}.npz"
    if fixture.exists():
        assert Q.rel_err(c.reshape(-1), np.load(fixture)["expected"]) < 1e-2


@pytest.mark.parametrize("scaled", [False, True])
@pytest.mark.parametrize("m,n,k", [(300, 136, 264), (1, 8, 8), (129, 256, 4096), (77, 100, 96),
                                   (5, 13, 7)])
def test_w8a16_tiled_and_fallback(gpu, m, n, k, scaled):
    """The tiled kernel (N, K, strides multiples of 8) on ragged tiles, and the
    per-element fallback (n = 100, 13; k = 7), against the float64 oracle on
    the fp16-rounded activations."""
    g = torch.Generator().manual_seed(m * 7 + n + k)
    a = torch.randn(m, k, generator=g).half()
    b = torch.randint(-128, 128, (k, n), generator=g, dtype=torch.int8)
    s = (torch.rand(n, generator=g) * 0.1 + 0.001).half()
    c = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    if scaled:
        neso_amd.w8a16_scaled_matmul(a.to(DEV), b.to(DEV), c, s.to(DEV), k, k, n, n, M=m, N=n)
        ref = Q.w8a16_scaled_matmul(a.double().numpy(), b.double().numpy(), s.double().numpy())
    else:
        neso_amd.w8a16_matmul(a.to(DEV), b.to(DEV), c, k, k, n, n, M=m, N=n)
        ref = Q.w8a16_matmul(a.double().numpy(), b.double().numpy())
    torch.cuda.synchronize()
    assert Q.rel_err(c.cpu().numpy(), ref) < 1e-4


@pytest.mark.parametrize("scaled", [False, True])
@pytest.mark.parametrize("m,n,k", [(4000, 4104, 520), (1300, 11008, 256)])
def test_w8a16_large_tiles(gpu, scaled, m, n, k):
    """The 256 x 256-tile kernel (chosen once its tiles give every CU a
    workgroup) on ragged M (4000 = 15.6 tiles), N with a 16-byte B piece
    straddling the end (4104 % 16 = 8) and K not a multiple of the 64-wide
    K-step; and on 6 x 43 tiles, whose tile order (groups of four m-tiles)
    ends in a group of two.  Against the float64 oracle on the fp16-rounded
    activations."""
    import json
    from neso_amd import _lib
    g = torch.Generator().manual_seed(17)
    a = torch.randn(m, k, generator=g).half()
    b = torch.randint(-128, 128, (k, n), generator=g, dtype=torch.int8)
    s = (torch.rand(n, generator=g) * 0.1 + 0.001).half()
    c = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
    ad, bd, sd = a.to(DEV), b.to(DEV), s.to(DEV)
    lib = _lib.load()
    args = [ad.data_ptr(), bd.data_ptr(), c.data_ptr()] + ([sd.data_ptr()] if scaled else []) + \
        [k, k, n, n, m, n, None]
    fn = lib.neso_w8a16_scaled_matmul if scaled else lib.neso_w8a16_matmul
    assert lib.neso_plan_begin(0) == _lib.NESO_OK
    try:
        assert fn(*args) == _lib.NESO_OK
    finally:
        plan = json.loads(lib.neso_plan_end().decode())["launches"]
    if torch.cuda.get_device_properties(0).multi_processor_count <= 16 * 17:
        assert plan[0]["template_args"] == [256], plan
    if scaled:
        neso_amd.w8a16_scaled_matmul(ad, bd, c, sd, k, k, n, n, M=m, N=n)
        ref = Q.w8a16_scaled_matmul(a.double().numpy(), b.double().numpy(), s.double().numpy())
    else:
        neso_amd.w8a16_matmul(ad, bd, c, k, k, n, n, M=m, N=n)
        ref = Q.w8a16_matmul(a.double().numpy(), b.double().numpy())
    torch.cuda.synchronize()
    assert torch.isfinite(c).all()
    assert Q.rel_err(c.cpu().numpy(), ref) < 1e-4


@pytest.mark.parametrize("sync", ["0", "1"])
@pytest.mark.parametrize("kgroups", ["1", "2", "3", "4", "5", "6", "7"])
@pytest.mark.parametrize("m,n,k", [(128, 11008, 4096), (200, 300, 4096), (256, 1000, 4128),
                                   (300, 129, 96), (640, 256, 1024), (96, 200, 11008)])
def test_tile_gemm(gpu, monkeypatch, kgroups, sync, m, n, k):
    """The tile GEMM in its seven forms (128 x 128 tiles with one or two
    K-groups, 128 x 64 with two or four, 64 x 64 and 32 x 64 with four,
    32 x 32 with eight),
    each with workgroup barriers and with per-group arrival counters:
    ragged M and N tiles, K not a multiple of its 64-code step, a K
    shorter than one step per group, and a long K loop."""
    monkeypatch.setenv("NESO_AMD_W4_TILE_GEMM", kgroups)
    monkeypatch.setenv("NESO_AMD_W4_TILE_SYNC", sync)
    x, codes, scales = I.qmatmul_inputs(m, k, n, seed=m + n + k)
    words = Q.pack_int4(codes.numpy())
    y = gpu_w4(x, words, scales)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3


def test_tile_one_wave_groups_repeat(gpu, monkeypatch):
    """The 32 x 32 form's K-groups are one wave each and order their LDS
    double buffer with a wave-level fence only: five launches on the same
    inputs (22 steps per group) give identical results, within the
    oracle's bound."""
    monkeypatch.setenv("NESO_AMD_W4_TILE_GEMM", "7")
    x, codes, scales = I.qmatmul_inputs(64, 11008, 1000, seed=7)
    words = Q.pack_int4(codes.numpy())
    xd, wd, sd = x.to(DEV), torch.as_tensor(words).to(DEV), scales.to(DEV)
    ys = [neso_amd.w4a16_linear(xd, wd, sd, group_size=32, zero_point=8) for _ in range(5)]
    torch.cuda.synchronize()
    assert all(torch.equal(ys[0], y) for y in ys[1:])
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(ys[0].float().cpu().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("kgroups", ["2", "3", "4", "5", "6"])
def test_tile_sync_identical(gpu, monkeypatch, kgroups):
    """Per-group arrival counters and workgroup barriers order the same
    LDS traffic, so the two syncs give bit-identical results."""
    monkeypatch.setenv("NESO_AMD_W4_TILE_GEMM", kgroups)
    x, codes, scales = I.qmatmul_inputs(200, 11008, 300, seed=int(kgroups))
    words = Q.pack_int4(codes.numpy())
    ys = []
    for sync in ("0", "1"):
        monkeypatch.setenv("NESO_AMD_W4_TILE_SYNC", sync)
        ys.append(gpu_w4(x, words, scales))
    assert torch.equal(ys[0], ys[1])
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy())
    assert Q.rel_err(ys[1].float().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("sync", ["0", "1"])
@pytest.mark.parametrize("kgroups", ["1", "2", "3", "4", "5", "6", "7"])
@pytest.mark.parametrize("group,zero", [(64, 8), (128, 7), (32, 0), (4096, 15)])
def test_tile_gemm_groups(gpu, monkeypatch, kgroups, sync, group, zero):
    monkeypatch.setenv("NESO_AMD_W4_TILE_GEMM", kgroups)
    monkeypatch.setenv("NESO_AMD_W4_TILE_SYNC", sync)
    x, codes, scales = I.qmatmul_inputs(256, 4096, 300, group=group, seed=group + zero)
    words = Q.pack_int4(codes.numpy())
    y = gpu_w4(x, words, scales, group, zero)
    ref = Q.w4a16_matmul(x.numpy(), words, scales.numpy(), group, zero)
    assert Q.rel_err(y.float().numpy(), ref) <= 2e-3
