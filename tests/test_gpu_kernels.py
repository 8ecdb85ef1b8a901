"""Op-level parity of the HIP kernels against the CPU oracle (run on an MI355X; marked gpu).

Shapes are the Qwen3-0.6B decode projections (out x in): Wq 2048x1024, Wk/Wv 1024x1024, Wo 1024x2048,
gate/up 3072x1024, down 1024x3072, LM head 151936x1024; fp16 activations N(0,1), fp16 weights N(0,0.02).
"""
import numpy as np
import pytest

import soc_amd as S

pytestmark = pytest.mark.gpu

GEMV_SHAPES = [(2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072), (151936, 1024)]


def _err_bound(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Bound for two fp32 sums of the same K products in different orders: ~K * 2^-24 * sum|x_i w_i|."""
    k = x.shape[-1]
    mag = np.abs(w.astype(np.float32)) @ np.abs(x.astype(np.float32)).T
    return (2.0 * k * 2.0 ** -24) * mag.T + 1e-7


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_f16_matches_oracle(gpu_ctx, oracle_mod, n, k):
    ctx = gpu_ctx
    w = S.synth_normal_f16(2, f"gemv.w.{n}x{k}", 0.02, n * k).reshape(n, k)
    x = S.synth_normal_f16(2, f"gemv.x.{k}", 1.0, k)
    dw, dx, dy = ctx.upload(w), ctx.upload(x), ctx.alloc(n * 4)
    try:
        S.gemv_f16(ctx, dw, dx, dy, n, k)
        y = ctx.download(dy, (n,), np.float32)
    finally:
        for p in (dw, dx, dy):
            ctx.free(p)
    xf = x.view(np.float16).astype(np.float32)[None, :]
    ref = oracle_mod.linear_f16(xf, w)[0]
    bound = _err_bound(xf, w.view(np.float16))[0]
    assert np.all(np.abs(y - ref) <= bound), float(np.max(np.abs(y - ref) - bound))


def test_device_f16_decode_exhaustive(gpu_ctx):
    """Every fp16 code decoded on the device equals the exact IEEE value (Float16ToFloat32, dtype.cpp:76-106)."""
    ctx = gpu_ctx
    n, k = 65536, 8
    w = np.zeros((n, k), dtype=np.uint16)
    w[:, 0] = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = np.zeros(k, dtype=np.float16)
    x[0] = 1.0
    dw, dx, dy = ctx.upload(w), ctx.upload(x.view(np.uint16)), ctx.alloc(n * 4)
    try:
        S.gemv_f16(ctx, dw, dx, dy, n, k)
        y = ctx.download(dy, (n,), np.float32)
    finally:
        for p in (dw, dx, dy):
            ctx.free(p)
    want = w[:, 0].view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    # value equality (the dot product starts from +0.0, so the -0.0 code comes back as +0.0); every other code,
    # subnormals included, must come back exactly
    assert np.array_equal(y[fin], want[fin])
    nz = fin & (want != 0)
    assert np.array_equal(y[nz].view(np.uint32), want[nz].view(np.uint32))
    assert np.all(np.isnan(y[np.isnan(want)]))
    assert np.array_equal(y[np.isinf(want)], want[np.isinf(want)])


QMM_SHAPES = [(2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072), (151936, 1024),
              # short rows: 16 lanes per row (int8 K 256, int4 K 512) and the one-lane-per-16-k kernel (K 128)
              (96, 256), (80, 512), (40, 128)]


def _qmm_inputs(n, k, bits, m):
    codes = S.synth_codes(3, f"qmm.codes.{bits}.{n}x{k}", bits, n * k)
    codes = codes.reshape(n, k if bits == 8 else k // 2)
    scales = S.synth_uniform_f16(3, f"qmm.scales.{n}x{k}", 0.005, 0.02, n * (k // 64)).reshape(n, k // 64)
    x = S.synth_normal_f16(3, f"qmm.x.{m}x{k}", 1.0, m * k).reshape(m, k)
    return codes, scales, x


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("n,k", QMM_SHAPES)
@pytest.mark.parametrize("mode,m", [("auto", 1), ("auto", 2), ("auto", 4), ("auto", 8),
                                    ("mfma", 2), ("mfma", 4), ("mfma", 8)])
def test_qmm_matches_oracle(gpu_ctx, oracle_mod, monkeypatch, bits, m, n, k, mode):
    """auto: the dot-product kernel at m = 1 and for short matrices, the MFMA kernel for tall ones at m >= 2;
    mfma: the MFMA kernel wherever it applies (it serves m >= 2)."""
    if mode == "mfma":
        monkeypatch.setenv("SOC_QMM", "mfma")
    ctx = gpu_ctx
    codes, scales, x = _qmm_inputs(n, k, bits, m)
    dc, ds, dx, dy = ctx.upload(codes), ctx.upload(scales), ctx.upload(x), ctx.alloc(m * n * 4)
    try:
        S.qmm(ctx, dx, dc, bits, ds, dy, m, n, k)
        y = ctx.download(dy, (m, n), np.float32)
    finally:
        for p in (dc, ds, dx, dy):
            ctx.free(p)
    ref = oracle_mod.qmm_group(x, codes, bits, scales, k, n)
    wdq = oracle_mod.dequant_group(codes, bits, scales, n, k)
    bound = _err_bound(x.view(np.float16).astype(np.float32), wdq)
    assert np.all(np.abs(y - ref) <= bound), float(np.max(np.abs(y - ref) - bound))


@pytest.mark.parametrize("bits", [8, 4])
def test_dequant_bit_exact(gpu_ctx, oracle_mod, bits):
    ctx = gpu_ctx
    n, k = 3072, 1024
    codes, scales, _ = _qmm_inputs(n, k, bits, 1)
    dc, ds, dw = ctx.upload(codes), ctx.upload(scales), ctx.alloc(n * k * 4)
    try:
        S.dequant(ctx, dc, bits, ds, dw, n, k)
        w = ctx.download(dw, (n, k), np.float32)
    finally:
        for p in (dc, ds, dw):
            ctx.free(p)
    ref = oracle_mod.dequant_group(codes, bits, scales, n, k)
    assert np.array_equal(w.view(np.uint32), ref.view(np.uint32))
