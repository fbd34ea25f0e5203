"""The vision encoder's MFMA GEMMs (matmul_coopd.wgsl / ffn_coopd.wgsl semantics) on the GPU against numpy fp64.

X and W are f16 (W the q8_0 weight dequantised to f16 at load: f16(q·d·scale), as the reference converts its vision
weights to f16 once at load, vision.rs:122-142); products of two f16 are exact in f32, so the f32-accumulated result
sits within f32 summation error of the fp64 product of the same f16 inputs: bar rel-L2 ≤ 1e-5 (the stated bar for the
vision GEMMs is 2e-3). The FFN's f16 output: within one f16 rounding (2^-11 relative) of the fp64 value."""
import numpy as np
import pytest

import htr
from helpers import rel_l2

pytestmark = pytest.mark.gpu


def f16_weight(seed, rows, cols, scale=1.0):
    blocks = htr.synth_q8_0(seed, rows, cols)
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    w16 = (q * d * np.float32(scale)).astype(np.float16).reshape(rows, cols)
    return blocks, w16


def x16(seed, m, k, std=1.0):
    return (htr.synth_normal(seed, m * k, 0.0, std)).astype(np.float16).reshape(m, k)


@pytest.mark.parametrize("m,n,k", [(77, 128, 96), (128, 256, 64), (300, 384, 1024)])
def test_gemm_f16_small_shapes(dev, m, n, k):
    blocks, w16 = f16_weight(m + n + k, n, k)
    x = x16(7 * m + k, m, k)
    w = htr.Weight(dev, blocks, n, k, f16=True)
    xb = dev.upload(x)
    y = dev.upload(np.full((m, n), np.nan, np.float32))
    htr.gemm_f16(dev, xb, m, w, y)
    got = y.download(np.float32).reshape(m, n)
    want = x.astype(np.float64) @ w16.astype(np.float64).T
    assert rel_l2(got, want) < 1e-5
    # accumulate onto the residual
    base = htr.synth_normal(5, m * n).reshape(m, n)
    y.upload(base)
    htr.gemm_f16(dev, xb, m, w, y, acc=True)
    got = y.download(np.float32).reshape(m, n)
    assert rel_l2(got, base.astype(np.float64) + want) < 1e-5
    w.free()


def test_gemm_f16_does_not_touch_rows_past_m(dev):
    m, n, k = 130, 128, 64
    blocks, w16 = f16_weight(3, n, k)
    w = htr.Weight(dev, blocks, n, k, f16=True)
    xb = dev.upload(x16(4, m, k))
    y = dev.upload(np.full((m + 200) * n, 7.0, np.float32))
    htr.gemm_f16(dev, xb, m, w, y)
    got = y.download(np.float32)
    assert np.all(got[m * n:] == 7.0)
    w.free()


def test_ffn_f16_matches_fp64(dev):
    m, n, k = 200, 256, 128
    bg, wg16 = f16_weight(11, n, k)
    bu, wu16 = f16_weight(12, n, k)
    x = x16(13, m, k)
    wg, wu = htr.Weight(dev, bg, n, k, f16=True), htr.Weight(dev, bu, n, k, f16=True)
    xb = dev.upload(x)
    g16 = dev.alloc(m * n * 2)
    htr.gemm_ffn_f16(dev, xb, m, wg, wu, 1.0 / 64, g16)
    got = g16.download(np.float16).reshape(m, n).astype(np.float64)
    g = x.astype(np.float64) @ wg16.astype(np.float64).T
    u = x.astype(np.float64) @ wu16.astype(np.float64).T
    want = g / (1 + np.exp(-g)) * u / 64
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -10 + 1e-6)
    wg.free()
    wu.free()


def test_gemm_rejects_bad_shapes(dev):
    blocks, _ = f16_weight(1, 100, 64)
    w = htr.Weight(dev, blocks, 100, 64, f16=True)
    xb = dev.alloc(64 * 2 * 4)
    y = dev.alloc(100 * 4 * 4)
    with pytest.raises(htr.HtrError, match="multiple of 128"):
        htr.gemm_f16(dev, xb, 4, w, y)
    w.free()
    wq = htr.Weight(dev, htr.synth_q8_0(1, 128, 64), 128, 64)
    with pytest.raises(htr.HtrError, match="f16 plane"):
        htr.gemm_f16(dev, xb, 4, wq, y)
    wq.free()


@pytest.mark.parametrize("n,k", [(1024, 1024), (1024, 4096)])
def test_gemm_config4_shapes(dev, n, k):
    """config 4's GEMMs: 12100 patch rows (q / k / v / o: 1024 × 1024; down: 1024 × 4096, weights × 64)"""
    m = 12100
    scale = 64.0 if k == 4096 else 1.0
    blocks, w16 = f16_weight(n + k, n, k, scale)
    x = x16(21, m, k, 0.05 if k == 4096 else 1.0)
    w = htr.Weight(dev, blocks, n, k, f16=True, scale=scale)
    xb = dev.upload(x)
    y = dev.alloc(m * n * 4)
    htr.gemm_f16(dev, xb, m, w, y)
    got = y.download(np.float32).reshape(m, n)
    want = x.astype(np.float64) @ w16.astype(np.float64).T
    e = rel_l2(got, want)
    print(f"\n[gemm {m}x{n}x{k}] rel-L2 vs fp64 {e:.2e}")
    assert e < 1e-5
    w.free()


def test_ffn_config4_shape(dev):
    m, n, k = 12100, 4096, 1024
    bg, wg16 = f16_weight(31, n, k)
    bu, wu16 = f16_weight(32, n, k)
    x = x16(33, m, k)
    wg, wu = htr.Weight(dev, bg, n, k, f16=True), htr.Weight(dev, bu, n, k, f16=True)
    g16 = dev.alloc(m * n * 2)
    htr.gemm_ffn_f16(dev, dev.upload(x), m, wg, wu, 1.0 / 64, g16)
    got = g16.download(np.float16).reshape(m, n).astype(np.float64)
    rows = np.arange(0, m, 97)
    xr = x[rows].astype(np.float64)
    g = xr @ wg16.astype(np.float64).T
    u = xr @ wu16.astype(np.float64).T
    want = g / (1 + np.exp(-g)) * u / 64
    e = rel_l2(got[rows], want)
    print(f"\n[ffn {m}x{n}x{k}] rel-L2 vs fp64 (every 97th row) {e:.2e}")
    assert e < 1e-3
    wg.free()
    wu.free()
