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
    with pytest.raises(htr.HtrError, match="multiple of 64"):
        htr.gemm_f16(dev, xb, 4, w, y)
    w.free()
    blocks, _ = f16_weight(1, 192, 64)
    wg = htr.Weight(dev, blocks, 192, 64, f16=True)
    with pytest.raises(htr.HtrError, match="multiple of 128"):
        htr.gemm_ffn_f16(dev, xb, 4, wg, wg, 1.0, y)
    wg.free()
    wq = htr.Weight(dev, htr.synth_q8_0(1, 128, 64), 128, 64)
    with pytest.raises(htr.HtrError, match="f16 plane"):
        htr.gemm_f16(dev, xb, 4, wq, y)
    wq.free()


@pytest.mark.parametrize("n,k", [(1024, 1024), (1024, 4096)])
def test_gemm_page_shapes(dev, n, k):
    """the vision page's GEMMs: 12100 patch rows (q / k / v / o: 1024 × 1024; down: 1024 × 4096, weights × 64)"""
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
    htr.gemm_f16(dev, xb, m, w, y, acc=True)  # onto itself: every element doubles exactly
    assert np.array_equal(y.download(np.float32).reshape(m, n), 2 * got)
    w.free()


def test_ffn_page_shape(dev):
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


# the tile shapes the launch picks (the largest with ≥ 128 workgroups on 256 CUs, else the one with the most):
# (1, 1024, 2048) 64 × 64; (1023, 1024, 3072) 64 × 64 (the prefill's down); (512, 4096, 1024) 128 × 128;
# (1024, 4032, 64) 128 × 128 with a last tile half past N; (50, 192, 64) 64 × 64 over 3 column tiles; (2000, 4096,
# 256) 192 × 256 (176 tiles in one round against 128 of 256 rows), its last tile row 80 rows past M; (4096, 4096, 64)
# 256 × 256 (256 tiles in one round against 352 of 192 rows in two)
@pytest.mark.parametrize("m,n,k", [(1, 1024, 2048), (1023, 1024, 3072), (512, 4096, 1024), (1024, 4032, 64),
                                   (50, 192, 64), (2000, 4096, 256), (4096, 4096, 64)])
def test_gemm_f16_tile_shapes(dev, m, n, k):
    blocks, w16 = f16_weight(m + 3 * n + k, n, k)
    x = x16(5 * m + k, m, k, 0.5)
    w = htr.Weight(dev, blocks, n, k, f16=True)
    xb = dev.upload(x)
    y = dev.upload(np.full((m + 3) * n, np.nan, np.float32))
    htr.gemm_f16(dev, xb, m, w, y)
    got = y.download(np.float32)
    want = x.astype(np.float64) @ w16.astype(np.float64).T
    e = rel_l2(got[: m * n].reshape(m, n), want)
    print(f"\n[gemm f16 {m}x{n}x{k}] rel-L2 vs fp64 {e:.2e}")
    assert e < 1e-5
    assert np.all(np.isnan(got[m * n:]))  # rows past M untouched
    # the same product accumulated onto itself: p + p is exact in f32, so every element doubles bit for bit
    htr.gemm_f16(dev, xb, m, w, y, acc=True)
    got2 = y.download(np.float32)
    assert np.array_equal(got2[: m * n], 2 * got[: m * n])
    assert np.all(np.isnan(got2[m * n:]))
    w.free()


@pytest.mark.parametrize("m,n,k", [(1023, 3072, 1024), (5, 128, 64)])
def test_ffn_f16_tile_shapes(dev, m, n, k):
    """the prefill's gate / up (128 × 128 tiles), SwiGLU fused, scale 1 (the text FFN). Per element: one f16 rounding
    of the output (2^-11 relative, bar 2^-10) plus the f32 sums' error in g and u carried through silu(g)·u
    (|∂/∂g|·δg + |silu(g)|·δu with δ = 2^-20 of the sum of the terms' magnitudes — it matters where g or u nearly
    cancels over K = 1024)"""
    bg, wg16 = f16_weight(41, n, k)
    bu, wu16 = f16_weight(42, n, k)
    x = x16(43, m, k)
    wg, wu = htr.Weight(dev, bg, n, k, f16=True), htr.Weight(dev, bu, n, k, f16=True)
    g16 = dev.alloc(m * n * 2)
    htr.gemm_ffn_f16(dev, dev.upload(x), m, wg, wu, 1.0, g16)
    got = g16.download(np.float16).reshape(m, n).astype(np.float64)
    x64, wg64, wu64 = x.astype(np.float64), wg16.astype(np.float64), wu16.astype(np.float64)
    g, u = x64 @ wg64.T, x64 @ wu64.T
    sig = 1 / (1 + np.exp(-g))
    want = g * sig * u
    dg, du = 2.0 ** -20 * (np.abs(x64) @ np.abs(wg64).T), 2.0 ** -20 * (np.abs(x64) @ np.abs(wu64).T)
    bound = np.abs(want) * 2.0 ** -10 + np.abs(sig * (1 + g * (1 - sig)) * u) * dg + np.abs(g * sig) * du + 1e-7
    err = np.abs(got - want)
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    assert np.all(err <= bound), (f"{int(np.sum(err > bound))} elements; worst {worst}: got {got[worst]}, "
                                  f"want {want[worst]}, g {g[worst]}, u {u[worst]}, bound {bound[worst]}")
    wg.free()
    wu.free()


@pytest.mark.parametrize("m,n,k", [(7, 96, 256), (70, 100, 96), (130, 64, 32), (64, 192, 1024)])
def test_matmul_q8_0_on_both_compute_paths(dev, m, n, k):
    """Batch::matmul with a q8_0 weight (gpu.rs:1963-2014) on the F32 path (exact dequant, f32 sums) and the f16 path
    (X and q·d rounded to f16, f32 sums) against the oracle's restatement of each (bar 1e-5: f32 summation order). Each
    result must also sit far closer to its own path's oracle than to the other path's — a dropped or extra rounding
    fails (the two paths differ by about 3e-4 here)."""
    import oracle as orc

    blocks = htr.synth_q8_0(m + n + k, n, k)
    x = htr.synth_normal(3 * m + k, m * k).reshape(m, k)
    base = htr.synth_normal(9, m * n).reshape(m, n)
    w = htr.Weight(dev, blocks, n, k)
    xb = dev.upload(x)
    want = {p: orc.matmul_q8_0(x, blocks, n, r16=p == htr.COMPUTE_F16) for p in (htr.COMPUTE_F32, htr.COMPUTE_F16)}
    keep = dev.compute
    try:
        for path in (htr.COMPUTE_F32, htr.COMPUTE_F16):
            other = htr.COMPUTE_F16 if path == htr.COMPUTE_F32 else htr.COMPUTE_F32
            dev.compute = path
            y = dev.upload(base)
            htr.matmul_q8_0(dev, xb, m, w, y, acc=True)
            got = y.download(np.float32).reshape(m, n) - base
            e, e_other = rel_l2(got, want[path]), rel_l2(got, want[other])
            print(f"\n[matmul q8_0 {m}x{n}x{k} path {path}] vs oracle {e:.2e}, vs the other path {e_other:.2e}")
            assert e < 1e-5
            assert e_other > 20 * e
    finally:
        dev.compute = keep
    w.free()


def test_compute_path_setting(dev):
    keep = dev.compute
    assert keep in (htr.COMPUTE_F32, htr.COMPUTE_F16)
    with pytest.raises(htr.HtrError, match="compute path"):
        dev.compute = 7
    assert dev.compute == keep


@pytest.mark.parametrize("m,n,k", [(1023, 1024, 2048), (1023, 1024, 3072), (40, 256, 1024)])
def test_split_k_is_exact_and_deterministic(dev, m, n, k):
    """prompt-sized GEMMs with few tiles split K over workgroups; the last of a tile's splits adds the partials in split
    order, so repeated runs (any arrival order) are bit-identical; accumulate mode onto a residual, against fp64"""
    blocks, w16 = f16_weight(m * 3 + n + k, n, k)
    x = x16(m + 11 * k, m, k, 0.5)
    w = htr.Weight(dev, blocks, n, k, f16=True)
    xb = dev.upload(x)
    base = htr.synth_normal(m + n, m * n).reshape(m, n)
    outs = []
    for _ in range(3):
        y = dev.upload(base)
        htr.gemm_f16(dev, xb, m, w, y, acc=True)
        outs.append(y.download(np.float32).reshape(m, n))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    want = base.astype(np.float64) + x.astype(np.float64) @ w16.astype(np.float64).T
    e = rel_l2(outs[0], want)
    print(f"\n[split-K {m}x{n}x{k}] rel-L2 vs fp64 {e:.2e}")
    assert e < 1e-5
    w.free()
