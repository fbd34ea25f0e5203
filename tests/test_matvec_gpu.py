"""q8_0 dequant-matvec family on the GPU against the oracle and the fp64 dequantised reference.

Tolerances: rel-L2 ≤ 1e-3 against fp64 (the stated bar for float outputs); on the reference tests' own shapes also
their bars (1e-4 abs, text.rs:726; rel 1e-3, text.rs:883)."""
import numpy as np
import pytest

import htr
import oracle as orc
from helpers import rel_l2

pytestmark = pytest.mark.gpu


def _np_deq(blocks, rows, cols):
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float64)
    return (b[:, 2:].view(np.int8).astype(np.float64) * d).reshape(rows, cols)


def test_matvec_reference_shape(dev):
    """text.rs:707-741: 37 rows × 96 (3 blocks), plain and accumulating"""
    n, k = 37, 96
    g = orc.Lcg(11)
    blocks, _ = orc.q8_0_quantize(g.f32(n * k, 0.3))
    x = g.f32(k)
    base = g.f32(n)
    w = htr.Weight(dev, blocks, n, k)
    xb = dev.upload(x)
    for acc in (False, True):
        yb = dev.upload(base)
        htr.matvec_q8_0(dev, w, xb, yb, acc=acc)
        y = yb.download(np.float32)
        want = orc.matvec_q8_0(blocks, n, k, x, base, acc)
        assert np.abs(y - want).max() < 1e-4, acc
        yb.free()


def test_fused_matvecs_reference_shapes(dev):
    """text.rs:864-925: dmv_norm 37 rows, dmv_qkv 32 / 16 / 16 rows, dmv_ffn 37 rows, K = 96"""
    k, eps = 96, 1e-6
    g = orc.Lcg(41)
    x = g.f32(k, 2.0)
    nw = g.f32(k)
    xb, nwb = dev.upload(x), dev.upload(nw)
    close = lambda got, want: np.all(np.abs(got - want) < 1e-3 * (1 + np.abs(want)))

    def mat(rows):
        b, _ = orc.q8_0_quantize(g.f32(rows * k, 0.3))
        return b, htr.Weight(dev, b, rows, k)

    b, w = mat(37)
    y = dev.alloc(37 * 4)
    htr.matvec_q8_0(dev, w, xb, y, norm_w=nwb, eps=eps)
    assert close(y.download(np.float32), orc.dmv(b, 37, k, x, nw, eps))
    (bq, wq), (bk, wk), (bv, wv) = mat(32), mat(16), mat(16)
    qkv = dev.alloc(64 * 4)
    htr.matvec_qkv(dev, wq, wk, wv, xb, nwb, eps, qkv)
    assert close(qkv.download(np.float32), orc.dmv_qkv(bq, bk, bv, 32, 16, k, x, nw, eps))
    (bg, wg), (bu, wu) = mat(37), mat(37)
    gb = dev.alloc(37 * 4)
    htr.matvec_ffn(dev, wg, wu, xb, nwb, eps, gb)
    assert close(gb.download(np.float32), orc.dmv_ffn(bg, bu, 37, k, x, nw, eps))


@pytest.mark.parametrize("rows,k", [(3072, 1024), (1024, 2048), (1024, 3072), (4096, 1024), (151936, 1024)])
def test_matvec_decoder_shapes_vs_fp64(dev, rows, k):
    """the W [3072 × 1024] projection and every decoder projection shape, including the 151936-row LM head"""
    blocks = htr.synth_q8_0(100 + rows + k, rows, k)
    x = htr.synth_normal(7, k)
    w = htr.Weight(dev, blocks, rows, k)
    xb, yb = dev.upload(x), dev.alloc(rows * 4)
    htr.matvec_q8_0(dev, w, xb, yb)
    y = yb.download(np.float32)
    assert rel_l2(y, orc.matvec_f64(blocks, rows, k, x)) < 1e-3
    # and against the f32 restatement of dmv.wgsl: same inputs, f32 sums in another order
    assert rel_l2(y, orc.dmv(blocks, rows, k, x)) < 1e-5
    w.free()


def test_lm_head_with_norm_vs_fp64(dev):
    rows, k, eps = 151936, 1024, 1e-6
    blocks = htr.synth_q8_0(5, rows, k)
    x = htr.synth_normal(6, k, 0.0, 3.0)
    nw = htr.synth_normal(8, k, 1.0, 0.02)
    w = htr.Weight(dev, blocks, rows, k)
    yb = dev.alloc(rows * 4)
    htr.matvec_q8_0(dev, w, dev.upload(x), yb, norm_w=dev.upload(nw), eps=eps)
    y = yb.download(np.float32)
    xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps) * nw
    assert rel_l2(y, _np_deq(blocks, rows, k) @ xn) < 1e-3
    assert rel_l2(y, orc.dmv(blocks, rows, k, x, nw, eps)) < 1e-5
    w.free()


def test_matvec_many_equals_single(dev):
    """the rotation entry point computes exactly what the single launches compute (same per-row order)"""
    rows, k, n = 3072, 1024, 6
    ws = [htr.Weight(dev, htr.synth_q8_0(200 + i, rows, k), rows, k) for i in range(n)]
    xb = dev.upload(htr.synth_normal(9, k))
    ym = dev.alloc(n * rows * 4)
    htr.matvec_q8_0_many(dev, ws, xb, ym)
    got = ym.download(np.float32).reshape(n, rows)
    for i, w in enumerate(ws):
        yb = dev.alloc(rows * 4)
        htr.matvec_q8_0(dev, w, xb, yb)
        assert np.array_equal(got[i], yb.download(np.float32)), i
        w.free()
