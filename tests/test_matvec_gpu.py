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


def _dmv_full_name(dev, rows, k, mode):
    """the instance launch_dmv picks for a decoder shape: one workgroup a CU, rows / (4·CUs) rows a wave"""
    n_cu = dev.info()[1]
    if rows % (4 * n_cu) or k % 1024 or rows // (4 * n_cu) > 4:
        return None
    return f"k_dmv_full<{rows // (4 * n_cu)},{k // 1024},{mode}>"


def test_decode_qkv_instance(dev):
    """the decode step's Q / K / V matvec as the 28-layer decoder runs it (text.rs:638, dmv_qkv.wgsl): q 2048, k 1024,
    v 1024 rows × K 1024 with attn_norm fused — the k_dmv_full QKV instance (4 rows a wave on 256 CUs) — against the
    oracle's restatement (≤ 1e-5, f32 in another order) and the fp64 closed form (≤ 1e-3); bars of text.rs:864-905"""
    k, eps, qd, kvd = 1024, 1e-6, 2048, 1024
    bq, bk, bv = (htr.synth_q8_0(300 + i, r, k) for i, r in enumerate((qd, kvd, kvd)))
    x = htr.synth_normal(31, k, 0.0, 2.0)
    nw = htr.synth_normal(32, k, 1.0, 0.02)
    ws = [htr.Weight(dev, b, r, k) for b, r in ((bq, qd), (bk, kvd), (bv, kvd))]
    y = dev.alloc((qd + 2 * kvd) * 4)
    htr.matvec_qkv(dev, *ws, dev.upload(x), dev.upload(nw), eps, y)
    want_name = _dmv_full_name(dev, qd + 2 * kvd, k, "qkv")
    if want_name:
        assert dev.last_kernel() == want_name
    got = y.download(np.float32)
    assert rel_l2(got, orc.dmv_qkv(bq, bk, bv, qd, kvd, k, x, nw, eps)) < 1e-5
    xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps) * nw
    want = np.concatenate([_np_deq(b, r, k) @ xn for b, r in ((bq, qd), (bk, kvd), (bv, kvd))])
    assert rel_l2(got, want) < 1e-3
    for part, (lo, hi) in (("q", (0, qd)), ("k", (qd, qd + kvd)), ("v", (qd + kvd, qd + 2 * kvd))):
        assert rel_l2(got[lo:hi], want[lo:hi]) < 1e-3, part
    for w in ws:
        w.free()


def test_decode_ffn_instance(dev):
    """the decode step's gate / up matvec with ffn_norm and SwiGLU fused (text.rs:643, dmv_ffn.wgsl): 3072 × 1024 each,
    the k_dmv_full FFN instance (3 rows a wave on 256 CUs), against the oracle (≤ 1e-5) and fp64 silu(g)·u (≤ 1e-3)"""
    rows, k, eps = 3072, 1024, 1e-6
    bg, bu = htr.synth_q8_0(310, rows, k), htr.synth_q8_0(311, rows, k)
    x = htr.synth_normal(33, k, 0.0, 2.0)
    nw = htr.synth_normal(34, k, 1.0, 0.02)
    wg, wu = htr.Weight(dev, bg, rows, k), htr.Weight(dev, bu, rows, k)
    y = dev.alloc(rows * 4)
    htr.matvec_ffn(dev, wg, wu, dev.upload(x), dev.upload(nw), eps, y)
    want_name = _dmv_full_name(dev, rows, k, "ffn")
    if want_name:
        assert dev.last_kernel() == want_name
    got = y.download(np.float32)
    assert rel_l2(got, orc.dmv_ffn(bg, bu, rows, k, x, nw, eps)) < 1e-5
    xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps) * nw
    g, u = _np_deq(bg, rows, k) @ xn, _np_deq(bu, rows, k) @ xn
    assert rel_l2(got, g / (1 + np.exp(-g)) * u) < 1e-3
    wg.free()
    wu.free()


@pytest.mark.parametrize("rows,k,name", [(1024, 2048, "o"), (1024, 3072, "down")])
def test_decode_residual_instances(dev, rows, k, name):
    """the decode step's o and down projections, accumulating onto the residual (text.rs:642, 644: dmv with acc = 1):
    the k_dmv_full plain instance (1 row a wave on 256 CUs), y + W·x against the oracle (≤ 1e-5) and fp64 (≤ 1e-3)"""
    blocks = htr.synth_q8_0(320 + k, rows, k)
    x = htr.synth_normal(35 + k, k)
    base = htr.synth_normal(36 + k, rows, 0.0, 4.0)
    w = htr.Weight(dev, blocks, rows, k)
    yb = dev.upload(base)
    htr.matvec_q8_0(dev, w, dev.upload(x), yb, acc=True)
    want_name = _dmv_full_name(dev, rows, k, "plain")
    if want_name:
        assert dev.last_kernel() == want_name
    got = yb.download(np.float32)
    assert rel_l2(got, orc.dmv(blocks, rows, k, x, None, 0.0, base, True)) < 1e-5, name
    want = base.astype(np.float64) + _np_deq(blocks, rows, k) @ x.astype(np.float64)
    assert rel_l2(got, want) < 1e-3, name
    # the product alone, the accumulated part taken back off
    assert rel_l2(got - base, want - base) < 1e-3, name
    w.free()


def test_graph_capture_replays_the_same_matvecs(dev):
    """htr_capture_begin / end: 8 matvecs over 4 weights recorded once, replayed 3 times with eager work and host
    reads between the replays; every replay equals the eager result bit for bit. A call that would allocate or wait
    fails while recording, and the device stays usable."""
    rows, k = 3072, 1024
    ws = [htr.Weight(dev, htr.synth_q8_0(400 + i, rows, k), rows, k) for i in range(4)]
    xb = dev.upload(htr.synth_normal(41, k))
    ys = [dev.alloc(rows * 4) for _ in range(8)]
    for i, y in enumerate(ys):
        htr.matvec_q8_0(dev, ws[i % 4], xb, y)
    eager = [y.download(np.float32) for y in ys]
    poison = np.full(rows, np.nan, np.float32)
    for y in ys:
        y.upload(poison)
    dev.capture_begin()
    for i, y in enumerate(ys):
        htr.matvec_q8_0(dev, ws[i % 4], xb, y)
    with pytest.raises(htr.HtrError, match="captured"):
        dev.sync()
    with pytest.raises(htr.HtrError, match="captured"):
        dev.alloc(64)
    g = dev.capture_end()
    for rep in range(3):
        for y in ys:  # eager work between the replays: poison the outputs
            y.upload(poison)
        g.launch()
        dev.sync()
        for i, y in enumerate(ys):
            assert np.array_equal(y.download(np.float32), eager[i]), (rep, i)
    g.free()
    dev.alive()
    for w in ws:
        w.free()
