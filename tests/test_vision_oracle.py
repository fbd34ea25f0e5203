"""Pins the vision oracle (oracle/htr_vision_oracle.c) before any GPU result is compared with it.

Every function is checked against an independent numpy statement: index maps by reshape / transpose (patchify, the
2x2 unfold in torch-unfold order), closed forms in fp64 (RoPE angles, rms norm, GEMMs, SwiGLU, GELU, softmax
attention), and a whole tiny encoder forward written here in numpy with the f16 path's roundings. The reference's own
bars for these kernels (text.rs:1123-1293): rms_norm_h rel-L2 < 1e-3, matmul_f16x < 1e-4, ffn_f16 < 2e-3, vision
attention < 5e-3 against fp64.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import rel_l2

CLIP_MEAN = [0.48145466, 0.4578275, 0.40821073]
CLIP_STD = [0.26862954, 0.26130258, 0.27577711]


def f16r(a):
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def test_pixel_lut_and_patchify_match_reshape_im2col():
    rng = np.random.default_rng(1)
    side, px, py = 14, 4, 3
    rgb = rng.integers(0, 256, (py * side, px * side, 3), dtype=np.uint8)
    lut = orc.pixel_lut(CLIP_MEAN, CLIP_STD)
    want_lut = ((np.arange(256)[None, :] / 255.0 - np.array(CLIP_MEAN)[:, None]) / np.array(CLIP_STD)[:, None])
    assert np.allclose(lut.reshape(3, 256), want_lut, atol=1e-6)
    P = orc.patchify(rgb, side, lut)
    norm = lut.reshape(3, 256)[np.arange(3)[None, None, :], rgb]  # [h][w][3]
    # im2col by reshape: (py, ky, px, kx, c) → (py, px, c, ky, kx)
    want = norm.reshape(py, side, px, side, 3).transpose(0, 2, 4, 1, 3).reshape(py * px, 3 * side * side)
    assert np.array_equal(P, want.astype(np.float32))


def test_rope2d_table_and_rotation_match_fp64():
    theta, d, max_pos = 1e4, 64, 110
    cs = orc.rope2d_table(theta, d, max_pos).astype(np.float64)
    pos = np.arange(max_pos)[:, None]
    k = np.arange(d // 4)[None, :]
    ang0 = pos * theta ** (-2.0 * k / (d / 2))
    ang1 = ang0 * theta ** (-2.0 / d)
    # f32 recurrence vs the fp64 closed form: ≤ 1e-4 at angles up to 110 rad
    assert np.abs(cs[0, :, :, 0] - np.cos(ang0)).max() < 1e-4
    assert np.abs(cs[0, :, :, 1] - np.sin(ang0)).max() < 1e-4
    assert np.abs(cs[1, :, :, 0] - np.cos(ang1)).max() < 1e-4
    assert np.abs(cs[1, :, :, 1] - np.sin(ang1)).max() < 1e-4
    # the rotation: token t at row t // px, column t % px; adjacent pairs of each half
    n_head, px, py = 3, 5, 4
    rng = np.random.default_rng(2)
    q = rng.standard_normal((px * py, n_head * d)).astype(np.float32)
    got = orc.rope2d(q, n_head, d, px, max_pos, cs.astype(np.float32)).astype(np.float64)
    want = q.astype(np.float64).reshape(px * py, n_head, 2, d // 4, 2).copy()
    t = np.arange(px * py)
    for half, p in ((0, t // px), (1, t % px)):
        c, s = cs[half, p, :, 0][:, None, :], cs[half, p, :, 1][:, None, :]
        x0, x1 = want[:, :, half, :, 0].copy(), want[:, :, half, :, 1].copy()
        want[:, :, half, :, 0] = x0 * c - x1 * s
        want[:, :, half, :, 1] = x0 * s + x1 * c
    assert np.abs(got - want.reshape(px * py, n_head * d)).max() < 1e-5


def test_rms_norm_h_matmul_f16_ffn_match_fp64():
    """text.rs:1123-1193 shapes: 100 rows, K = 128, N = F = 128"""
    rng = np.random.default_rng(3)
    m, d, f = 100, 128, 128
    x = (rng.standard_normal((m, d)) * 4).astype(np.float32)
    nw = (1 + rng.standard_normal(d) * 0.2).astype(np.float32)
    h = orc.rms_norm_h(x, nw, 1e-5).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5) * nw
    assert np.all(np.abs(h - want) <= np.abs(want) * 2.0 ** -11 + 1e-7)
    w16 = (rng.standard_normal((d, d)) * 0.2).astype(np.float16)
    base = rng.standard_normal((m, d)).astype(np.float32)
    y = orc.matmul_f16(h.astype(np.float16), w16, base)
    assert rel_l2(y, base + h @ w16.astype(np.float64).T) < 1e-6
    wg = (rng.standard_normal((f, d)) * 0.2).astype(np.float16)
    wu = (rng.standard_normal((f, d)) * 0.2).astype(np.float16)
    g = orc.ffn_f16(h.astype(np.float16), wg, wu, 0.125).astype(np.float64)
    a, u = h @ wg.astype(np.float64).T, h @ wu.astype(np.float64).T
    want = a / (1 + np.exp(-a)) * u * 0.125
    assert np.all(np.abs(g - want) <= np.abs(want) * 2.0 ** -10 + 1e-6)


def test_q8_0_to_f16_is_rne_of_the_exact_dequant():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(64 * 96) * 0.3).astype(np.float32)
    blocks, deq = orc.q8_0_quantize(x)
    for scale in (1.0, 64.0):
        got = orc.q8_0_to_f16(blocks, 64, 96, scale)
        assert np.array_equal(got.view(np.uint16), (deq * np.float32(scale)).astype(np.float16).reshape(64, 96).view(np.uint16))


def np_attention(q, k, v, n_head, scale):
    n = q.shape[0]
    out = np.zeros_like(q, dtype=np.float64)
    for h in range(n_head):
        sl = slice(64 * h, 64 * h + 64)
        s = (q[:, sl] @ k[:, sl].T) * scale
        e = np.exp(s - s.max(1, keepdims=True))
        out[:, sl] = (e / e.sum(1, keepdims=True)) @ v[:, sl]
    return out


@pytest.mark.parametrize("n", [70, 129])
def test_attention_coop_matches_fp64(n):
    """text.rs:1229-1255: 70 tokens x 2 heads, O (f16) within 5e-3 of fp64 softmax attention on the unrounded inputs;
    and within 2e-3 of fp64 attention on the f16 path's rounded q·scale, K and V"""
    rng = np.random.default_rng(n)
    nh = 2
    q = (rng.uniform(-1, 1, (n, nh * 64)) * 2).astype(np.float32)
    k = (rng.uniform(-1, 1, (n, nh * 64)) * 2).astype(np.float32)
    v = rng.uniform(-1, 1, (n, nh * 64)).astype(np.float32)
    scale = np.float32(1 / 8)
    o = orc.attention_coop(q, k, v, nh, scale).astype(np.float64)
    assert rel_l2(o, np_attention(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), nh, scale)) < 5e-3
    want = np_attention(f16r(q * scale), f16r(k), f16r(v), nh, 1.0)
    assert rel_l2(o, want) < 2e-3


def test_unfold2x2_and_gelu():
    rng = np.random.default_rng(6)
    px, py, d = 6, 4, 5
    x = rng.standard_normal((px * py, d)).astype(np.float32)
    z = orc.unfold2x2(x, px, py)
    # torch unfold order: channel-major, then kernel row, then kernel column
    want = x.reshape(py // 2, 2, px // 2, 2, d).transpose(0, 2, 4, 1, 3).reshape((px // 2) * (py // 2), 4 * d)
    assert np.array_equal(z, want)
    g = orc.gelu(np.array([-30.0, -3.0, -0.5, 0.0, 0.5, 3.0, 30.0], np.float32)).astype(np.float64)
    xs = np.array([-30.0, -3.0, -0.5, 0.0, 0.5, 3.0, 30.0])
    want = 0.5 * xs * (1 + np.tanh(np.clip(np.sqrt(2 / np.pi) * xs * (1 + 0.044715 * xs ** 2), -15, 15)))
    assert np.abs(g - want).max() < 1e-5


def tiny_vision_cfg():
    return dict(n_layer=2, dim=128, n_head=2, n_ff=512, patch=14, proj_dim=128, eps=1e-5, rope_theta=1e4,
                mean=CLIP_MEAN, std=CLIP_STD)


def tiny_vision_tensors(cfg, seed=5):
    """q8_0 layer and projector weights from the reference tests' quantizer, f32 patch embedding and norms"""
    g = orc.Lcg(seed)
    d, f, pp = cfg["dim"], cfg["n_ff"], 3 * cfg["patch"] ** 2

    def q8(rows, cols, s):
        return orc.q8_0_quantize(g.f32(rows * cols, s))[0]

    def nv(n):
        return (1 + g.f32(n, 0.1)).astype(np.float32)

    layers = []
    for _ in range(cfg["n_layer"]):
        layers.append(dict(ln1=nv(d), ln2=nv(d), q=q8(d, d, 0.1), k=q8(d, d, 0.1), v=q8(d, d, 0.1), o=q8(d, d, 0.05),
                           gate=q8(f, d, 0.1), up=q8(f, d, 0.1), down=q8(d, f, 0.05 / 64)))
    return dict(patch_embd=g.f32(d * pp, 0.05), pre_ln=nv(d), layers=layers, input_norm=nv(d),
                merger=q8(d, 4 * d, 0.03), mm1=q8(cfg["proj_dim"], d, 0.05), mm2=q8(cfg["proj_dim"], cfg["proj_dim"], 0.05))


def tiny_page(cfg, w=56, h=84, seed=7):
    return np.random.default_rng(seed).integers(0, 256, (h, w, 3), dtype=np.uint8)


def np_vision_forward(cfg, t, rgb, n_layers=-1):
    """an independent numpy statement of run_f16 + project (fp64, with the f16 path's roundings)"""
    d, f, nh, p = cfg["dim"], cfg["n_ff"], cfg["n_head"], cfg["patch"]
    h, w, _ = rgb.shape
    px, py = w // p, h // p
    n = px * py
    lut = ((np.arange(256)[None, :] / 255.0 - np.array(cfg["mean"])[:, None]) / np.array(cfg["std"])[:, None])
    norm = lut[np.arange(3)[None, None, :], rgb]
    P = norm.reshape(py, p, px, p, 3).transpose(0, 2, 4, 1, 3).reshape(n, 3 * p * p)

    def deq(b, rows, cols, s=1.0):
        bb = b.reshape(-1, 34)
        dd = bb[:, :2].copy().view(np.float16).astype(np.float32)
        return f16r((bb[:, 2:].view(np.int8).astype(np.float32) * dd * np.float32(s)).reshape(rows, cols))

    def rms(x, wv):
        return x / np.sqrt((x ** 2).mean(1, keepdims=True) + cfg["eps"]) * wv

    x = rms(P @ t["patch_embd"].reshape(d, -1).astype(np.float64).T, t["pre_ln"])
    mp = max(px, py)
    tt = np.arange(n)
    k = np.arange(16)

    def rope(z):
        z = z.reshape(n, nh, 2, 16, 2).copy()
        for half, pos in ((0, tt // px), (1, tt % px)):
            ang = pos[:, None] * cfg["rope_theta"] ** (-2.0 * k / 32)[None, :] * (1.0 if half == 0 else cfg["rope_theta"] ** (-2.0 / 64))
            c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
            a0, a1 = z[:, :, half, :, 0].copy(), z[:, :, half, :, 1].copy()
            z[:, :, half, :, 0] = a0 * c - a1 * s
            z[:, :, half, :, 1] = a0 * s + a1 * c
        return z.reshape(n, nh * 64)

    nl = cfg["n_layer"] if n_layers < 0 else n_layers
    for L in t["layers"][:nl]:
        hh = f16r(rms(x, L["ln1"]))
        q = rope(hh @ deq(L["q"], d, d).T)
        kk = rope(hh @ deq(L["k"], d, d).T)
        v = hh @ deq(L["v"], d, d).T
        a = f16r(np_attention(f16r(q / 8), f16r(kk), f16r(v), nh, 1.0))
        x = x + a @ deq(L["o"], d, d).T
        hh = f16r(rms(x, L["ln2"]))
        g = hh @ deq(L["gate"], f, d).T
        u = hh @ deq(L["up"], f, d).T
        gg = f16r(g / (1 + np.exp(-g)) * u / 64)
        x = x + gg @ deq(L["down"], d, f, 64.0).T
    if n_layers >= 0:
        return x
    z = rms(x, t["input_norm"]).reshape(py // 2, 2, px // 2, 2, d).transpose(0, 2, 4, 1, 3).reshape(n // 4, 4 * d)
    mg = z @ deq(t["merger"], d, 4 * d).T
    m1 = mg @ deq(t["mm1"], cfg["proj_dim"], d).T
    m1 = 0.5 * m1 * (1 + np.tanh(np.clip(np.sqrt(2 / np.pi) * m1 * (1 + 0.044715 * m1 ** 2), -15, 15)))
    return m1 @ deq(t["mm2"], cfg["proj_dim"], cfg["proj_dim"]).T


def test_vision_encode_matches_numpy_forward():
    cfg = tiny_vision_cfg()
    t = tiny_vision_tensors(cfg)
    rgb = tiny_page(cfg)
    for nl in (0, 1, -1):
        got = orc.vision_encode(cfg, t, rgb, nl)
        want = np_vision_forward(cfg, t, rgb, nl)
        assert got.shape == want.shape
        e = rel_l2(got, want)
        assert e < 2e-3, (nl, e)
    with pytest.raises(ValueError):
        orc.vision_encode(cfg, t, rgb[:70], -1)  # 70 rows: not on the 28-pixel grid


def f16_planes(cfg, t):
    """the f16 weight planes an mmproj load would hold for the q8_0 tensors of `t` (f16 of the exact dequant; the
    down projection × 64, as vision.rs:124-142 and 31-35 scale it)"""
    d, f, pd = cfg["dim"], cfg["n_ff"], cfg["proj_dim"]
    shapes = dict(q=(d, d), k=(d, d), v=(d, d), o=(d, d), gate=(f, d), up=(f, d), down=(d, f))
    layers = []
    for ly in t["layers"]:
        p = dict(ln1=ly["ln1"], ln2=ly["ln2"])
        for name, (r, c) in shapes.items():
            p[name] = orc.q8_0_to_f16(ly[name], r, c, 64.0 if name == "down" else 1.0)
        layers.append(p)
    return dict(patch_embd=t["patch_embd"], pre_ln=t["pre_ln"], layers=layers, input_norm=t["input_norm"],
                merger=orc.q8_0_to_f16(t["merger"], d, 4 * d), mm1=orc.q8_0_to_f16(t["mm1"], pd, d),
                mm2=orc.q8_0_to_f16(t["mm2"], pd, pd))


def test_vision_encode_on_f16_planes_is_the_q8_0_encode():
    """the oracle's f16-plane entry (weights converted at load) on the planes the q8_0 path converts to inside: the
    same output bit for bit at every depth"""
    cfg = tiny_vision_cfg()
    t = tiny_vision_tensors(cfg)
    t16 = f16_planes(cfg, t)
    rgb = tiny_page(cfg)
    for nl in (0, 1, -1):
        a = orc.vision_encode(cfg, t, rgb, nl)
        b = orc.vision_encode(cfg, t16, rgb, nl, w16=True)
        assert np.array_equal(a, b), nl


def test_vision_resume_composes_with_encode():
    """or_vision_resume (the encoder from a given residual, the per-layer check of the GPU's page encode) is the same
    layer loop and projector: resumed from vision_encode's residual after L layers, it is vision_encode after L + k
    layers, and after every layer and the projector, bit for bit"""
    cfg = tiny_vision_cfg()
    t = tiny_vision_tensors(cfg)
    rgb = tiny_page(cfg, 56, 84)
    px, py = 56 // cfg["patch"], 84 // cfg["patch"]
    n_layer = cfg["n_layer"]
    x0 = orc.vision_encode(cfg, t, rgb, 0)
    for first in range(n_layer):
        x = orc.vision_encode(cfg, t, rgb, first)
        for count in range(n_layer - first + 1):
            got = orc.vision_resume(cfg, t, x, px, py, first, count)
            assert np.array_equal(got, orc.vision_encode(cfg, t, rgb, first + count)), (first, count)
    assert np.array_equal(orc.vision_resume(cfg, t, x0, px, py, 0, n_layer, project=True), orc.vision_encode(cfg, t, rgb))
    # and it is not the identity: a layer moves the residual
    assert rel_l2(orc.vision_resume(cfg, t, x0, px, py, 0, 1), x0) > 1e-3
