"""Vision::from_gguf (vision.rs:55-84, 117-150, 177-233) on the GPU: an mmproj GGUF's BF16 / F32 weights streamed
onto the device and converted there (f16_from_bf16.wgsl: f16 of value × scale, the down projection × 64) must give
the encode the oracle computes on the f16 planes numpy makes from the same bits (its float16 cast: round to nearest
even, subnormals kept) — rel-L2 within the tiny encoder's bars (1e-5 after the patch embedding, 2e-4 after a layer and
through the projector) — and the reference's load checks hold: projector, SwiGLU, head dim, the absent tensors, types,
shapes, F32 norms, three-value mean / std, and the refusal of values beyond f16's range (counted per 32-bit word)."""

import numpy as np
import pytest

import htr
import oracle as orc
from gguf_writer import BOOL, F32, GGML_F16, GGML_F32, STR, U32, ARR, bf16_bits, bf16_value, vision_model_gguf
from helpers import rel_l2
from test_vision_oracle import tiny_page, tiny_vision_cfg

pytestmark = pytest.mark.gpu


def mmproj_tensors(cfg, seed=11, f32_kinds=()):
    """weights as an mmproj holds them: BF16 bits (uint16 [rows][cols]), or the float32 values for the kinds named in
    ``f32_kinds`` (patch_embd, merger, mm1, mm2, or the layer kinds q … down); f32 norms"""
    g = orc.Lcg(seed)
    d, f, pd, pp = cfg["dim"], cfg["n_ff"], cfg["proj_dim"], 3 * cfg["patch"] ** 2

    def wt(kind, rows, cols, s):
        a = g.f32(rows * cols, s).reshape(rows, cols)
        return a.astype(np.float32) if kind in f32_kinds else bf16_bits(a)

    def nv(n):
        return (1 + g.f32(n, 0.1)).astype(np.float32)

    layers = []
    for _ in range(cfg["n_layer"]):
        layers.append(dict(ln1=nv(d), ln2=nv(d), q=wt("q", d, d, 0.1), k=wt("k", d, d, 0.1), v=wt("v", d, d, 0.1),
                           o=wt("o", d, d, 0.05), gate=wt("gate", f, d, 0.1), up=wt("up", f, d, 0.1),
                           down=wt("down", d, f, 0.05 / 64)))
    return dict(patch_embd=wt("patch_embd", d, pp, 0.05), pre_ln=nv(d), layers=layers, input_norm=nv(d),
                merger=wt("merger", d, 4 * d, 0.03), mm1=wt("mm1", pd, d, 0.05), mm2=wt("mm2", pd, pd, 0.05))


def f16_plane(a, scale=1.0):
    """the f16 weight a load holds for an mmproj tensor: f16(value × scale) of its BF16 bits or F32 values"""
    v = bf16_value(a) if a.dtype == np.uint16 else a
    return (v * np.float32(scale)).astype(np.float16).view(np.uint16)


def oracle_planes(t):
    """the oracle's f16-plane inputs for mmproj tensors ``t``: the patch embedding as the f32 values the device keeps
    (a BF16 tensor's f16 values; an F32 tensor's own)"""
    pe = t["patch_embd"]
    pe = f16_plane(pe).view(np.float16).astype(np.float32) if pe.dtype == np.uint16 else pe
    layers = []
    for ly in t["layers"]:
        p = dict(ln1=ly["ln1"], ln2=ly["ln2"])
        for k in ("q", "k", "v", "o", "gate", "up", "down"):
            p[k] = f16_plane(ly[k], 64.0 if k == "down" else 1.0)
        layers.append(p)
    return dict(patch_embd=pe, pre_ln=t["pre_ln"], layers=layers, input_norm=t["input_norm"],
                merger=f16_plane(t["merger"]), mm1=f16_plane(t["mm1"]), mm2=f16_plane(t["mm2"]))


@pytest.mark.parametrize("f32_kinds", [(), ("patch_embd", "merger", "mm2", "up")], ids=["bf16", "mixed-f32"])
def test_mmproj_encoder_matches_oracle(dev, tmp_path, f32_kinds):
    cfg = dict(tiny_vision_cfg(), image_size=1540)
    t = mmproj_tensors(cfg, f32_kinds=f32_kinds)
    path = tmp_path / "mmproj.gguf"
    path.write_bytes(vision_model_gguf(cfg, t))
    g = htr.Gguf(str(path))
    live0 = dev.mem_live()["weights"]
    v = htr.Vision.from_gguf(dev, g)
    g.close()
    try:
        c = v.cfg
        assert (c["n_layer"], c["dim"], c["n_head"], c["n_ff"], c["patch"], c["merge"], c["proj_dim"]) == \
            (2, 128, 2, 512, 14, 2, 128)
        assert c["image_size"] == 1540 and c["rope_theta"] == 1e4 and np.float32(c["eps"]) == np.float32(1e-5)
        assert np.array_equal(np.float32(c["mean"]), np.float32(cfg["mean"]))
        assert np.array_equal(np.float32(c["std"]), np.float32(cfg["std"]))
        t16 = oracle_planes(t)
        for w, h in ((56, 84), (112, 140)):
            rgb = tiny_page(cfg, w, h, seed=w + h)
            for nl in (0, 1, -1):
                got = v.encode(rgb, nl)
                want = orc.vision_encode(cfg, t16, rgb, nl, w16=True)
                e = rel_l2(got, want)
                print(f"\n[mmproj {'+'.join(f32_kinds) or 'bf16'} {w}x{h} layers {nl}] rel-L2 vs oracle {e:.2e}")
                assert e < (1e-5 if nl == 0 else 2e-4), (w, h, nl)
    finally:
        v.free()
    assert dev.mem_live()["weights"] == live0


def test_mmproj_streams_a_tensor_over_several_ranges(dev):
    """a 128 × 65536 SwiGLU (8.4 M values a weight: more than one 32 MiB staging range holds as f32 words) loads and
    encodes as the oracle does"""
    cfg = dict(tiny_vision_cfg(), n_layer=1, n_ff=65536, image_size=1540)
    t = mmproj_tensors(cfg, seed=3, f32_kinds=("gate",))
    g = htr.Gguf(data=vision_model_gguf(cfg, t))
    v = htr.Vision.from_gguf(dev, g)
    g.close()
    try:
        rgb = tiny_page(cfg, 56, 84, seed=1)
        t16 = oracle_planes(t)
        for nl in (1, -1):
            e = rel_l2(v.encode(rgb, nl), orc.vision_encode(cfg, t16, rgb, nl, w16=True))
            print(f"\n[mmproj n_ff 65536 layers {nl}] rel-L2 vs oracle {e:.2e}")
            assert e < 2e-4, nl
    finally:
        v.free()


def load_err(dev, cfg, t, **kw):
    g = htr.Gguf(data=vision_model_gguf(cfg, t, **kw))
    try:
        with pytest.raises(htr.HtrError) as ei:
            htr.Vision.from_gguf(dev, g).free()
        return str(ei.value)
    finally:
        g.close()


def test_mmproj_load_checks(dev):
    cfg = dict(tiny_vision_cfg(), image_size=1540)
    t = mmproj_tensors(cfg)
    d = cfg["dim"]
    live0 = dev.mem_live()
    cases = [
        (dict(kvs_over={"clip.projector_type": (STR, "pixtral")}), 'projector "pixtral"'),
        (dict(kvs_over={"clip.use_silu": (BOOL, 0)}), "would not be SwiGLU"),
        (dict(kvs_over={"clip.use_silu": None}), "no metadata key clip.use_silu"),
        (dict(kvs_over={"clip.vision.attention.head_count": (U32, 4)}), "head dim 128/4"),
        (dict(kvs_over={"clip.vision.image_size": (F32, 1540.0)}), "not u32"),
        (dict(kvs_over={"clip.vision.image_mean": (ARR, (F32, [0.5, 0.5]))}), "image_mean has 2 values"),
        (dict(kvs_over={"clip.vision.image_std": (ARR, (U32, [1, 1, 1]))}), "not f32"),
        (dict(extra_tensors=[("v.post_ln.weight", GGML_F32, [d], bytes(4 * d))]), "v.post_ln.weight is in the GGUF"),
        (dict(extra_tensors=[("mm.1.bias", GGML_F32, [d], bytes(4 * d))]), "mm.1.bias is in the GGUF"),
        (dict(skip=("v.blk.1.ffn_up.weight",)), "no tensor v.blk.1.ffn_up.weight"),
        (dict(skip=("mm.2.weight",)), "no tensor mm.2.weight"),
        (dict(skip=("v.blk.0.attn_k.weight",),
              extra_tensors=[("v.blk.0.attn_k.weight", GGML_F16, [d, d], bytes(2 * d * d))]),
         "v.blk.0.attn_k.weight: F16 weights are not supported in the vision encoder"),
        (dict(skip=("v.blk.0.attn_v.weight",),
              extra_tensors=[("v.blk.0.attn_v.weight", GGML_F32, [d, d // 2], bytes(2 * d * d))]),
         "v.blk.0.attn_v.weight: shape [128, 64], expected 128 values × 128 rows"),
        (dict(skip=("v.blk.1.ln2.weight",),
              extra_tensors=[("v.blk.1.ln2.weight", GGML_F32, [d // 2], bytes(2 * d))]),
         "v.blk.1.ln2.weight: F32 [64], expected F32 [128]"),
        (dict(skip=("v.pre_ln.weight",),
              extra_tensors=[("v.pre_ln.weight", GGML_F16, [d], bytes(2 * d))]),
         "v.pre_ln.weight: F16 [128], expected F32 [128]"),
    ]
    for kw, msg in cases:
        e = load_err(dev, cfg, t, **kw)
        assert msg in e, (kw, e)
    assert dev.mem_live() == live0


def test_mmproj_refuses_values_beyond_f16(dev):
    """vision.rs:224-232: a weight value whose f16 would be inf refuses the load, counted per 32-bit word of the
    BF16 tensor (two such values in one word count once); the down projection's values count after × 64"""
    cfg = dict(tiny_vision_cfg(), image_size=1540)
    t = mmproj_tensors(cfg)
    q = bf16_value(t["layers"][0]["q"]).copy()
    q.flat[0], q.flat[1], q.flat[5] = 7e4, -7e4, 7e4  # words 0 and 2
    q.flat[9] = 65504.0  # f16's largest has no bf16: it rounds to 65536, beyond (word 4)
    dn = bf16_value(t["layers"][1]["down"]).copy()
    dn.flat[2] = 1000.0  # × 64 = 64000: in range
    dn.flat[7] = 1100.0  # × 64 = 70400: beyond
    t["layers"][0]["q"], t["layers"][1]["down"] = bf16_bits(q), bf16_bits(dn)
    e = load_err(dev, cfg, t)
    assert "4 words of vision weights hold values beyond f16's range (65504)" in e, e
    # the same file with the values in range loads: 1000 × 64 = 64000 and 65280 (bf16's largest below 65504)
    dn.flat[7] = 1000.0
    q = bf16_value(mmproj_tensors(cfg)["layers"][0]["q"]).copy()
    q.flat[3] = -65280.0
    t["layers"][0]["q"], t["layers"][1]["down"] = bf16_bits(q), bf16_bits(dn)
    g = htr.Gguf(data=vision_model_gguf(cfg, t))
    htr.Vision.from_gguf(dev, g).free()
    g.close()


def test_mmproj_at_the_page_encoder_shape(dev, tmp_path):
    """an mmproj of the page encoder's shape (24 layers, hidden 1024, SwiGLU 4096, projector 1024; 810 MB of BF16,
    every layer holding the first one's weights) streamed from a file: its load time, the residual after the patch
    embedding of a 1540 × 1540 page against the oracle (1e-5), and the whole encode finite at 3025 × 1024. The layers'
    conversion is pinned by the tiny mmproj tests above (the oracle takes about 40 s for one layer of this page)"""
    import time

    from htr import synth

    cfg, t = synth.vision_model(n_layer=1)
    d, f, pd = cfg["dim"], cfg["n_ff"], cfg["proj_dim"]
    deq = lambda b, rows, cols: bf16_bits(orc.q8_0_dequant(b, rows * cols).reshape(rows, cols))
    shapes = dict(q=(d, d), k=(d, d), v=(d, d), o=(d, d), gate=(f, d), up=(f, d), down=(d, f))
    ly = dict(ln1=t["layers"][0]["ln1"], ln2=t["layers"][0]["ln2"],
              **{k: deq(t["layers"][0][k], *rc) for k, rc in shapes.items()})
    tb = dict(patch_embd=bf16_bits(t["patch_embd"]), pre_ln=t["pre_ln"], input_norm=t["input_norm"], layers=[ly] * 24,
              merger=deq(t["merger"], d, 4 * d), mm1=deq(t["mm1"], pd, d), mm2=deq(t["mm2"], pd, pd))
    path = tmp_path / "mmproj-page.gguf"
    path.write_bytes(vision_model_gguf(dict(cfg, n_layer=24), tb))
    g = htr.Gguf(str(path))
    t0 = time.perf_counter()
    v = htr.Vision.from_gguf(dev, g)
    dt = time.perf_counter() - t0
    g.close()
    size = path.stat().st_size
    print(f"\n[mmproj page shape] {size / 1e6:.0f} MB loaded in {dt * 1e3:.0f} ms ({size / dt / 1e9:.1f} GB/s)")
    try:
        assert v.cfg["n_layer"] == 24
        rgb = synth.page(99, 1540, 1540)
        t16 = oracle_planes(dict(tb, layers=[ly]))
        e = rel_l2(v.encode(rgb, 0), orc.vision_encode(cfg, t16, rgb, 0, w16=True))
        print(f"[mmproj page shape 1540x1540 layers 0] rel-L2 vs oracle {e:.2e}")
        assert e < 1e-5
        out = v.encode(rgb)
        assert out.shape == (3025, 1024) and np.all(np.isfinite(out))
    finally:
        v.free()
