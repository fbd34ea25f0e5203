"""TextModel::load from a GGUF (text.rs:43-76, 101-118, 332-375) on the GPU: the weights streamed from the file and
repacked on the device must be the weights the host-array path uploads — the logits of a prefill and of decode steps
are bit-identical between the two models, on both compute paths — and the reference's load checks hold (architecture,
head dim, biases, a fused attn_qkv, an untied output, shapes and types)."""
import time

import numpy as np
import pytest

import htr
from gguf_writer import GGML_F16, GGML_F32, GGML_Q8_0, STR, U32, text_model_gguf
from helpers import synth_text_model, tiny_prompt, tiny_text_model, to_htr_cfg

pytestmark = pytest.mark.gpu


def on_path(dev, path, make):
    keep = dev.compute
    dev.compute = path
    try:
        return make()
    finally:
        dev.compute = keep


@pytest.mark.parametrize("path", [htr.COMPUTE_F32, htr.COMPUTE_F16])
def test_tiny_model_from_gguf_equals_host_arrays(dev, path):
    cfg, te, on, layers = tiny_text_model()
    g = htr.Gguf(data=text_model_gguf(cfg, te, on, layers))
    a = on_path(dev, path, lambda: htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers))
    b = on_path(dev, path, lambda: htr.TextModel.from_gguf(dev, g))
    assert b.cfg.n_layer == 5 and b.cfg.dim == 256 and b.cfg.n_vocab == 1000 and b.cfg.n_ctx_train == 4096
    prompt = tiny_prompt()
    sa, sb = a.session(prompt.size + 8), b.session(prompt.size + 8)
    la, lb = sa.prefill(prompt), sb.prefill(prompt)
    assert np.array_equal(la, lb)
    for _ in range(4):
        t = int(np.argmax(la))
        la, lb = sa.step(t), sb.step(t)
        assert np.array_equal(la, lb)
    for x in (sa, sb, a, b):
        x.free()
    g.close()


def bad(cfg, te, on, layers, **kw):
    return htr.Gguf(data=text_model_gguf(cfg, te, on, layers, **kw))


def test_load_checks(dev):
    cfg, te, on, layers = tiny_text_model()
    d = cfg["dim"]
    cases = [
        (dict(extra_kvs=[("general.architecture", STR, "llama")]), "duplicate metadata key"),
        (dict(extra_kvs=[("qwen3.rope.dimension_count", U32, 64)]), "partial rope"),
        (dict(extra_tensors=[("blk.1.attn_q.bias", GGML_F32, [256], bytes(1024))]), "not part of this engine's graph"),
        (dict(extra_tensors=[("blk.0.attn_qkv.weight", GGML_F32, [4], bytes(16))]), "fused attn_qkv"),
        (dict(extra_tensors=[("output.weight", GGML_F32, [4], bytes(16))]), "ties the output"),
        (dict(skip=("blk.2.ffn_up.weight",)), "no tensor blk.2.ffn_up.weight"),
        (dict(skip=("output_norm.weight",)), "no tensor output_norm.weight"),
    ]
    for kw, msg in cases:
        with pytest.raises(htr.HtrError, match=msg):
            htr.TextModel.from_gguf(dev, bad(cfg, te, on, layers, **kw))
    # an f16 projection where q8_0 is read; a norm of the wrong length
    ly = [dict(x) for x in layers]
    g = bad(cfg, te, on, ly, skip=("blk.3.attn_k.weight",),
            extra_tensors=[("blk.3.attn_k.weight", GGML_F16, [d, 128], bytes(d * 128 * 2))])
    with pytest.raises(htr.HtrError, match="q8_0 weights"):
        htr.TextModel.from_gguf(dev, g)
    g = bad(cfg, te, on, ly, skip=("blk.0.ffn_norm.weight",),
            extra_tensors=[("blk.0.ffn_norm.weight", GGML_F32, [d - 32], bytes((d - 32) * 4))])
    with pytest.raises(htr.HtrError, match="expected F32"):
        htr.TextModel.from_gguf(dev, g)
    # a transposed projection: attn_k stored [kvd, d] = [128, 256] instead of [d, kvd]
    g = bad(cfg, te, on, ly, skip=("blk.1.attn_k.weight",),
            extra_tensors=[("blk.1.attn_k.weight", GGML_Q8_0, [128, d], np.asarray(ly[1]["k"]).tobytes())])
    with pytest.raises(htr.HtrError, match="shape"):
        htr.TextModel.from_gguf(dev, g)


def test_architecture_and_head_dim_checks(dev):
    from gguf_writer import gguf_bytes

    cfg, te, on, layers = tiny_text_model()
    base = text_model_gguf(cfg, te, on, layers)
    arch = base.replace(b"\x05\x00\x00\x00\x00\x00\x00\x00qwen3", b"\x05\x00\x00\x00\x00\x00\x00\x00llama", 1)
    with pytest.raises(htr.HtrError, match="qwen3 only"):
        htr.TextModel.from_gguf(dev, htr.Gguf(data=arch))
    key = b"qwen3.attention.key_length"
    at = base.index(key) + len(key) + 4
    hd = base[:at] + np.uint32(64).tobytes() + base[at + 4:]
    with pytest.raises(htr.HtrError, match="head dim 64"):
        htr.TextModel.from_gguf(dev, htr.Gguf(data=hd))
    assert gguf_bytes  # the writer module is the one the other tests use


def test_full_size_model_from_a_file(dev, tmp_path):
    """the 28-layer decoder shape (633 MB of q8_0) written to a GGUF file and streamed onto the device: the same logits as the
    host-array model after a 16-token prompt and 4 steps"""
    cfg, te, on, layers = synth_text_model()
    p = tmp_path / "text-q8_0.gguf"
    p.write_bytes(text_model_gguf(cfg, te, on, layers))
    a = on_path(dev, htr.COMPUTE_F32, lambda: htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers))
    dev.sync()
    t0 = time.perf_counter()
    with htr.Gguf(p) as g:
        b = on_path(dev, htr.COMPUTE_F32, lambda: htr.TextModel.from_gguf(dev, g))
    dt = time.perf_counter() - t0
    print(f"\n[gguf load] {p.stat().st_size / 1e6:.0f} MB in {dt * 1e3:.0f} ms ({p.stat().st_size / dt / 1e9:.2f} GB/s)")
    prompt = (np.abs(htr.synth_normal(79, 16)) * 1e5).astype(np.int64) % cfg["n_vocab"]
    sa, sb = a.session(24), b.session(24)
    la, lb = sa.prefill(prompt), sb.prefill(prompt)
    assert np.array_equal(la, lb)
    for _ in range(4):
        t = int(np.argmax(la))
        la, lb = sa.step(t), sb.step(t)
        assert np.array_equal(la, lb)
    for x in (sa, sb, a, b):
        x.free()
