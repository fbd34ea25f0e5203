"""HTR_POISON=1, the reference's OCR_WGPU_POISON=1 diagnostic (gpu.rs:739-768, 821-823, 1307-1310): a device opened
with it hands out memory filled with 0xFF bytes (NaN as f32 and f16) instead of zeros — counters and tickets that
must start at zero excepted — and fills memory again when it is given back. A kernel that read anything nothing wrote
(a cache row past the keys, a pad of a GEMM tile, the exchange words before their first token, a stale partial) would
then see NaN. The decode path is deterministic, so every result on the poisoned device must equal the normal device's
bit for bit: the f16 path's prefill (MFMA GEMMs, causal attention and its key blocks), the one-launch step and the
per-kernel step, decode_gpu on both, a KV cache grown with the read (its new rows poisoned), and the F32 path's
prefill, step and read.
"""
import os

import numpy as np
import pytest

import htr
from helpers import synth_text_model, tiny_prompt, tiny_text_model, to_htr_cfg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pdev():
    keep = os.environ.get("HTR_POISON")
    os.environ["HTR_POISON"] = "1"
    try:
        d = htr.Device(0)
    finally:
        if keep is None:
            del os.environ["HTR_POISON"]
        else:
            os.environ["HTR_POISON"] = keep
    yield d
    d.close()


def bits(a) -> np.ndarray:
    return np.asarray(a, np.float32).view(np.uint32)


def poisoned_alloc_is_nan(pdev):
    b = pdev.alloc(64)
    v = b.download(np.float32, 16)
    b.free()
    return bool(np.all(np.isnan(v)))


def decoder_run(dev, cfg, te, on, layers, prompt, path, fused, kv_grow=None, new=48):
    keep = dev.compute
    dev.compute = path
    try:
        m = htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep
    s = m.session(len(prompt) + new + 8, kv_grow)
    if path == htr.COMPUTE_F16 and cfg["dim"] == 1024:
        s.fused_step = fused
    out = {"prefill": s.prefill(prompt[:-1]), "step": s.step(int(prompt[-1]))}
    ch = s.choice(htr.Preset(repetition_penalty=1.3, repetition_window=16, frequency_penalty=0.4, max_new_tokens=new),
                  prompt, chunk=16, depth=2)
    out["tokens"] = np.array(s.decode_gpu(ch, new), np.int64)
    out["last"] = s.logits()
    out["fused"] = s.fused_step
    ch.free()
    s.free()
    m.free()
    return out


@pytest.fixture(scope="module")
def decoder():
    from htr import synth

    cfg, te, on, layers = synth_text_model(n_layer=3, n_vocab=4096, seed=606)
    return cfg, te, on, layers, synth.prompt_ids(66, 700, cfg["n_vocab"])


def test_poisoned_memory_reads_nan(dev, pdev):
    assert poisoned_alloc_is_nan(pdev)
    b = dev.alloc(64)
    assert np.all(b.download(np.uint32, 16) == 0)
    b.free()


@pytest.mark.parametrize("fused,kv_grow", [(True, None), (False, None), (True, 61)],
                         ids=["one_launch", "per_kernel", "one_launch_kv_grown"])
def test_decoder_equal_under_poison(dev, pdev, decoder, fused, kv_grow):
    cfg, te, on, layers, prompt = decoder
    a = decoder_run(dev, cfg, te, on, layers, prompt, htr.COMPUTE_F16, fused, kv_grow)
    b = decoder_run(pdev, cfg, te, on, layers, prompt, htr.COMPUTE_F16, fused, kv_grow)
    assert a["fused"] == b["fused"] == fused
    for k in ("prefill", "step", "last"):
        assert np.all(np.isfinite(b[k])), k
        assert np.array_equal(bits(a[k]), bits(b[k])), k
    assert np.array_equal(a["tokens"], b["tokens"])
    print(f"\n[poison] decoder f16 path, {'one-launch' if fused else 'per-kernel'} step"
          f"{', KV grown by 61 rows' if kv_grow else ''}: prefill, step, 48 tokens and the last logits bit-equal",
          flush=True)


def test_f32_path_equal_under_poison(dev, pdev):
    cfg, te, on, layers = tiny_text_model()
    prompt = np.concatenate([tiny_prompt(), tiny_prompt(40) + 1]) % cfg["n_vocab"]
    a = decoder_run(dev, cfg, te, on, layers, prompt, htr.COMPUTE_F32, False, None, 40)
    b = decoder_run(pdev, cfg, te, on, layers, prompt, htr.COMPUTE_F32, False, None, 40)
    for k in ("prefill", "step", "last"):
        assert np.all(np.isfinite(b[k])) and np.array_equal(bits(a[k]), bits(b[k])), k
    assert np.array_equal(a["tokens"], b["tokens"])
