"""The text decoder on the GPU: prefill, the CPU-choice step and the run-ahead GPU-choice decode, against the oracle.

Token identity is checked teacher-forced: at every position the oracle computes its own logits from the tokens the GPU
chose so far and makes its own choice; a differing token is accepted only as a documented near-tie (the oracle's
logits of the two tokens within 1e-6 relative). Float logits: rel-L2 against the oracle's f32 restatement.

Both compute paths: the F32 path (exact q8_0 values in the prefill GEMMs) is pinned tightly end to end. The f16 path
(the default; X and q·d rounded to f16 in the prefill GEMMs, as the reference on a device with f16) is pinned tightly
per GEMM (test_gemm_gpu); end to end its logits are only defined to the sensitivity of f16 rounding: on the tiny model
a 1e-7 relative nudge of the embeddings moves the fp64 forward with f16-rounded GEMM operands by 1.0e-3 rel-L2 (the
f32 forward: 3.7e-6), on the 28-layer decoder's shape a 2e-7 nudge of one norm moves the oracle's f16 prefill by 1.9e-3 — two
correct f16-path results in different summation orders differ by that much. Bars: 5e-3 (tiny), 1e-2 (28 layers)."""
import numpy as np
import pytest

import htr
import oracle as orc
from helpers import near_tie, rel_l2, synth_text_model, tiny_prompt, tiny_text_model, to_htr_cfg

pytestmark = pytest.mark.gpu


def model_on(dev, path, cfg, te, on, layers):
    """a TextModel created on the given compute path (a model keeps the path of its creation)"""
    keep = dev.compute
    dev.compute = path
    try:
        return htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep


@pytest.fixture(scope="module")
def tiny(dev):
    cfg, te, on, layers = tiny_text_model()
    m = model_on(dev, htr.COMPUTE_F32, cfg, te, on, layers)
    yield cfg, te, on, layers, m
    m.free()


def teacher_forced(o: orc.Session, first_logits, prompt, toks, rp, window, tie_log):
    """the oracle's choice at every position given the GPU's earlier tokens; returns the number of near-ties"""
    lo = first_logits
    hist = [int(t) for t in prompt]
    for i, t in enumerate(toks):
        pen = lo.copy()
        want = orc.choose(pen, rp, window, 0.0, hist)
        if want != t:
            assert near_tie(pen, want, t), f"step {i}: oracle {want} ({pen[want]!r}), GPU {t} ({pen[t]!r})"
            tie_log.append((i, want, t))
        hist.append(int(t))
        if i + 1 < len(toks):
            lo = o.step(int(t))


def test_tiny_prefill_and_steps_match_oracle(dev, tiny):
    """the reference's tiny model (text.rs:1297-1323) and prompt (text.rs:1333): prefill logits against the fp64
    forward (rel-L2 ≤ 1e-3) and the oracle, then 40 greedy CPU-choice steps (TextModel::step), every logits row against
    the oracle's.

    Bar against the oracle: 2e-4. Both are f32 computations of the same graph in different summation orders (the
    prefill GEMMs and attention tile differently); the oracle's own rel-L2 to the fp64 forward is 3.0e-5 on this
    prompt, and the two f32 results sit on either side of it."""
    from test_oracle import np_forward

    cfg, te, on, layers, m = tiny
    prompt = tiny_prompt()
    s = m.session(prompt.size + 150)
    o = orc.Session(cfg, te, on, layers, prompt.size + 150)
    lg, lo = s.prefill(prompt), o.prefill(prompt)
    want = np_forward(cfg, te, on, layers, list(prompt))[-1]
    e64, eo = rel_l2(lg, want), rel_l2(lg, lo)
    print(f"\n[tiny prefill] rel-L2 vs fp64 {e64:.2e} (oracle vs fp64 {rel_l2(lo, want):.2e}), vs oracle {eo:.2e}")
    assert e64 < 1e-3
    assert eo < 2e-4
    assert s.n_past == prompt.size
    for i in range(40):
        t = int(np.argmax(lg))
        lo_t = int(np.argmax(lo))
        assert t == lo_t or near_tie(lo, lo_t, t), i
        lg, lo = s.step(t), o.step(t)
        assert rel_l2(lg, lo) < 2e-4, i
    assert s.n_past == prompt.size + 40
    s.free()


def test_tiny_decode_gpu_matches_oracle_and_is_chunk_invariant(dev, tiny):
    """text.rs:1366-1377: the GPU choice run ahead (4 × 2 in flight) for 150 tokens with rp 1.1 / window 20; the same
    tokens for other chunk / depth settings and for the CPU-choice path with the oracle's choose on the GPU logits"""
    cfg, te, on, layers, m = tiny
    prompt = tiny_prompt()
    n_new = 150
    preset = htr.Preset(repetition_penalty=1.1, repetition_window=20, max_new_tokens=n_new)
    runs = {}
    for chunk, depth in ((4, 2), (1, 1), (16, 3), (64, 1)):
        s = m.session(prompt.size + n_new)
        s.prefill(prompt)
        ch = s.choice(preset, prompt, chunk, depth)
        runs[(chunk, depth)] = s.decode_gpu(ch, n_new)
        assert len(runs[(chunk, depth)]) == n_new
        assert s.n_past == prompt.size + n_new - 1  # the last choice needs no row
        ch.free()
        s.free()
    first = runs[(4, 2)]
    for k, v in runs.items():
        assert v == first, k
    # the CPU-choice path: GPU logits, the oracle's (bit-exact) choose on them
    s = m.session(prompt.size + n_new)
    lg = s.prefill(prompt)
    hist, toks = list(prompt), []
    for i in range(n_new):
        t = orc.choose(lg.copy(), 1.1, 20, 0.0, hist)
        toks.append(t)
        hist.append(t)
        if i + 1 < n_new:
            lg = s.step(t)
    assert toks == first
    s.free()
    # teacher-forced against the oracle's own logits
    o = orc.Session(cfg, te, on, layers, prompt.size + n_new)
    ties = []
    teacher_forced(o, o.prefill(prompt), prompt, first, 1.1, 20, ties)
    print(f"\n[tiny decode] {n_new} tokens, near-ties: {ties}")


def test_generate_is_the_cpu_choice_read(dev, tiny):
    """sampling.rs:252-278 generate over TextModel::step with a sampled preset (T 0.7, top-p 0.9, rp 1.1 / 20,
    fp 0.1, seed 1234): the tokens of a step-by-step loop that chooses with the oracle's choose on the GPU's own logits,
    the history, counts and Rng advanced as generate does (every token is stepped, the last one too); an early stop
    from the callback; and with a greedy preset the tokens of the GPU choice (decode_gpu)"""
    cfg, te, on, layers, m = tiny
    prompt = tiny_prompt()
    n = 40
    p = htr.Preset(repetition_penalty=1.1, repetition_window=20, frequency_penalty=0.1, max_new_tokens=n,
                   temperature=0.7, top_p=0.9)
    s = m.session(prompt.size + n)
    s.prefill(prompt)
    toks = s.generate(p, 1234, prompt)
    assert len(toks) == n and s.n_past == prompt.size + n
    s2 = m.session(prompt.size + n)
    lg = s2.prefill(prompt)
    hist, counts, r, want = [int(t) for t in prompt], {}, orc.Rng(1234), []
    for i in range(n):
        t = orc.choose_sampled(lg.copy(), 0.7, 0.9, 1.1, 20, 0.1, hist, counts, r)
        want.append(t)
        hist.append(t)
        counts[t] = counts.get(t, 0) + 1
        lg = s2.step(t)
    assert toks == want
    print(f"\n[generate, sampled] {toks[:12]}…")
    s3 = m.session(prompt.size + n)
    s3.prefill(prompt)
    seen = []
    got = s3.generate(p, 1234, prompt, on_token=lambda t: (seen.append(t), len(seen) < 7)[1])
    assert got == want[:7] and s3.n_past == prompt.size + 6
    greedy = htr.Preset(repetition_penalty=1.1, repetition_window=20, max_new_tokens=30)
    s4 = m.session(prompt.size + 30)
    s4.prefill(prompt)
    g_cpu = s4.generate(greedy, 0, prompt)
    s5 = m.session(prompt.size + 30)
    s5.prefill(prompt)
    ch = s5.choice(greedy, prompt, 4, 2)
    assert g_cpu == s5.decode_gpu(ch, 30)
    ch.free()
    for x in (s, s2, s3, s4, s5):
        x.free()


def test_decode_gpu_stops_when_the_callback_says_so(dev, tiny):
    cfg, te, on, layers, m = tiny
    prompt = tiny_prompt()
    s = m.session(prompt.size + 64)
    s.prefill(prompt)
    ch = s.choice(htr.Preset(max_new_tokens=64), prompt, 4, 2)
    seen = []
    got = s.decode_gpu(ch, 64, lambda t: (seen.append(t), len(seen) < 10)[1])
    assert len(got) == 10 and got == seen
    with pytest.raises(htr.HtrError, match="history holds"):
        s.decode_gpu(ch, 65)
    ch.free()
    s.free()


def test_model_and_session_errors(dev, tiny):
    cfg, te, on, layers, m = tiny
    with pytest.raises(htr.HtrError, match="trained on"):
        m.session(5000)
    s = m.session(8)
    with pytest.raises(htr.HtrError, match="outside the vocabulary"):
        s.prefill([1, 1000])
    with pytest.raises(htr.HtrError, match="overflow"):
        s.prefill(list(range(9)))
    with pytest.raises(htr.HtrError, match="empty prompt"):
        s.prefill([])
    with pytest.raises(htr.HtrError, match="temperature"):
        s.choice(htr.Preset(temperature=0.7), [])
    with pytest.raises(htr.HtrError, match="positive normal"):
        s.choice(htr.Preset(repetition_penalty=1e-45), [])
    with pytest.raises(htr.HtrError, match="run-ahead"):
        s.choice(htr.Preset(), [], 65, 1)
    s.free()
    bad = dict(cfg, d_head=64)
    with pytest.raises(htr.HtrError, match="head dim"):
        htr.TextModel(dev, to_htr_cfg(bad), te, on, layers)


def test_full_size_decoder_matches_oracle(dev):
    """the full model shape (28 layers, dim 1024, 16 / 8 heads, ffn 3072, vocab 151936, tied head) with a 64-token
    prompt and 24 greedy tokens (rp 1.1, window 64): prefill logits and the decode teacher-forced against the oracle"""
    cfg, te, on, layers = synth_text_model()
    m = model_on(dev, htr.COMPUTE_F32, cfg, te, on, layers)
    prompt = (np.abs(htr.synth_normal(77, 64)) * 1e5).astype(np.int64) % cfg["n_vocab"]
    n_new = 24
    s = m.session(prompt.size + n_new)
    lg = s.prefill(prompt)
    o = orc.Session(cfg, te, on, layers, prompt.size + n_new)
    lo = o.prefill(prompt)
    e = rel_l2(lg, lo)
    print(f"\n[full prefill] rel-L2 vs oracle {e:.2e}")
    assert e < 1e-4
    ch = s.choice(htr.Preset(repetition_penalty=1.1, repetition_window=64, max_new_tokens=n_new), prompt, 8, 2)
    toks = s.decode_gpu(ch, n_new)
    ties = []
    teacher_forced(o, lo, prompt, toks, 1.1, 64, ties)
    print(f"[full decode] tokens {toks[:8]}…, near-ties {ties}")
    ch.free()
    s.free()
    m.free()


def test_device_health_is_sticky():
    """gpu.rs:900-961 / 2421-2448: a device marked lost fails every later call with the first reason; the hook
    fires once; an impossible allocation latches outOfMemory (no GPU fault either way)"""
    fired = []
    d = htr.Device(0)
    d.set_fatal_hook(lambda k, m: fired.append((k, m)))
    d.alive()
    with pytest.raises(htr.HtrError):
        d.alloc(1 << 60)
    assert fired and fired[0][0] == "outOfMemory"
    with pytest.raises(htr.HtrError, match="outOfMemory"):
        d.alive()
    with pytest.raises(htr.HtrError, match="outOfMemory"):
        d.alloc(16)
    assert len(fired) == 1
    d.close()
    d = htr.Device(0)
    d.set_fatal_hook(lambda k, m: fired.append((k, m)))
    d.mark_lost("test: device.destroy()")
    for _ in range(2):
        with pytest.raises(htr.HtrError, match="device.destroy"):
            d.sync()
    assert fired[-1] == ("destroyed", "test: device.destroy()") and len(fired) == 2
    d.close()


def test_tiny_prefill_f16_path_matches_oracle(dev):
    """the f16 compute path (MFMA GEMMs on f16 planes; the tiny model's Q / K / V stack 256 + 128 + 128 rows) against
    the oracle's f16-path prefill and the fp64 forward with f16-rounded GEMM operands, then 10 CPU-choice steps"""
    from test_oracle import np_forward

    cfg, te, on, layers = tiny_text_model()
    m = model_on(dev, htr.COMPUTE_F16, cfg, te, on, layers)
    prompt = tiny_prompt()
    s = m.session(prompt.size + 16)
    o = orc.Session(cfg, te, on, layers, prompt.size + 16, f16=True)
    lg, lo = s.prefill(prompt), o.prefill(prompt)
    want16 = np_forward(cfg, te, on, layers, list(prompt), r16=True)[-1]
    eo, e16 = rel_l2(lg, lo), rel_l2(lg, want16)
    print(f"\n[tiny prefill f16] rel-L2 vs oracle {eo:.2e}, vs fp64 (f16 operands) {e16:.2e}")
    assert eo < 5e-3 and e16 < 5e-3
    for i in range(10):
        t = int(np.argmax(lo))
        lg, lo = s.step(t), o.step(t)
        assert rel_l2(lg, lo) < 5e-3, i
    s.free()
    m.free()


def test_f16_path_other_shapes_use_the_rounding_tiled_kernel(dev):
    """a model whose dim (160) is no multiple of 64: the f16 path's GEMMs run the tiled kernel with the same rounding
    (matmul128h_q8_0) — its prefill against the oracle's f16 path"""
    g = orc.Lcg(77)
    dim, n_ff, n_vocab, n_layer = 160, 224, 300, 2

    def w(rows, cols, scale):
        return orc.q8_0_quantize(g.f32(rows * cols, scale))[0]

    def nv(n):
        return (1.0 + g.f32(n, 0.05)).astype(np.float32)

    layers = [{"attn_norm": nv(dim), "q": w(256, dim, 0.2), "k": w(128, dim, 0.2), "v": w(128, dim, 0.2),
               "o": w(dim, 256, 0.1), "q_norm": nv(128), "k_norm": nv(128), "ffn_norm": nv(dim),
               "gate": w(n_ff, dim, 0.2), "up": w(n_ff, dim, 0.2), "down": w(dim, n_ff, 0.1)} for _ in range(n_layer)]
    cfg = {"n_layer": n_layer, "dim": dim, "n_head": 2, "n_kv": 1, "d_head": 128, "n_ff": n_ff, "n_vocab": n_vocab,
           "n_ctx_train": 4096, "eps": 1e-6, "rope_base": 1e6}
    te, on = w(n_vocab, dim, 1.0), nv(dim)
    prompt = [int(t) for t in orc.Lcg(5).bits(24) % n_vocab]
    lo16 = orc.Session(cfg, te, on, layers, 32, f16=True).prefill(prompt)
    lo32 = orc.Session(cfg, te, on, layers, 32).prefill(prompt)
    m = model_on(dev, htr.COMPUTE_F16, cfg, te, on, layers)
    s = m.session(32)
    lg = s.prefill(prompt)
    e, e32 = rel_l2(lg, lo16), rel_l2(lg, lo32)
    print(f"\n[dim 160 prefill f16] rel-L2 vs oracle f16 path {e:.2e}, vs its F32 path {e32:.2e}")
    assert e < 5e-3
    s.free()
    m.free()


def test_full_size_decoder_f16_path_matches_oracle(dev):
    """the full model shape on the f16 path: prefill logits against the oracle's f16-path prefill (bar 1e-2, the path's
    sensitivity), then 16 greedy tokens teacher-forced against the oracle decoding from the same cache (the GPU's rows
    handed over) and the GPU's prefill logits: the first choice is the oracle's choose on those logits"""
    cfg, te, on, layers = synth_text_model()
    m = model_on(dev, htr.COMPUTE_F16, cfg, te, on, layers)
    prompt = (np.abs(htr.synth_normal(78, 64)) * 1e5).astype(np.int64) % cfg["n_vocab"]
    n_new = 16
    s = m.session(prompt.size + n_new)
    lg = s.prefill(prompt)
    o = orc.Session(cfg, te, on, layers, prompt.size + n_new, f16=True)
    lo = o.prefill(prompt)
    e = rel_l2(lg, lo)
    print(f"\n[full prefill f16] rel-L2 vs oracle {e:.2e}")
    assert e < 1e-2
    assert int(np.argmax(lg)) == int(np.argmax(lo)) or near_tie(lo, int(np.argmax(lo)), int(np.argmax(lg)))
    for li in range(cfg["n_layer"]):
        k, v = s.kv_rows(li, 0, prompt.size)
        o.set_kv(li, 0, k, v)
    ch = s.choice(htr.Preset(repetition_penalty=1.1, repetition_window=64, max_new_tokens=n_new), prompt, 8, 2)
    toks = s.decode_gpu(ch, n_new)
    assert len(toks) == n_new
    ties = []
    teacher_forced(o, lg, prompt, toks, 1.1, 64, ties)
    print(f"[full decode f16] tokens {toks[:8]}…, near-ties {ties}")
    ch.free()
    s.free()
    m.free()
