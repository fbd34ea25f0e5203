"""The 28-layer decoder at the measured workload: the bench's own read, token for token against the oracle.

The read (bench.py's decode leg; TextModel::prefill + step + decode_gpu, text.rs:437-625): the Qwen3-0.6B-shaped
random q8_0 decoder, a 1024-token prompt of uniform ids (seed 4242), prefill of the first 1023, one step for the last,
then 512 GPU-chosen greedy tokens with the repetition penalty 1.1 over a 64-token window, 16 choices a graph launch, 2
launches in flight, a 1536-row session — on the default f16 compute path, and again on the F32 path.

What each part is held to:
  - the prefill logits against the oracle's prefill of the same path: rel-L2 ≤ 1e-2 on the f16 path (the path's own
    sensitivity to f16 rounding: a 2e-7 nudge of one norm moves the oracle's f16 prefill by 1.9e-3 on this shape) and
    ≤ 1e-4 on the F32 path (exact q8_0 values, f32 sums in two orders);
  - the decode (what the bench times) from the same cache: the GPU's rows 0 … 1022 are handed to the oracle, which
    then steps with its own arithmetic. On the f16 path the read runs on the one-launch step (k_decode_token<3>: 48-key
    attention chunks at the 1536-row cache, 22 and 32 of them busy a KV head at 1024 and 1535 keys), which the test
    asserts; on the F32 path the per-kernel step. The step for the prompt's last token and the last step of the read
    (1024 and 1535 keys) match the oracle's logits at rel-L2 ≤ 2e-4; every
    one of the 512 tokens is the oracle's choice given the GPU's earlier tokens (teacher-forced), except documented
    near-ties (the oracle's logits of the two tokens within 1e-6 relative), which are printed.
"""
import numpy as np
import pytest

import htr
import oracle as orc
from helpers import near_tie, rel_l2, synth_text_model, to_htr_cfg

pytestmark = pytest.mark.gpu

PROMPT, NEW, CTX, RP, WINDOW = 1024, 512, 1536, 1.1, 64


@pytest.fixture(scope="module")
def decoder():
    from htr import synth

    cfg, te, on, layers = synth_text_model()
    return cfg, te, on, layers, synth.prompt_ids(4242, PROMPT, cfg["n_vocab"])


def model_on(dev, path, cfg, te, on, layers):
    keep = dev.compute
    dev.compute = path
    try:
        return htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep


def hand_over(s: htr.Session, o: orc.Session, n: int, n_layer: int) -> None:
    """the GPU session's cache rows 0 … n − 1 of every layer into the oracle's session, which is rewound to n"""
    for li in range(n_layer):
        k, v = s.kv_rows(li, 0, n)
        o.set_kv(li, 0, k, v)
    o.rewind(n)


def teacher_forced(o: orc.Session, first, prompt, toks, ties):
    """the oracle's choice at every position given the GPU's earlier tokens; → the last position's penalised logits"""
    lo, hist, pen = first, [int(t) for t in prompt], None
    for i, t in enumerate(toks):
        pen = lo.copy()
        want = orc.choose(pen, RP, WINDOW, 0.0, hist)
        if want != t:
            assert near_tie(pen, want, t), f"token {i}: oracle {want} ({pen[want]!r}), GPU {t} ({pen[t]!r})"
            ties.append((i, want, t, float(pen[want]), float(pen[t])))
        hist.append(int(t))
        if i + 1 < len(toks):
            lo = o.step(int(t))
    return pen


@pytest.mark.parametrize("path", [htr.COMPUTE_F16, htr.COMPUTE_F32], ids=["f16_path", "f32_path"])
def test_config3_read_matches_oracle(dev, decoder, path):
    cfg, te, on, layers, prompt = decoder
    f16 = path == htr.COMPUTE_F16
    print(f"\n[config 3] {'f16' if f16 else 'F32'} path: prefill {PROMPT - 1}, step, {NEW} tokens", flush=True)
    m = model_on(dev, path, cfg, te, on, layers)
    s = m.session(CTX)
    lg = s.prefill(prompt[:-1])
    o = orc.Session(cfg, te, on, layers, CTX, f16=f16)
    lo = o.prefill(prompt[:-1])
    e = rel_l2(lg, lo)
    print(f"[config 3] prefill logits rel-L2 vs the oracle {e:.2e}", flush=True)
    assert e < (1e-2 if f16 else 1e-4)
    # the rows the oracle's own prefill stored are the GPU's within f16 rounding (one layer shown: the first)
    ko, vo = o.get_kv(0, 0, PROMPT - 1)
    kg, vg = s.kv_rows(0, 0, PROMPT - 1)
    for a, b in ((kg, ko), (vg, vo)):
        fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
        assert rel_l2(fa, fb) < (2e-2 if f16 else 1e-3)
    hand_over(s, o, PROMPT - 1, cfg["n_layer"])
    lg1, lo1 = s.step(int(prompt[-1])), o.step(int(prompt[-1]))
    e1 = rel_l2(lg1, lo1)
    print(f"[config 3] step at position {PROMPT - 1} (1024 keys): rel-L2 {e1:.2e}", flush=True)
    assert e1 < 2e-4
    ch = s.choice(htr.Preset(repetition_penalty=RP, repetition_window=WINDOW, max_new_tokens=NEW), prompt, chunk=16,
                  depth=2)
    toks = s.decode_gpu(ch, NEW)
    assert len(toks) == NEW and s.n_past == PROMPT + NEW - 1
    # the form that made the choices: the one-launch step on the f16 path (and it stayed on it), kernels on F32
    assert s.fused_step == f16
    if f16:
        assert dev.last_kernel() == "k_decode_token<3>"
    ties = []
    pen = teacher_forced(o, lo1, prompt, toks, ties)
    # the read's last logits (position 1534, 1535 keys), penalised in place by the last choice on both sides
    e_last = rel_l2(s.logits(), pen)
    print(f"[config 3] {NEW} tokens teacher-forced, first {toks[:8]}; near-ties {ties}; last step rel-L2 "
          f"{e_last:.2e}", flush=True)
    assert e_last < 2e-4
    # CPU-choice steps at later positions of the same session (TextModel::step): rewound to 1400, 4 steps
    s.rewind(1400)
    o.rewind(1400)
    for t in toks[400:404]:
        a, b = s.step(t), o.step(t)
        assert rel_l2(a, b) < 2e-4
    ch.free()
    s.free()
    m.free()


def test_fused_attention_ignores_stale_rows_past_the_position(dev):
    """a rewound session whose cache still holds old rows at and after the position (here planted: V = +inf, K = NaN
    from the position to the end of its 16-key chunk): the step's fused attention stores the new row and reads no
    stale one — its logits are finite and the oracle's, stepping from the same rows 0 … pos − 1 (attn_decode.wgsl:82-89
    reads V below n_keys only)"""
    from helpers import tiny_prompt, tiny_text_model

    cfg, te, on, layers = tiny_text_model()
    m = model_on(dev, htr.COMPUTE_F16, cfg, te, on, layers)
    s = m.session(200)
    prompt = np.concatenate([tiny_prompt(), tiny_prompt(40) + 1]) % cfg["n_vocab"]
    s.prefill(prompt)  # 60 positions
    pos = 50
    s.rewind(pos)
    kvd = cfg["n_kv"] * 128
    n_bad = 64 - pos  # rows 50 … 63: the rest of the chunk of 16 keys that holds position 50
    kbad = np.full((n_bad, kvd), 0x7E00, np.uint16)  # f16 NaN
    vbad = np.full((n_bad, kvd), 0x7C00, np.uint16)  # f16 +inf
    for li in range(cfg["n_layer"]):
        s.set_kv_rows(li, pos, kbad, vbad)
    o = orc.Session(cfg, te, on, layers, 200, f16=True)
    hand_over(s, o, pos, cfg["n_layer"])
    tok = int(prompt[pos])
    lg, lo = s.step(tok), o.step(tok)
    assert np.all(np.isfinite(lg))
    e = rel_l2(lg, lo)
    print(f"\n[stale rows] step at {pos} over planted inf / NaN rows: rel-L2 vs the oracle {e:.2e}")
    assert e < 2e-4
    # the new row is stored (finite, the oracle's within one f16 rounding); the planted rows after it are untouched
    for li in range(cfg["n_layer"]):
        kg, vg = s.kv_rows(li, pos, 2)
        ko, vo = o.get_kv(li, pos, 1)
        for a, b in ((kg[0], ko[0]), (vg[0], vo[0])):
            fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
            assert np.all(np.isfinite(fa)) and np.all(np.abs(fa - fb) <= 2e-3 * (1 + np.abs(fb)))
        assert np.array_equal(kg[1], kbad[1]) and np.array_equal(vg[1], vbad[1])
    s.free()
    m.free()


def test_fused_step_ignores_stale_rows_past_the_position(dev):
    """the same on the one-launch step (the decoder's shape, 3 layers, a 1536-row cache: 48-key chunks): a session
    rewound to 1000 with K = NaN and V = +inf planted from the position to the end of its chunk (rows 1000 … 1007) —
    the step's logits are finite and the oracle's, its new row stored, the planted rows after it untouched"""
    from htr import synth

    cfg, te, on, layers = synth_text_model(n_layer=3, n_vocab=4096, seed=2024)
    m = model_on(dev, htr.COMPUTE_F16, cfg, te, on, layers)
    s = m.session(CTX)
    assert s.fused_step
    prompt = synth.prompt_ids(17, 1100, cfg["n_vocab"])
    s.prefill(prompt)
    pos = 1000
    s.rewind(pos)
    kvd = cfg["n_kv"] * 128
    n_bad = 1008 - pos  # the rest of the 48-key chunk 960 … 1007 that holds position 1000
    kbad = np.full((n_bad, kvd), 0x7E00, np.uint16)
    vbad = np.full((n_bad, kvd), 0x7C00, np.uint16)
    for li in range(cfg["n_layer"]):
        s.set_kv_rows(li, pos, kbad, vbad)
    o = orc.Session(cfg, te, on, layers, CTX, f16=True)
    hand_over(s, o, pos, cfg["n_layer"])
    tok = int(prompt[pos])
    lg, lo = s.step(tok), o.step(tok)
    assert dev.last_kernel() == "k_decode_token<3>" and s.fused_step
    assert np.all(np.isfinite(lg))
    e = rel_l2(lg, lo)
    print(f"\n[stale rows, one-launch step] step at {pos} over planted inf / NaN rows: rel-L2 vs the oracle {e:.2e}")
    assert e < 2e-4
    for li in range(cfg["n_layer"]):
        kg, vg = s.kv_rows(li, pos, n_bad)
        ko, vo = o.get_kv(li, pos, 1)
        for a, b in ((kg[0], ko[0]), (vg[0], vo[0])):
            fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
            assert np.all(np.isfinite(fa)) and np.all(np.abs(fa - fb) <= 2e-3 * (1 + np.abs(fb)))
        assert np.array_equal(kg[1:], kbad[1:]) and np.array_equal(vg[1:], vbad[1:])
    s.free()
    m.free()
