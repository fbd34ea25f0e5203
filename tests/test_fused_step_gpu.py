"""The decode step as one launch per token (token_step.hip) against the per-kernel step and the oracle.

The one-launch step computes what the per-kernel fused step computes (text.rs:540-552 + layers_fused,
text.rs:630-647) with the same arithmetic, except that the split-K attention merge sums its chunks in another order.
So: its KV rows of layer 0 are the per-kernel step's bit for bit (nothing before them differs), later layers' within
f16 rounding; its logits are the per-kernel step's within 1e-5 rel-L2 and the oracle's (stepping from the same cache
rows) within 2e-4 — the per-kernel step's own bar; its greedy tokens are the oracle's, teacher-forced, except logged
near-ties (< 1e-6 relative). Positions cover the chunk edges of the attention phase (64 keys a chunk at n_ctx 2048: 1,
64, 65, 128 keys), a long context (1024 keys) and the last row of the cache (2048 keys, every chunk of every KV head
busy).
"""
import os

import numpy as np
import pytest

import htr
import oracle as orc
from helpers import near_tie, rel_l2, synth_text_model, to_htr_cfg

pytestmark = pytest.mark.gpu

N_LAYER, N_VOCAB, CTX = 3, 4096, 2048


@pytest.fixture(scope="module")
def small_decoder():
    """the decoder's shape (dim 1024, 16 / 8 heads of 128, SwiGLU 3072) with 3 layers and a 4096-id vocabulary"""
    return synth_text_model(n_layer=N_LAYER, n_vocab=N_VOCAB, seed=2024)


@pytest.fixture(scope="module")
def model(dev, small_decoder):
    cfg, te, on, layers = small_decoder
    keep = dev.compute
    dev.compute = htr.COMPUTE_F16
    try:
        m = htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep
    yield m
    m.free()


def hand_over(s, o, n, n_layer):
    for li in range(n_layer):
        k, v = s.kv_rows(li, 0, n)
        o.set_kv(li, 0, k, v)
    o.rewind(n)


def test_fused_step_is_the_default_for_the_decoder_shape(dev, model):
    s = model.session(CTX)
    try:
        if os.environ.get("HTR_FUSED_STEP", "1") != "0":
            assert s.fused_step and s.fused_step_unavailable() is None
        s.fused_step = False
        assert not s.fused_step
        s.fused_step = True
        assert s.fused_step
    finally:
        s.free()


def test_fused_step_refused_where_it_does_not_apply(dev):
    """another shape (the tiny model): the per-kernel step, and the reason"""
    from helpers import tiny_text_model

    cfg, te, on, layers = tiny_text_model()
    keep = dev.compute
    dev.compute = htr.COMPUTE_F16
    try:
        m = htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep
    s = m.session(64)
    assert not s.fused_step and "1024 / 2048 / 3072" in s.fused_step_unavailable()
    with pytest.raises(htr.HtrError, match="not available"):
        s.fused_step = True
    s.free()
    m.free()


def test_fused_step_refused_past_8192_rows(dev, model):
    s = model.session(8193)
    assert not s.fused_step and "8192" in s.fused_step_unavailable()
    s.free()


@pytest.mark.parametrize("n_past", [0, 63, 64, 127, 1023, CTX - 1])
def test_fused_step_matches_per_kernel_step_and_oracle(dev, model, small_decoder, n_past):
    cfg, te, on, layers = small_decoder
    from htr import synth

    prompt = synth.prompt_ids(77, CTX, N_VOCAB)
    sf, sk = model.session(CTX), model.session(CTX)
    sk.fused_step = False
    assert sf.fused_step
    print(f"\n[fused step] position {n_past} ({n_past + 1} keys)", flush=True)
    for s in (sf, sk):
        if n_past:
            s.prefill(prompt[:n_past])
    tok = int(prompt[n_past])
    lf, lk = sf.step(tok), sk.step(tok)
    e_k = rel_l2(lf, lk)
    # layer 0's new rows: the same values; every layer's within f16 rounding
    for li in range(N_LAYER):
        kf, vf = sf.kv_rows(li, n_past, 1)
        kk, vk = sk.kv_rows(li, n_past, 1)
        if li == 0:
            assert np.array_equal(kf, kk) and np.array_equal(vf, vk)
        for a, b in ((kf, kk), (vf, vk)):
            fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
            assert np.all(np.abs(fa - fb) <= 2e-3 * (1 + np.abs(fb))), li
    o = orc.Session(cfg, te, on, layers, CTX, f16=True)
    hand_over(sk, o, n_past, N_LAYER)
    lo = o.step(tok)
    e_o = rel_l2(lf, lo)
    print(f"[fused step] rel-L2 vs the per-kernel step {e_k:.2e}, vs the oracle {e_o:.2e} "
          f"(per-kernel vs oracle {rel_l2(lk, lo):.2e})", flush=True)
    assert e_k < 1e-5
    assert e_o < 2e-4
    sf.free()
    sk.free()


@pytest.mark.parametrize("n_ctx,n_past", [(1000, 999), (1000, 500), (1536, 1535), (1536, 1100), (1536, 1008),
                                          (1536, 1011), (3072, 3071),
                                          (3072, 2000), (4096, 4095), (4096, 2100), (6144, 6143), (6144, 4000),
                                          (8192, 8191), (8192, 5000)])
def test_fused_step_other_chunk_sizes(dev, model, small_decoder, n_ctx, n_past):
    """the other instances of the attention phase: chunks of 32 keys (caches ≤ 1024 rows), 48 (≤ 1536; 3 keys a
    thread, its scores padded to 4), 96 (≤ 3072; 6, padded to 8), 128 (≤ 4096), 192 (≤ 6144; 12, padded to 16) and
    256 (≤ 8192), at the cache's last row and inside it (at 1009 and 1012 keys the last 48-key chunk holds 1 and 4
    keys: its waves past the first have no key, maximum −inf) — against the per-kernel step and the oracle as above"""
    cfg, te, on, layers = small_decoder
    from htr import synth

    prompt = synth.prompt_ids(n_ctx + n_past, n_past + 1, N_VOCAB)
    sf, sk = model.session(n_ctx), model.session(n_ctx)
    sk.fused_step = False
    assert sf.fused_step
    print(f"\n[fused step] {n_ctx}-row cache, position {n_past}", flush=True)
    for s in (sf, sk):
        s.prefill(prompt[:n_past])
    tok = int(prompt[n_past])
    lf = sf.step(tok)
    ni = next(ni for ni in (2, 3, 4, 6, 8, 12, 16) if n_ctx <= 512 * ni)  # the smallest chunks that cover the cache
    assert dev.last_kernel() == f"k_decode_token<{ni}>"
    lk = sk.step(tok)
    o = orc.Session(cfg, te, on, layers, n_ctx, f16=True)
    hand_over(sk, o, n_past, N_LAYER)
    lo = o.step(tok)
    e_k, e_o = rel_l2(lf, lk), rel_l2(lf, lo)
    print(f"[fused step] rel-L2 vs the per-kernel step {e_k:.2e}, vs the oracle {e_o:.2e}", flush=True)
    assert e_k < 1e-5 and e_o < 2e-4
    kf, vf = sf.kv_rows(0, n_past, 1)
    kk, vk = sk.kv_rows(0, n_past, 1)
    assert np.array_equal(kf, kk) and np.array_equal(vf, vk)
    sf.free()
    sk.free()


@pytest.mark.parametrize("rp,window,fp", [(1.1, 64, 0.0), (1.3, 16, 0.4)], ids=["rp1.1_w64", "rp1.3_w16_fp0.4"])
def test_fused_decode_gpu_teacher_forced(dev, model, small_decoder, rp, window, fp):
    """decode_gpu on the one-launch step (a graph of 16 launches, each the step with the LM head and the choice in
    its tail, 2 in flight) and on the per-kernel step: 96 greedy tokens after a 700-token prompt, each the oracle's
    choice (sampling.rs:38-62: penalty over the window, frequency penalty over the read's counts) given the read's
    earlier ones (near-ties logged); the read's last logits are the oracle's, with the window penalty applied in place
    (the frequency penalty only compared, as the reference's GPU choice does)"""
    cfg, te, on, layers = small_decoder
    from htr import synth

    prompt = synth.prompt_ids(91, 700, N_VOCAB)
    new = 96
    reads = []
    for fused in (True, False):
        s = model.session(CTX)
        s.fused_step = fused
        s.prefill(prompt[:-1])
        first = s.step(int(prompt[-1]))
        ch = s.choice(htr.Preset(repetition_penalty=rp, repetition_window=window, frequency_penalty=fp,
                                 max_new_tokens=new), prompt, chunk=16, depth=2)
        toks = s.decode_gpu(ch, new)
        assert len(toks) == new and s.n_past == len(prompt) + new - 1
        last = s.logits()
        o = orc.Session(cfg, te, on, layers, CTX, f16=True)
        hand_over(s, o, len(prompt) - 1, N_LAYER)
        ch.free()
        s.free()
        lo = o.step(int(prompt[-1]))
        assert rel_l2(first, lo) < 2e-4
        hist, ties, counts = [int(t) for t in prompt], [], {}
        for i, t in enumerate(toks):
            if i + 1 == len(toks):  # the session's logits after the read: rp applied in place, fp only compared
                pen_rp = lo.copy()  # (choose_max.wgsl:5-7, 39)
                orc.choose(pen_rp, rp, window, 0.0, hist)
            pen = lo.copy()
            want = orc.choose(pen, rp, window, fp, hist, counts)
            if want != t:
                assert near_tie(pen, want, t), f"{'fused' if fused else 'per-kernel'} token {i}: oracle {want}, GPU {t}"
                ties.append(i)
            hist.append(int(t))
            counts[int(t)] = counts.get(int(t), 0) + 1
            if i + 1 < len(toks):
                lo = o.step(int(t))
        assert rel_l2(last, pen_rp) < 2e-4
        reads.append(list(toks))
        print(f"\n[{'fused' if fused else 'per-kernel'} decode] {new} tokens teacher-forced, near-ties {ties}",
              flush=True)
    print(f"[decode] the two reads agree: {reads[0] == reads[1]}", flush=True)


def test_fused_step_profile_stamps(dev, model):
    from htr import synth

    s = model.session(CTX)
    s.prefill(synth.prompt_ids(5, 1279, N_VOCAB))
    us = s.profile_fused_step(17)
    assert us.shape == (1 + 12 * N_LAYER + 3,) and us[0] == 0.0
    assert np.all(np.diff(us) >= 0.0) and us[-1] < 1e4
    print(f"\n[fused step] stamps (µs): {np.round(us, 2).tolist()}", flush=True)
    assert s.n_past == 1279
    s.free()


def test_fused_step_recovers_from_a_wait_that_ran_out(dev, model, monkeypatch):
    """a 1 µs limit (HTR_FUSED_SPIN_US, read when the session is made): every wait of the one-launch step runs out, the
    launch still ends, and the step is redone on the per-kernel step, which the session keeps (with the reason) — its
    logits are then the per-kernel session's bit for bit. The measurement entry (profile_fused_step) reports the error
    instead. With the normal limit and set_fused_step(1) the session steps in one launch again."""
    from htr import synth

    prompt = synth.prompt_ids(3, 40, N_VOCAB)
    monkeypatch.setenv("HTR_FUSED_SPIN_US", "1")
    s = model.session(CTX)
    monkeypatch.delenv("HTR_FUSED_SPIN_US")
    sk = model.session(CTX)
    sk.fused_step = False
    assert s.fused_step
    for x in (s, sk):
        x.prefill(prompt[:-2])
    with pytest.raises(htr.HtrError, match="waited past its limit"):
        s.profile_fused_step(int(prompt[-2]))
    assert s.fused_step  # a measurement does not switch the form
    a, b = s.step(int(prompt[-2])), sk.step(int(prompt[-2]))
    assert not s.fused_step and "ran past its limit" in s.fused_step_unavailable()
    assert np.array_equal(a, b) and s.n_past == sk.n_past == len(prompt) - 1
    s.set_wait_limit(None)
    s.fused_step = True
    assert s.fused_step and s.fused_step_unavailable() is None
    # a session whose row 38 the per-kernel step wrote as well: the next one-launch steps agree bit for bit
    s2 = model.session(CTX)
    s2.prefill(prompt[:-2])
    s2.fused_step = False
    s2.step(int(prompt[-2]))
    s2.fused_step = True
    assert np.array_equal(s.step(int(prompt[-1])), s2.step(int(prompt[-1])))  # the one-launch step, as before
    assert s.fused_step and dev.last_kernel().startswith("k_decode_token<")
    for x in (s, sk, s2):
        x.free()


@pytest.mark.parametrize("where", ["first_chunk", "mid_read"])
def test_fused_decode_gpu_recovers_from_a_wait_that_ran_out(dev, model, small_decoder, where, monkeypatch):
    """decode_gpu (chunk 16, depth 2, rp 1.3 over 16 with fp 0.4) when waits of the one-launch step run out: in the
    first chunk (a 1 µs limit from the session's start; the read's first choice is the choice kernel's, on the
    prefill's logits) or in the third (the limit set to 1 µs from on_token at the read's 6th token: the chunks recorded
    after it carry it). No id of a failed chunk reaches on_token; the read goes on from the chunk's first step on the
    per-kernel step, with the frequency counts, position and token rewound. So: 96 ids, each passed once; in the first
    case the whole read is the per-kernel session's read; in both, every id is the oracle's choice given the earlier
    ones (teacher-forced from the GPU's prefill rows; near-ties logged), the session on the per-kernel step after."""
    cfg, te, on, layers = small_decoder
    from htr import synth

    prompt = synth.prompt_ids(92, 600, N_VOCAB)
    rp, window, fp, new = 1.3, 16, 0.4, 96
    preset = htr.Preset(repetition_penalty=rp, repetition_window=window, frequency_penalty=fp, max_new_tokens=new)
    if where == "first_chunk":
        monkeypatch.setenv("HTR_FUSED_SPIN_US", "1")
    s = model.session(CTX)
    monkeypatch.delenv("HTR_FUSED_SPIN_US", raising=False)
    assert s.fused_step
    s.prefill(prompt)
    ch = s.choice(preset, prompt, chunk=16, depth=2)
    seen = []

    def on_token(t):
        seen.append(t)
        if where == "mid_read" and len(seen) == 6:
            s.set_wait_limit(1.0)
        return True

    toks = s.decode_gpu(ch, new, on_token)
    assert toks == seen and len(toks) == new and s.n_past == len(prompt) + new - 1
    assert not s.fused_step and "ran past its limit" in s.fused_step_unavailable()
    ch.free()
    # the per-kernel read from the same prefill
    sk = model.session(CTX)
    sk.fused_step = False
    sk.prefill(prompt)
    chk = sk.choice(preset, prompt, chunk=16, depth=2)
    ref = sk.decode_gpu(chk, new)
    chk.free()
    if where == "first_chunk":
        assert toks == ref
    # teacher-forced: every id the oracle's choice given the read's earlier ones
    o = orc.Session(cfg, te, on, layers, CTX, f16=True)
    hand_over(s, o, len(prompt), N_LAYER)
    o.rewind(len(prompt) - 1)
    lo = o.step(int(prompt[-1]))
    hist, counts, ties = [int(t) for t in prompt], {}, []
    for i, t in enumerate(toks):
        pen = lo.copy()
        want = orc.choose(pen, rp, window, fp, hist, counts)
        if want != t:
            assert near_tie(pen, want, t), f"{where}: token {i}: oracle {want}, GPU {t}"
            ties.append(i)
        hist.append(int(t))
        counts[int(t)] = counts.get(int(t), 0) + 1
        if i + 1 < len(toks):
            lo = o.step(int(t))
    print(f"\n[recovery, {where}] {new} ids teacher-forced (near-ties {ties}); the per-kernel read's: "
          f"{toks == ref}", flush=True)
    s.free()
    sk.free()


def test_fused_step_refused_for_a_small_vocabulary(dev):
    """the LM-head tail gives each of the 256 workgroups at least one row: a decoder of the right shape with 100 ids
    steps kernel by kernel, and says why"""
    cfg, te, on, layers = synth_text_model(n_layer=1, n_vocab=100, seed=77)
    keep = dev.compute
    dev.compute = htr.COMPUTE_F16
    try:
        m = htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep
    s = m.session(64)
    assert not s.fused_step and "256 to 262144 ids" in s.fused_step_unavailable()
    s.prefill(np.arange(10, dtype=np.int32))
    assert np.all(np.isfinite(s.step(11)))
    s.free()
    m.free()


def test_fused_step_at_its_shape_limits(dev):
    """42 layers (the stamp table's size) and 262,144 vocabulary ids (1024 LM-head rows a workgroup, the window marks'
    size): the step against the per-kernel step, the GPU choice's tokens with a window that marks the last row of a
    workgroup's share, and the profile's 1 + 12·42 + 3 stamps; 43 layers are refused with the reason"""
    from htr import synth

    cfg, te, on, layers = synth_text_model(n_layer=42, n_vocab=262144, seed=4242)
    keep = dev.compute
    dev.compute = htr.COMPUTE_F16
    try:
        m = htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep
    try:
        prompt = synth.prompt_ids(17, 300, cfg["n_vocab"])
        prompt[-5:] = [1023, 2047, 262143, 0, 1024]  # ids at the edges of the workgroups' row shares
        sf, sk = m.session(512), m.session(512)
        sk.fused_step = False
        assert sf.fused_step
        for s in (sf, sk):
            s.prefill(prompt[:-1])
        lf, lk = sf.step(int(prompt[-1])), sk.step(int(prompt[-1]))
        assert rel_l2(lf, lk) < 1e-5
        toks = []
        for s in (sf, sk):
            s.rewind(len(prompt) - 1)
            first = s.step(int(prompt[-1]))
            ch = s.choice(htr.Preset(repetition_penalty=1.3, repetition_window=64, max_new_tokens=48), prompt,
                          chunk=8, depth=2)
            toks.append(s.decode_gpu(ch, 48))
            ch.free()
            # every token the oracle's choice given the read's earlier ones (teacher-forced from the GPU's rows)
            o = orc.Session(cfg, te, on, layers, 512, f16=True)
            hand_over(s, o, len(prompt) - 1, cfg["n_layer"])
            lo = o.step(int(prompt[-1]))
            assert rel_l2(first, lo) < 2e-4
            hist, ties = [int(t) for t in prompt], []
            for i, t in enumerate(toks[-1]):
                pen = lo.copy()
                want = orc.choose(pen, 1.3, 64, 0.0, hist)
                if want != t:
                    assert near_tie(pen, want, t), f"{'fused' if s is sf else 'per-kernel'} token {i}: {want} vs {t}"
                    ties.append(i)
                hist.append(int(t))
                if i + 1 < len(toks[-1]):
                    lo = o.step(int(t))
            del o
            print(f"\n[fused step, 42 layers, 262144 ids] {'one-launch' if s is sf else 'per-kernel'} read: 48 tokens "
                  f"teacher-forced, near-ties {ties}", flush=True)
        print(f"[fused step, 42 layers, 262144 ids] the two forms' tokens agree: {toks[0] == toks[1]}", flush=True)
        sf.rewind(200)
        us = sf.profile_fused_step(int(prompt[200]))
        assert us.shape == (1 + 12 * 42 + 3,) and np.all(np.diff(us) >= 0.0)
        sf.free()
        sk.free()
    finally:
        m.free()
    cfg43, te43, on43, layers43 = synth_text_model(n_layer=43, n_vocab=4096, seed=43)
    keep = dev.compute
    dev.compute = htr.COMPUTE_F16
    try:
        m43 = htr.TextModel(dev, to_htr_cfg(cfg43), te43, on43, layers43)
    finally:
        dev.compute = keep
    s43 = m43.session(64)
    assert not s43.fused_step and "1024 / 2048 / 3072" in s43.fused_step_unavailable()
    s43.free()
    m43.free()
