"""A KV cache grown with the read (Session::reserve, text.rs:287-327) against one sized up front.

Follows kv_growth_matches_presized_cache (text.rs:1325-1379): the tiny model, its 20-token LCG prompt, 40 steps of the
CPU-choice path (greedy on the read-back logits) and 150 tokens of the GPU choice run ahead (4 choices a launch, 2
launches in flight), for growths of n_ctx, 1, 3 and 61 rows — inside a run-ahead launch's window, across the
attention's key chunks. Every logits row is the presized session's bit for bit and the tokens are the same; the cache
holds the rows reserved (prompt + grow after the prefill, at most grow past the read at its end), counted in the
device's KV ledger, and is gone with the session. On both compute paths, and on the decoder's shape, whose sessions
step by one launch per token (the layer table and the cache's row stride follow each growth).
"""
import numpy as np
import pytest

import htr
from helpers import synth_text_model, tiny_prompt, tiny_text_model, to_htr_cfg

pytestmark = pytest.mark.gpu

N_NEW, N_STEPS = 150, 40


def make_model(dev, compute, which):
    cfg, te, on, layers = tiny_text_model() if which == "tiny" else synth_text_model(n_layer=3, n_vocab=4096, seed=77)
    keep = dev.compute
    dev.compute = compute
    try:
        return htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep


@pytest.mark.parametrize("compute,which", [(htr.COMPUTE_F32, "tiny"), (htr.COMPUTE_F16, "tiny"),
                                           (htr.COMPUTE_F16, "decoder")], ids=["f32_tiny", "f16_tiny", "f16_decoder"])
def test_kv_growth_matches_presized_cache(dev, compute, which):
    m = make_model(dev, compute, which)
    c = m.cfg
    prompt = tiny_prompt(20) % c.n_vocab
    n_ctx = len(prompt) + N_NEW
    row_bytes = 2 * c.n_layer * c.n_kv * c.d_head * 2
    base_kv = dev.mem_live()["kv_cache"]
    want = None
    try:
        for grow in (None, n_ctx, 1, 3, 61):  # None: htr_session_create, the whole cache at once
            print(f"\n[kv growth] {which}, compute {compute}, grow {grow}", flush=True)
            s = m.session(n_ctx, grow)
            fused = s.fused_step
            if which == "decoder":
                assert fused, s.fused_step_unavailable()
            assert s.reserved_rows == (n_ctx if grow is None else 0)
            logits = [s.prefill(prompt)]
            assert s.reserved_rows == (n_ctx if grow is None else min(len(prompt) + grow, n_ctx)), grow
            for _ in range(N_STEPS):
                logits.append(s.step(int(np.argmax(logits[-1]))))
            assert dev.mem_live()["kv_cache"] - base_kv == s.reserved_rows * row_bytes, grow
            s.free()
            assert dev.mem_live()["kv_cache"] == base_kv, f"grow {grow}: the KV cache outlived its session"

            s = m.session(n_ctx, grow)
            s.prefill(prompt)
            ch = s.choice(htr.Preset(repetition_penalty=1.1, repetition_window=20, frequency_penalty=0.0,
                                     max_new_tokens=N_NEW), prompt, chunk=4, depth=2)
            toks = s.decode_gpu(ch, N_NEW)
            assert len(toks) == N_NEW
            # the last choice needs no row; the cache holds at most `grow` rows past the read
            assert s.n_past == n_ctx - 1, grow
            if grow is not None:
                assert s.n_past <= s.reserved_rows <= min(s.n_past + grow, n_ctx), (grow, s.reserved_rows)
            last = s.logits()
            ch.free()
            s.free()
            assert dev.mem_live()["kv_cache"] == base_kv
            if want is None:
                want = (logits, toks, last)
                continue
            for i, (a, b) in enumerate(zip(want[0], logits)):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"grow {grow}: logits of step {i} differ"
            assert want[1] == toks, f"grow {grow}: the GPU-chosen tokens differ"
            assert np.array_equal(want[2].view(np.uint32), last.view(np.uint32)), f"grow {grow}: the last logits"
            print(f"[kv growth] grow {grow}: {N_STEPS + 1} logits rows and {N_NEW} tokens as presized "
                  f"(one-launch step: {fused})", flush=True)
    finally:
        m.free()


def test_kv_growth_of_zero_rows_refused(dev):
    m = make_model(dev, htr.COMPUTE_F16, "tiny")
    try:
        with pytest.raises(htr.HtrError, match="growth of 0 rows"):
            m.session(64, 0)
    finally:
        m.free()


def test_kv_growth_under_the_sampled_read(dev):
    """the CPU-choice read with a sampled preset (sampling.rs:252-278; T 0.7, top-p 0.9, seed 1234) on a cache that
    grows every 3 rows: the tokens of a presized cache, and the cache holds at most 3 rows past the read"""
    m = make_model(dev, htr.COMPUTE_F16, "tiny")
    try:
        prompt = tiny_prompt(20)
        n = 40
        p = htr.Preset(repetition_penalty=1.1, repetition_window=20, frequency_penalty=0.1, max_new_tokens=n,
                       temperature=0.7, top_p=0.9)
        got = []
        for grow in (None, 3):
            s = m.session(prompt.size + n, grow)
            s.prefill(prompt)
            got.append(s.generate(p, 1234, prompt))
            assert s.n_past == prompt.size + n
            if grow is not None:
                assert s.n_past <= s.reserved_rows <= s.n_past + grow
            s.free()
        assert got[0] == got[1] and len(got[0]) == n
    finally:
        m.free()
