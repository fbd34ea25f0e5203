"""The one-launch decode step's own token choice (k_decode_token's tail: LM head, window penalty, frequency penalty,
first maximum) on the reference's edge cases, bit for bit.

The reference pins its GPU choice with gpu_choice_matches_choose (text.rs:1001-1054): exact ties, ±0, −inf, NaN,
penalty reversal and fp against ocr-decode's choose (sampling.rs:38-62). The decode's headline read makes its choices
in the one-launch step's tail, so the same cases are driven through it here, with LM-head weights that force them:

  - how each choice is checked: a twin session of the same model, stepped by htr_step on the one-launch step (the same
    kernel without the choice: same cache rows, same arithmetic) with the read's own tokens, gives the exact logits the
    tail chose from. Every token of decode_gpu (chunk 16, depth 2) must be the oracle's choose on those logits — no
    near-tie exemption — and the choice kernel's (k_choose) on the same logits and window; the read's last logits, which
    the tail penalises in place, must be the oracle's penalised ones bit for bit;
  - a random decoder of the decoder's shape whose token_embd holds duplicated rows with a large scale (exact ties: the
    LM head's wave sum pairs lanes the same way for every row, so equal rows give equal bits) inside one workgroup's
    share of the vocabulary and across two shares (ids 15 / 16, 2047 / 2048), at ids 0 and n_vocab − 1, inside one
    wave and across waves — the ties the 256 workgroups' best keys must resolve to the lower id;
  - a designed model (every layer weight zero, so the residual at the LM head is the token's own embedding, and sparse
    small-integer embedding rows): exact ties everywhere, maxima of +0 (the output norm's negative weights make every
    overlapping row negative), penalty reversal, rows whose logit is always NaN (an infinite scale on zero quants) or
    −inf (an f32 overflow), the frequency penalty, rp below 1;
  - NaN at index 0: the reference's choose returns 0 (its first maximum starts there), so does the tail.

The same zero-layer construction pins the embedding gather on its own: the LM head's input is then the gathered row.
"""
import numpy as np
import pytest

import htr
import oracle as orc
from helpers import rel_l2, synth_text_model, to_htr_cfg

pytestmark = pytest.mark.gpu

N_LAYER, N_VOCAB, DIM, CTX = 3, 4096, 1024, 512


def f16_bytes(v: float) -> tuple[int, int]:
    b = np.array([v], np.float16).view(np.uint8)
    return int(b[0]), int(b[1])


def blocks_of(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """q8_0 blocks (ocr-gguf lib.rs:128-135: f16 scale, 32 int8) of rows q int8 [n][K] with one scale a row"""
    n, k = q.shape
    b = np.zeros((n, k // 32, 34), np.uint8)
    b[:, :, :2] = np.array(d, np.float16).view(np.uint8).reshape(n, 1, 2)
    b[:, :, 2:] = q.reshape(n, k // 32, 32).view(np.uint8)
    return b.reshape(-1)


def make_model(dev, cfg, te, on, layers):
    keep = dev.compute
    dev.compute = htr.COMPUTE_F16
    try:
        return htr.TextModel(dev, to_htr_cfg(cfg), te, on, layers)
    finally:
        dev.compute = keep


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """equal f32 bits, any two NaNs counted equal"""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | both_nan))


def read_and_check(dev, m, prompt, rp, window, fp, n_new, label):
    """decode_gpu on the one-launch step, every choice checked against the oracle's and the choice kernel's on the
    twin session's logits; → coverage counts"""
    sa, sb = m.session(CTX), m.session(CTX)
    assert sa.fused_step and sb.fused_step
    for s in (sa, sb):
        s.prefill(prompt[:-1])
    sa.step(int(prompt[-1]))
    preset = htr.Preset(repetition_penalty=rp, repetition_window=window, frequency_penalty=fp, max_new_tokens=n_new)
    ch = sa.choice(preset, prompt, chunk=16, depth=2)
    toks = sa.decode_gpu(ch, n_new)
    assert dev.last_kernel().startswith("k_decode_token<") and sa.fused_step
    last = sa.logits()
    ch.free()
    sa.free()
    # the choice kernel on the same logits: its own window (the seed ids and the read's tokens) and counts
    lg_d = dev.alloc(N_VOCAB * 4)
    hist_d = dev.alloc((len(prompt) + n_new) * 4)
    tok_d = dev.alloc(4)
    cnt_d, fpen_d = dev.alloc(N_VOCAB * 4), dev.alloc(N_VOCAB * 4)
    hist, counts = [int(t) for t in prompt], {}
    cov = {"tied_max": 0, "zero_max": 0, "reversed": 0, "nan": 0, "neg_inf": 0, "ties_across_shares": 0}
    lo = sb.step(int(prompt[-1]))
    for i, t in enumerate(toks):
        pen = lo.copy()
        want = orc.choose(pen, rp, window, fp, hist, counts)
        assert t == want, f"{label} token {i}: the one-launch step chose {t}, the oracle {want}"
        # the choice kernel (k_choose) on the same logits, window and counts
        lg_d.upload(lo)
        hist_d.upload(np.array(hist, np.uint32))
        c = np.zeros(N_VOCAB, np.uint32)
        f = np.zeros(N_VOCAB, np.float32)
        for k, v in counts.items():
            c[k], f[k] = v, np.float32(fp) * np.float32(v)
        cnt_d.upload(c)
        fpen_d.upload(f)
        htr.choose(dev, lg_d, N_VOCAB, hist_d, len(hist), window, rp, tok_d, fp, cnt_d if fp else None,
                   fpen_d if fp else None)
        assert int(tok_d.download(np.uint32, 1)[0]) == t, f"{label} token {i}: the choice kernel differs"
        top = np.flatnonzero(pen == pen[t])
        cov["tied_max"] += top.size >= 2
        cov["ties_across_shares"] += len({int(x) * 256 // N_VOCAB for x in top}) >= 2
        cov["zero_max"] += bool(pen[t] == 0.0)
        with np.errstate(invalid="ignore"):
            cov["reversed"] += int(np.nanargmax(np.where(np.isnan(lo), -np.inf, lo))) != t
        cov["nan"] += bool(np.isnan(lo).any())
        cov["neg_inf"] += bool(np.isneginf(lo).any())
        if i + 1 == len(toks):  # the tail's in-place penalty: rp only (the frequency penalty is only compared)
            pen_rp = lo.copy()
            orc.choose(pen_rp, rp, window, 0.0, hist)
            assert same_bits(last, pen_rp), f"{label}: the read's last penalised logits differ"
        hist.append(int(t))
        counts[int(t)] = counts.get(int(t), 0) + 1
        if i + 1 < len(toks):
            lo = sb.step(int(t))
    for b in (lg_d, hist_d, tok_d, cnt_d, fpen_d):
        b.free()
    sb.free()
    print(f"\n[fused choice] {label}: {n_new} tokens bit-exact ({len(set(toks))} distinct), coverage {cov}",
          flush=True)
    return toks, cov


# ---- a random decoder with duplicated, dominant embedding rows ------------------------------------------------------

TIE_GROUPS = [(0, N_VOCAB - 1), (15, 16), (2047, 2048), (100, 101), (200, 204), (4000, 4001, 4002)]


@pytest.fixture(scope="module")
def tied_model(dev):
    cfg, te, on, layers = synth_text_model(n_layer=N_LAYER, n_vocab=N_VOCAB, seed=5150)
    rows = te.reshape(N_VOCAB, DIM // 32, 34).copy()
    big = f16_bytes(0.05)  # 25× the rows' typical scale: a group's shared logit is usually the maximum
    for gi, grp in enumerate(TIE_GROUPS):
        src = rows[1000 + gi].copy()
        src[:, 0], src[:, 1] = big
        for r in grp:
            rows[r] = src
    m = make_model(dev, cfg, rows.reshape(-1), on, layers)
    yield m
    m.free()


@pytest.mark.parametrize("rp,window,fp", [(1.1, 64, 0.0), (1.3, 16, 0.4), (0.7, 7, 0.37), (1.0, 64, 0.0)],
                         ids=["rp1.1_w64", "rp1.3_w16_fp0.4", "rp0.7_w7_fp0.37", "greedy"])
def test_fused_choice_exact_ties(dev, tied_model, rp, window, fp):
    """ties across workgroup shares, at both ends of the vocabulary, inside a wave and across waves; the prompt's
    window already holds one member of three groups (the first choices are reversals when those groups lead)"""
    from htr import synth

    prompt = synth.prompt_ids(808, 300, N_VOCAB)
    prompt[-6:] = [16, 101, 4001, 7, 2047, 9]
    toks, cov = read_and_check(dev, tied_model, prompt, rp, window, fp, 48, f"tied rows rp {rp} w {window} fp {fp}")
    if rp >= 1.0:  # rp < 1 raises a chosen member over its twin: the tie breaks once one of them is in the window
        assert cov["tied_max"] >= 4 and cov["ties_across_shares"] >= 1
    else:
        assert cov["tied_max"] >= 1
    if rp != 1.0:
        assert cov["reversed"] >= 1


# ---- a designed model: zero layers, sparse small-integer embedding rows ---------------------------------------------

R_NAN, R_NEG_INF = 3000, 3001


def designed_model(seed: int, nan_at_0: bool = False):
    """every layer weight zero (the residual reaching the LM head is the token's embedding, exactly); embedding rows
    with 1 or 2 quants in {−2, −1, 1, 2} at elements 0 … 7 and a scale of 1 or 2 (30 % all-zero rows: a logit of +0
    whatever the token); output_norm −1 on elements 4 … 7 (whose quants are positive only, so a token there makes every
    overlapping row negative: the maximum is +0), −1e34 on element 5 (row R_NEG_INF, 127 × 60000 there, overflows to
    −inf); row R_NAN: zero quants at an infinite scale (0·inf: NaN always); nan_at_0: row 0 so as well"""
    g = np.random.default_rng(seed)
    q = np.zeros((N_VOCAB, DIM), np.int8)
    d = np.ones(N_VOCAB, np.float32)
    for r in range(N_VOCAB):
        if g.random() < 0.3 and r != 0:
            continue
        nz = int(g.integers(1, 3))
        el = g.choice(8, nz, replace=False)
        q[r, el] = g.choice([-2, -1, 1, 2], nz)
        q[r, 4:8] = np.abs(q[r, 4:8])
        d[r] = g.choice([1.0, 2.0])
    q[R_NAN], d[R_NAN] = 0, np.inf
    q[R_NEG_INF] = 0
    q[R_NEG_INF, 5], d[R_NEG_INF] = 127, 60000.0
    if nan_at_0:
        q[0], d[0] = 0, np.inf
    on = np.ones(DIM, np.float32)
    on[4:8] = -1.0
    on[5] = -1e34
    zero = lambda rows, cols: np.zeros(rows * cols // 32 * 34, np.uint8)  # noqa: E731
    ones = lambda n: np.ones(n, np.float32)  # noqa: E731
    layers = [{"attn_norm": ones(DIM), "q": zero(2048, DIM), "k": zero(1024, DIM), "v": zero(1024, DIM),
               "o": zero(DIM, 2048), "q_norm": ones(128), "k_norm": ones(128), "ffn_norm": ones(DIM),
               "gate": zero(3072, DIM), "up": zero(3072, DIM), "down": zero(DIM, 3072)} for _ in range(N_LAYER)]
    cfg = dict(n_layer=N_LAYER, dim=DIM, n_head=16, n_kv=8, d_head=128, n_ff=3072, n_vocab=N_VOCAB,
               n_ctx_train=40960, eps=1e-6, rope_base=1e6)
    return cfg, blocks_of(q, d), on, layers


@pytest.mark.parametrize("seed,rp,window,fp", [(11, 1.1, 64, 0.0), (11, 1.3, 16, 0.4), (11, 0.7, 7, 0.37),
                                               (19, 1.1, 64, 0.0)],
                         ids=["rp1.1_w64", "rp1.3_w16_fp0.4", "rp0.7_w7_fp0.37", "zero_maxima"])
def test_fused_choice_designed_logits(dev, seed, rp, window, fp):
    cfg, te, on, layers = designed_model(seed)
    m = make_model(dev, cfg, te, on, layers)
    try:
        prompt = np.random.default_rng(seed + 100).integers(0, N_VOCAB, 20).astype(np.int32)
        toks, cov = read_and_check(dev, m, prompt, rp, window, fp, 48, f"designed seed {seed} rp {rp} fp {fp}")
    finally:
        m.free()
    assert cov["tied_max"] >= 4 and cov["zero_max"] >= 1 and cov["nan"] == 48
    if seed == 11:  # the read visits element 5 (−inf at R_NEG_INF); rp > 1 reverses tied leaders
        assert cov["neg_inf"] >= 1 and (rp < 1.0 or cov["reversed"] >= 1)
    else:  # a read whose every choice is among ties at +0
        assert cov["zero_max"] >= 40


def test_fused_choice_nan_at_index_0(dev):
    """logits[0] NaN (row 0: zero quants at an infinite scale): the reference's choose returns 0 (its first maximum
    starts at index 0 and nothing compares greater than NaN), and so does the one-launch step's tail; token 0's
    embedding is then NaN, every later logit NaN, every later token 0"""
    cfg, te, on, layers = designed_model(11, nan_at_0=True)
    m = make_model(dev, cfg, te, on, layers)
    try:
        prompt = np.random.default_rng(111).integers(1, N_VOCAB, 20).astype(np.int32)
        toks, _ = read_and_check(dev, m, prompt, 1.1, 64, 0.0, 20, "NaN at index 0")
    finally:
        m.free()
    assert toks == [0] * 20


# ---- the embedding gather (embed_q8_0.wgsl:19-38, text.rs:547), through a model whose layers add nothing ------------


def test_embedding_gather_reaches_the_lm_head_as_the_tokens_row(dev):
    """every layer weight zero, so the residual at the LM head is the gathered row itself: logits = E·(rmsnorm(E[t])
    ⊙ output_norm) with E the dequantised token_embd. The rows' 32 blocks carry scales of their own (a gather that
    dropped or misplaced a block's scale changes the normed direction; a whole-row scale would cancel in the norm), and
    the tokens sit at the workgroup-share edges (0, 15 / 16, 2047 / 2048, n_vocab − 1). Checked on the one-launch step,
    the per-kernel step (k_embed) and the prefill's last row, against fp64"""
    g = np.random.default_rng(4242)
    q = g.integers(-127, 128, (N_VOCAB, DIM)).astype(np.int8)
    d = (np.abs(g.normal(0.0, 1.0, (N_VOCAB, DIM // 32))) * 0.002 + 1e-4).astype(np.float16)
    blocks = np.zeros((N_VOCAB, DIM // 32, 34), np.uint8)
    blocks[:, :, :2] = d.reshape(N_VOCAB, DIM // 32, 1).view(np.uint8)
    blocks[:, :, 2:] = q.reshape(N_VOCAB, DIM // 32, 32).view(np.uint8)
    on = (1.0 + g.normal(0.0, 0.02, DIM)).astype(np.float32)
    zero = lambda rows, cols: np.zeros(rows * cols // 32 * 34, np.uint8)  # noqa: E731
    ones = lambda n: np.ones(n, np.float32)  # noqa: E731
    layers = [{"attn_norm": ones(DIM), "q": zero(2048, DIM), "k": zero(1024, DIM), "v": zero(1024, DIM),
               "o": zero(DIM, 2048), "q_norm": ones(128), "k_norm": ones(128), "ffn_norm": ones(DIM),
               "gate": zero(3072, DIM), "up": zero(3072, DIM), "down": zero(DIM, 3072)} for _ in range(N_LAYER)]
    cfg = dict(n_layer=N_LAYER, dim=DIM, n_head=16, n_kv=8, d_head=128, n_ff=3072, n_vocab=N_VOCAB,
               n_ctx_train=40960, eps=1e-6, rope_base=1e6)
    e64 = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32, axis=1)

    def want(t: int) -> np.ndarray:
        x = e64[t]
        return e64 @ (x / np.sqrt(np.mean(x * x) + 1e-6) * on.astype(np.float64))

    toks = [0, 15, 16, 2047, 2048, N_VOCAB - 1, 777, 3001]
    m = make_model(dev, cfg, blocks.reshape(-1), on, layers)
    try:
        worst = {}
        for fused in (True, False):
            s = m.session(CTX)
            s.fused_step = fused
            assert s.fused_step == fused
            s.prefill(np.array([5, 6], np.int32))
            for t in toks:
                got = s.step(t)
                if fused:
                    assert dev.last_kernel().startswith("k_decode_token<")
                err = rel_l2(got, want(t))
                worst[fused] = max(worst.get(fused, 0.0), err)
                assert err <= 1e-5, f"{'one-launch' if fused else 'per-kernel'} step, token {t}: rel-L2 {err:.2e}"
            s.free()
        s = m.session(CTX)
        for t in (0, N_VOCAB - 1, 2048):
            s.rewind(0)
            err = rel_l2(s.prefill(np.array([9, 10, t], np.int32)), want(t))
            worst["prefill"] = max(worst.get("prefill", 0.0), err)
            assert err <= 1e-3, f"prefill, last token {t}: rel-L2 {err:.2e}"
        s.free()
    finally:
        m.free()
    print(f"\n[embedding gather] rel-L2 vs fp64: one-launch {worst[True]:.1e}, per-kernel {worst[False]:.1e}, "
          f"prefill {worst['prefill']:.1e}", flush=True)
