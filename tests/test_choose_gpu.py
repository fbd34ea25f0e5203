"""The GPU token choice (windowed repetition penalty + two-pass argmax) — bit-exact against the oracle's restatement
of ocr-decode's `choose` (sampling.rs:38-62)."""
import json
import os

import numpy as np
import pytest

import htr
import oracle as orc
from test_oracle import gpu_choice_matrix_inputs

pytestmark = pytest.mark.gpu
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))


def test_choice_matches_choose_on_reference_matrix(dev):
    """text.rs:1001-1054: the real and odd vocabularies; rp off / > 1 / < 1; windows 1 … 64; fp 0 and > 0; ties,
    ±0, −inf, all −inf; a dominant last token the penalties push down. The GPU keeps its own history and counts."""
    for case in GOLD["gpu_choice_matrix"]["cases"]:
        n_vocab, rp, window, fp, seed_hist = case
        steps = GOLD["gpu_choice_matrix"]["steps"]
        hist = dev.upload(np.array(list(seed_hist) + [0] * (steps + 1), np.uint32))
        counts = dev.alloc(n_vocab * 4) if fp > 0 else None
        fpen = dev.alloc(n_vocab * 4) if fp > 0 else None
        tok = dev.alloc(4)
        lb = dev.alloc(n_vocab * 4)
        chosen = []
        for i, (l, history, cnt, want) in enumerate(gpu_choice_matrix_inputs(case)):
            lb.upload(l)
            htr.choose(dev, lb, n_vocab, hist, len(seed_hist) + i, window, rp, tok, fp, counts, fpen)
            got = int(tok.download(np.uint32)[0])
            ref = l.copy()
            assert orc.choose(ref, rp, window, fp, history, cnt) == want
            assert got == want, f"vocab {n_vocab} rp {rp} window {window} fp {fp} step {i}"
            if fp == 0:  # the penalised logits, in place, bit for bit
                assert np.array_equal(lb.download(np.float32).view(np.uint32), ref.view(np.uint32)), i
            chosen.append(want)
        h = hist.download(np.uint32)
        assert h[len(seed_hist):len(seed_hist) + steps].tolist() == chosen


def test_choose_penalty_is_ieee_exact(dev):
    """text.rs:1061-1099, stricter: subnormal products compared too"""
    c = GOLD["choose_pen_exact"]
    n = c["n"]
    bits = orc.Lcg(c["seed"]).bits(n).astype(np.uint64)
    raw = np.where(np.arange(n) % 3 == 2, (0x0D800000 + bits % (0x7F000000 - 0x0D800000)) | 0x80000000,
                   bits % 0x7F800000).astype(np.uint32)
    raw[:6] = c["special_bits"]
    l0 = raw.view(np.float32)
    hist = dev.upload(np.arange(n + 1, dtype=np.uint32))
    tok = dev.alloc(4)
    for rp in c["rp"]:
        lb = dev.upload(l0)
        htr.choose(dev, lb, n, hist, n, n, rp, tok)
        r = np.float32(rp)
        with np.errstate(under="ignore", over="ignore"):
            want = np.where(l0 < 0, l0 * r, l0 / r)
        assert np.array_equal(lb.download(np.float32).view(np.uint32), want.view(np.uint32)), rp
        lb.free()


def config1_inputs(seed: int, rows: int, n_vocab: int = 151936, window: int = 64):
    """the choice workload's generator (htr.synth.choice_inputs): N(0, 3) logits with 8 planted equal maxima, 3 of
    them on window ids; 64 uniform history ids with 25 % repeats"""
    from htr import synth

    return synth.choice_inputs(seed, rows, n_vocab, window)


def test_config1_choice_bit_exact(dev):
    """the 151936-logit vocabulary: 64 independent rows in one launch and 16 single launches, each against the oracle"""
    rows, n_vocab, window, rp = 64, 151936, 64, 1.1
    logits, hist = config1_inputs(1, rows)
    hb = dev.upload(np.concatenate([hist, np.zeros((rows, 1), np.int32)], axis=1).astype(np.uint32))
    lb = dev.upload(logits)
    tok = dev.alloc(rows * 4)
    htr.choose_many(dev, lb, n_vocab, rows, hb, window + 1, window, window, rp, tok)
    got = tok.download(np.uint32)
    pen = lb.download(np.float32).reshape(rows, n_vocab)
    for r in range(rows):
        ref = logits[r].copy()
        want = orc.choose(ref, rp, window, 0.0, hist[r])
        assert int(got[r]) == want, r
        assert np.array_equal(pen[r].view(np.uint32), ref.view(np.uint32)), r
    h = hb.download(np.uint32).reshape(rows, window + 1)
    assert np.array_equal(h[:, window], got)
    # single launches
    one = dev.alloc(n_vocab * 4)
    h1 = dev.alloc((window + 1) * 4)
    for r in range(16):
        one.upload(logits[r])
        h1.upload(hist[r].astype(np.uint32))
        htr.choose(dev, one, n_vocab, h1, window, window, rp, tok)
        assert int(tok.download(np.uint32)[0]) == int(got[r])


def test_choose_nan_rules(dev):
    tok = dev.alloc(4)
    hist = dev.upload(np.zeros(4, np.uint32))
    for l, want in (([np.nan, 3.0, 5.0], 0), ([1.0, np.nan, 5.0], 2), ([-np.inf] * 5, 0), ([np.nan] * 3, 0)):
        a = np.array(l, np.float32)
        assert orc.choose(a.copy(), 1.0, 1, 0.0, []) == want
        htr.choose(dev, dev.upload(a), a.size, hist, 0, 1, 1.0, tok)
        assert int(tok.download(np.uint32)[0]) == want, l


def test_choose_rejects_bad_penalty(dev):
    tok = dev.alloc(4)
    with pytest.raises(htr.HtrError, match="repetition penalty"):
        htr.choose(dev, dev.alloc(16), 4, dev.alloc(16), 1, 1, 0.0, tok)
    with pytest.raises(htr.HtrError, match="repetition penalty"):
        htr.choose(dev, dev.alloc(16), 4, dev.alloc(16), 1, 1, 1e-40, tok)


@pytest.mark.parametrize("window,n_hist", [(600, 700), (300, 250), (257, 1000)])
def test_long_windows_penalise_each_distinct_id_once(dev, window, n_hist):
    """windows longer than a workgroup (256 threads: the ids past the first 256 are marked in a second pass), with
    ids repeated up to 5 times and some landing on the planted maxima, 151936 logits, rp 1.1 and 0.8: the token and
    the penalised logits (written back in place) equal the oracle's choose bit for bit"""
    n_vocab = 151936
    g = np.random.default_rng(window + n_hist)
    base, _ = synth_choice(window + 7, 1, n_vocab, 64)
    hist = g.integers(0, n_vocab, n_hist).astype(np.int32)
    rep = g.integers(0, n_hist, n_hist // 3)
    hist[rep] = hist[g.integers(0, n_hist, rep.size)]
    top = np.flatnonzero(base[0] == base[0].max())
    hist[-3:] = top[:3]  # the planted maxima inside the window
    hb = dev.upload(np.concatenate([hist, np.zeros(1, np.int32)]).astype(np.uint32))
    tok = dev.alloc(4)
    for rp in (1.1, 0.8):
        lb = dev.upload(base[0])
        htr.choose(dev, lb, n_vocab, hb, n_hist, window, rp, tok)
        ref = base[0].copy()
        want = orc.choose(ref, rp, window, 0.0, list(hist))
        assert int(tok.download(np.uint32)[0]) == want, rp
        assert np.array_equal(lb.download(np.float32).view(np.uint32), ref.view(np.uint32)), rp
        lb.free()


def synth_choice(seed, rows, n_vocab, window):
    from htr import synth

    return synth.choice_inputs(seed, rows, n_vocab, window)


def test_config1_bench_rows_bit_exact(dev):
    """the bench's own choice workload: its 512 rows (htr.synth.choice_inputs, seeds 7000 + 32·b), every row as a
    single launch (k_choose on one row, as the bench's 10k steps run it) and all 512 in one launch — every token and
    every penalised row the oracle's bit for bit; a second pass on rows restored from the pristine copy gives the same
    tokens (the bench restores its rows between passes so each step sees its seeded logits)"""
    from htr import synth

    n_buf, n_vocab, window, rp = 512, 151936, 64, 1.1
    logits = np.empty((n_buf, n_vocab), np.float32)
    hist = np.zeros((n_buf, window + 1), np.uint32)
    for i in range(0, n_buf, 32):
        lg, h = synth.choice_inputs(7000 + i, 32, n_vocab, window)
        logits[i:i + 32] = lg
        hist[i:i + 32, :window] = h
    want, pens = [], []
    for r in range(n_buf):
        ref = logits[r].copy()
        want.append(orc.choose(ref, rp, window, 0.0, [int(t) for t in hist[r, :window]]))
        pens.append(ref)
    lb, hb, tok = dev.upload(logits), dev.upload(hist), dev.alloc(n_buf * 4)
    L = htr.lib()
    for p in range(2):
        lb.upload(logits)
        for r in range(n_buf):
            rc = L.htr_choose(dev.h, lb.ptr + r * n_vocab * 4, n_vocab, hb.ptr + r * (window + 1) * 4, window, window,
                              rp, 0.0, None, None, tok.ptr + 4 * r)
            assert rc == 0, htr.last_error()
        got = tok.download(np.uint32, n_buf)
        assert [int(t) for t in got] == want, p
    pen = lb.download(np.float32).reshape(n_buf, n_vocab)
    for r in range(0, n_buf, 37):
        assert np.array_equal(pen[r].view(np.uint32), pens[r].view(np.uint32)), r
    lb.upload(logits)
    htr.choose_many(dev, lb, n_vocab, n_buf, hb, window + 1, window, window, rp, tok)
    assert [int(t) for t in tok.download(np.uint32, n_buf)] == want
    print(f"\n[config 1] the bench's 512 rows: single launches (twice) and one batched launch equal the oracle's "
          f"choice; {len(set(want))} distinct tokens", flush=True)
    for b in (lb, hb, tok):
        b.free()


def many(dev, rows, rp, window, hists, n_vocab):
    """choose_many over rows [n][n_vocab] with per-row windows (hists [n][window], left-padded with n_vocab, an id
    outside the vocabulary that neither kernel penalises) at len = window → tokens, penalised rows"""
    n = len(rows)
    hb = dev.upload(np.concatenate([np.asarray(hists, np.uint32), np.zeros((n, 1), np.uint32)], axis=1))
    lb = dev.upload(np.ascontiguousarray(rows, np.float32))
    tok = dev.alloc(n * 4)
    htr.choose_many(dev, lb, n_vocab, n, hb, window + 1, window, window, rp, tok)
    assert dev.last_kernel() == "k_choose_rows"
    got = [int(t) for t in tok.download(np.uint32, n)]
    pen = lb.download(np.float32).reshape(n, n_vocab)
    h = hb.download(np.uint32).reshape(n, window + 1)
    assert h[:, window].tolist() == got  # the token appended to each row's history
    for b in (hb, lb, tok):
        b.free()
    return got, pen


def padded(history, window, n_vocab):
    w = list(history[-window:]) if history else []
    return [n_vocab] * (window - len(w)) + w


def test_many_rows_on_the_reference_matrix(dev):
    """text.rs:1001-1054's cases without the frequency penalty (which the batched form does not take), every step of
    a case a row of one launch (a workgroup a row, k_choose_rows): the tokens and the penalised rows bit for bit"""
    for case in GOLD["gpu_choice_matrix"]["cases"]:
        n_vocab, rp, window, fp, _ = case
        if fp != 0:
            continue
        steps = list(gpu_choice_matrix_inputs(case))
        got, pen = many(dev, [l for l, _, _, _ in steps], rp, window,
                        [padded(h, window, n_vocab) for _, h, _, _ in steps], n_vocab)
        for i, (l, history, _, want) in enumerate(steps):
            ref = l.copy()
            assert orc.choose(ref, rp, window, 0.0, history) == want
            assert got[i] == want, f"vocab {n_vocab} rp {rp} window {window} step {i}"
            assert np.array_equal(pen[i].view(np.uint32), ref.view(np.uint32)), (n_vocab, rp, window, i)


@pytest.mark.parametrize("n_vocab", [1000, 1001])
def test_many_rows_edge_rules(dev, n_vocab):
    """the batched form's 16-byte path (1000 logits a row) and its logit-a-step path (1001): NaN at index 0 → 0, NaN
    elsewhere never wins, every logit −inf → 0, every logit NaN → 0, exact ties and ±0 maxima → the lowest index, a
    window id on the maximum (rp 1.3: the penalty reverses the choice, and rp 0.7 raises a negative one), a window
    repeating one id (penalised once) — each row against the oracle's choose, penalised rows bit for bit"""
    g = np.random.default_rng(n_vocab)
    rows, hists = [], []
    window = 5
    base = lambda: g.normal(0, 3, n_vocab).astype(np.float32)  # noqa: E731
    r = base(); r[0] = np.nan; rows.append(r)
    r = base(); r[7] = np.nan; r[9] = 40.0; rows.append(r)
    rows.append(np.full(n_vocab, -np.inf, np.float32))
    rows.append(np.full(n_vocab, np.nan, np.float32))
    r = base(); r[[3, 600, n_vocab - 1]] = 50.0; rows.append(r)
    r = -np.abs(base()) - 1.0; r[5] = -0.0; r[900] = 0.0; rows.append(r)
    r = base(); r[11] = 30.0; r[12] = 29.0; rows.append(r)
    r = -np.abs(base()) - 10.0; r[13] = -2.0; r[14] = -1.9; rows.append(r)
    wins = [[1, 2, 3, 4, 5], [7, 7, 7, 7, 7], [0, 1, 2, 3, 4], [0, 0, 1, 1, 2], [600, 600, 2, 2, 3],
            [5, 900, 900, 5, 8], [11, 11, 11, 11, 11], [13, 13, 13, 13, 13]]
    for rp in (1.3, 0.7):
        got, pen = many(dev, rows, rp, window, wins, n_vocab)
        for i, (row, w) in enumerate(zip(rows, wins)):
            ref = row.copy()
            want = orc.choose(ref, rp, window, 0.0, w)
            assert got[i] == want, f"rp {rp} row {i}: {got[i]} against {want}"
            a, b = pen[i], ref
            assert np.array_equal(np.isnan(a), np.isnan(b))
            assert np.array_equal(a[~np.isnan(a)].view(np.uint32), b[~np.isnan(b)].view(np.uint32)), (rp, i)


def test_many_rows_past_the_bitmap_take_the_per_span_kernel(dev):
    """a vocabulary whose window bitmap would pass 64 KB of LDS (600,000 ids): the batched form keeps the per-span
    kernel (k_choose<4096>, atomics per row) — tokens and penalised rows against the oracle"""
    n_vocab, n, window, rp = 600000, 3, 16, 1.2
    g = np.random.default_rng(600)
    rows = g.normal(0, 3, (n, n_vocab)).astype(np.float32)
    rows[0, [5, 599999]] = 40.0          # a tie across the row's ends: the lower id
    rows[1, 123456] = 50.0               # a window id on the maximum: reversed by the penalty
    rows[2, :] = -np.inf
    hists = [list(g.integers(0, n_vocab, window)), [123456] * window, list(g.integers(0, n_vocab, window))]
    hb = dev.upload(np.concatenate([np.asarray(hists, np.uint32), np.zeros((n, 1), np.uint32)], axis=1))
    lb = dev.upload(rows)
    tok = dev.alloc(n * 4)
    htr.choose_many(dev, lb, n_vocab, n, hb, window + 1, window, window, rp, tok)
    assert dev.last_kernel() == "k_choose"
    got = [int(t) for t in tok.download(np.uint32, n)]
    pen = lb.download(np.float32).reshape(n, n_vocab)
    for i in range(n):
        ref = rows[i].copy()
        want = orc.choose(ref, rp, window, 0.0, [int(t) for t in hists[i]])
        assert got[i] == want, i
        assert np.array_equal(pen[i].view(np.uint32), ref.view(np.uint32)), i
    assert got[2] == 0
    for b in (hb, lb, tok):
        b.free()
