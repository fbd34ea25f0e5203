"""The CPU choice (ocr-decode sampling.rs:23-89): the oracle's restatement pinned, and the library's htr_choose_host
against it, bit-exact. Host code only.

Pins of the oracle: the presets' seed rule (presets.rs:139-143, md5("abc") → 0x90015098); SplitMix64's published
outputs for state 0 (Steele, Lea, Flood; Vigna's splitmix64.c: 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4,
0x06c45d188009454f); the reference's own choose cases (sampling.rs:297-321); and for the sampled
branch what the mathematics fixes: a top_p below every probability keeps only the most likely token; the sampled
frequencies match the top-p kept set renormalised (T = 1: the softmax, T = 2: its square root renormalised), and
tokens outside the kept set never come."""
import numpy as np
import pytest

import htr
import oracle as orc

KAT = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_seed_rule_known_answer():
    # presets.rs:139-143: int(hashlib.md5(b"abc").hexdigest()[:8], 16) = 0x90015098
    assert htr.seed_for_stem("abc") == 0x90015098
    assert htr.seed_for_stem("") == 0xD41D8CD9  # md5("") = d41d8cd9 8f00b204 … (RFC 1321 A.5)


def test_rng_known_answers():
    r = orc.Rng(0)
    for z in KAT:
        assert r.next_f64() == (z >> 11) / 2.0 ** 53


def preset(t=0.0, top_p=1.0, rp=1.0, window=64, fp=0.0, max_new=10):
    return htr.Preset(repetition_penalty=rp, repetition_window=window, frequency_penalty=fp, max_new_tokens=max_new,
                      temperature=t, top_p=top_p)


def both(logits, p, hist, counts, seed):
    """(oracle token, library token, oracle logits after, library logits after, oracle state, library state)"""
    lo, ll = np.array(logits, np.float32), np.array(logits, np.float32)
    ro = orc.Rng(seed)
    to = orc.choose_sampled(lo, p.temperature, p.top_p, p.repetition_penalty, p.repetition_window,
                            p.frequency_penalty, hist, counts, ro)
    st = [seed]
    tl = htr.choose_host(ll, p, hist, counts, st)
    return to, tl, lo, ll, ro.state.value, st[0]


def test_reference_choose_cases():
    # sampling.rs:297-305: token 0 is outside the window of 2, token 1 twice inside counts once
    for f in (lambda l, p, h, c: orc.choose_sampled(l, p.temperature, p.top_p, p.repetition_penalty,
                                                     p.repetition_window, p.frequency_penalty, h, c, orc.Rng(1)),
              lambda l, p, h, c: htr.choose_host(l, p, h, c, [1])):
        l = np.array([2.0, 2.2, -1.0], np.float32)
        assert f(l, preset(rp=1.1, window=2), [0, 1, 1], {}) == 0
        assert abs(l[1] - 2.0) < 1e-6
        # sampling.rs:315-320
        l = np.array([1.0, 1.05], np.float32)
        assert f(l, preset(rp=1.0, fp=0.1, window=2), [], {1: 2}) == 0


def test_tiny_top_p_keeps_the_most_likely():
    rng = np.random.default_rng(3)
    for k in range(50):
        logits = rng.normal(0, 2, 500).astype(np.float32)
        hist = rng.integers(0, 500, 30)
        p = preset(t=0.8, top_p=1e-9, rp=1.3, window=16)
        want = np.array(logits)
        orc.choose(want, 1.3, 16, 0.0, hist)  # the greedy branch's penalties and argmax
        l = np.array(logits)
        got = orc.choose_sampled(l, 0.8, 1e-9, 1.3, 16, 0.0, hist, {}, orc.Rng(k))
        assert got == int(np.argmax(want))


@pytest.mark.parametrize("t,top_p", [(1.0, 0.8), (2.0, 0.8), (1.0, 1.0)])
def test_sampled_frequencies_follow_the_kept_distribution(t, top_p):
    p = np.array([0.4, 0.3, 0.15, 0.1, 0.05])
    logits = np.log(p).astype(np.float32)
    q = p ** (1 / t)
    q /= q.sum()
    order = np.argsort(-q, kind="stable")
    keep = np.searchsorted(np.cumsum(q[order]), top_p - 1e-12) + 1 if top_p < 1 else len(q)
    kept = order[:keep]
    want = np.zeros(5)
    want[kept] = q[kept] / q[kept].sum()
    n = 40_000
    r = orc.Rng(77)
    counts = np.zeros(5)
    for _ in range(n):
        counts[orc.choose_sampled(logits.copy(), t, top_p, 1.0, 1, 0.0, [], {}, r)] += 1
    freq = counts / n
    sigma = np.sqrt(want * (1 - want) / n)
    assert np.all(np.abs(freq - want) <= 5 * sigma + 1e-12), (freq, want)
    assert np.all(counts[want == 0] == 0)


def test_library_choose_matches_the_oracle_bit_for_bit():
    rng = np.random.default_rng(11)
    for k in range(300):
        nv = int(rng.integers(2, 3000))
        logits = (rng.normal(0, 3, nv)).astype(np.float32)
        if k % 7 == 0:  # exact ties: equal probabilities ordered by index
            logits[rng.integers(0, nv, nv // 2)] = logits[0]
        t = 0.0 if k % 5 == 0 else float(rng.uniform(0.05, 2.0))
        top_p = 1.0 if t == 0.0 or k % 3 == 0 else float(rng.uniform(0.05, 1.0))
        rp = float(rng.choice([1.0, 1.1, 1.35]))
        fp = float(rng.choice([0.0, 0.0, 0.2]))
        window = int(rng.integers(1, 80))
        hist = rng.integers(0, nv, int(rng.integers(0, 100)))
        ids = np.unique(rng.integers(0, nv, int(rng.integers(0, 20))))
        counts = {int(i): int(rng.integers(1, 5)) for i in ids}
        p = preset(t, top_p, rp, window, fp)
        seed = int(rng.integers(0, 2**63))
        to, tl, lo, ll, so, sl = both(logits, p, hist, counts, seed)
        assert to == tl, k
        assert np.array_equal(lo, ll), k
        assert so == sl, k


def test_library_choose_checks_its_preset():
    l = np.zeros(4, np.float32)
    for bad in (preset(t=-1.0), preset(t=0.0, top_p=0.5), preset(t=1.0, top_p=0.0), preset(rp=0.0),
                preset(window=0), preset(fp=-0.1), preset(max_new=0)):
        with pytest.raises(htr.HtrError, match="preset"):
            htr.choose_host(l, bad, [], {}, [0])
    with pytest.raises(htr.HtrError, match="outside the vocabulary"):
        htr.choose_host(l, preset(), [7], {}, [0])
