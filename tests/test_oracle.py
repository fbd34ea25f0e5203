"""Pins the oracle (oracle/htr_oracle.c) before any GPU result is compared with it.

Each oracle function is checked against something that does not share its code: the reference tests' golden values
(tests/golden/reference_cases.json), numpy's IEEE float32 / float16 arithmetic, and fp64 closed forms written here
independently. A plausible slip in the restatement (a dropped norm, a wrong scale index, a swapped RoPE sign, a
penalty on repeats) fails one of these.
"""
import json
import os

import numpy as np
import pytest

import oracle as orc
from helpers import kv_head_major, norm_vec, rel_l2, tiny_prompt, tiny_text_model

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))


# ---- independent numpy restatements (fp64) --------------------------------------------------------------------------

def np_dequant(blocks: np.ndarray, rows: int, cols: int) -> np.ndarray:
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float64)
    q = b[:, 2:].view(np.int8).astype(np.float64)
    return (q * d).reshape(rows, cols)


def np_rms(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def np_rope(x, pos, base=1e6):
    """x [..., 128] at position pos, NEOX pairs (i, i+64), θ = pos·base^(−2i/128) in f64"""
    i = np.arange(64)
    th = pos * base ** (-(2.0 * i) / 128.0)
    c, s = np.cos(th), np.sin(th)
    a, b = x[..., :64], x[..., 64:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


def np_attention(q, k, v, scale):
    """q [n_head][128] f64, k / v [n_keys][n_kv][128] f64 → [n_head][128]"""
    n_head, n_kv = q.shape[0], k.shape[1]
    out = np.zeros_like(q)
    for h in range(n_head):
        kh = h // (n_head // n_kv)
        s = k[:, kh, :] @ q[h] * scale
        e = np.exp(s - s.max())
        out[h] = (e / e.sum()) @ v[:, kh, :]
    return out


def np_choose(logits, rp, window, fp, history, counts):
    """sampling.rs:38-62 with numpy float32 scalar arithmetic (IEEE)"""
    l = np.array(logits, dtype=np.float32)
    if rp != 1.0:
        r = np.float32(rp)
        seen = set()
        for t in history[len(history) - min(window, len(history)):]:
            if t not in seen:
                seen.add(t)
                l[t] = l[t] * r if l[t] < 0 else l[t] / r
    if fp > 0:
        for t, c in counts.items():
            l[t] = l[t] - np.float32(fp) * np.float32(c)
    best = 0
    for i in range(l.size):
        if l[i] > l[best]:
            best = i
    return best, l


# ---- seeded inputs, f16, q8_0 ---------------------------------------------------------------------------------------

def test_lcg_matches_reference_generator():
    g = GOLD["lcg_seed11"]
    assert orc.Lcg(g["seed"]).f32(len(g["values"])).tolist() == g["values"]


def test_f16_round_to_nearest_even_matches_numpy():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6e-8, 2.98e-8, 2.9802322e-08, 5.9604645e-08,
                     6.1035156e-05, 6.1e-05, 1.0009765625, 1.00048828125, 1.00146484375, 1e-40], dtype=np.float32)
    for v in (x, edge, (rng.standard_normal(100000) * 3).astype(np.float32)):
        with np.errstate(over="ignore"):
            want = v.astype(np.float16).view(np.uint16)
        assert np.array_equal(orc.f16_bits(v), want)


def test_f16_to_f32_all_codes():
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = orc.f16_to_f32(codes)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_q8_0_golden_block():
    g = GOLD["gguf_q8_0_block"]
    out = orc.q8_0_dequant(np.array(g["bytes"], np.uint8), 32)
    assert (out[0], out[31]) == (g["first"], g["last"])
    assert np.array_equal(out, np.arange(-16, 16, dtype=np.float32) * 0.5)


def test_q8_0_quantizer_properties():
    x = orc.Lcg(11).f32(37 * 96, 0.3)
    blocks, deq = orc.q8_0_quantize(x)
    assert blocks.size == 37 * 96 // 32 * 34
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    q = b[:, 2:].view(np.int8).astype(np.int32)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.all(np.abs(q).max(axis=1) == 127)
    assert np.array_equal(deq, (q * d[:, None]).astype(np.float32).ravel())
    # round-to-nearest of x / d (with the exact id = 1/d of the unrounded d): error ≤ half a step (+ d's f16 rounding)
    assert np.all(np.abs(deq.reshape(-1, 32) - xb) <= 0.5 * d[:, None] + np.abs(q) * np.abs(d - amax / 127)[:, None] + 1e-7)


# ---- matvec family --------------------------------------------------------------------------------------------------

def test_matvec_and_dmv_match_fp64():
    """text.rs:707-741 shape (37 rows × 3 blocks: odd rows start on half words in the GGUF bytes), 1e-4 abs"""
    n, k = 37, 96
    g = orc.Lcg(11)
    blocks, _ = orc.q8_0_quantize(g.f32(n * k, 0.3))
    x = g.f32(k)
    base = g.f32(n)
    w = np_dequant(blocks, n, k)
    want = w @ x.astype(np.float64)
    for acc in (False, True):
        e = want + (base if acc else 0)
        assert np.abs(orc.matvec_q8_0(blocks, n, k, x, base, acc) - e).max() < 1e-4
        assert np.abs(orc.dmv(blocks, n, k, x, None, 0.0, base, acc) - e).max() < 1e-4
    assert np.abs(orc.matvec_f64(blocks, n, k, x) - want).max() < 1e-12


def test_fused_dmv_variants_match_fp64():
    """text.rs:864-925 (dmv_norm, dmv_qkv, dmv_ffn), rel 1e-3 as the reference"""
    k, eps = 96, 1e-6
    g = orc.Lcg(41)
    x = g.f32(k, 2.0)
    nw = g.f32(k)
    xn = np_rms(x, nw, eps)

    def mat(rows):
        b, _ = orc.q8_0_quantize(g.f32(rows * k, 0.3))
        return b, np_dequant(b, rows, k)

    close = lambda got, want: np.all(np.abs(got - want) < 1e-3 * (1 + np.abs(want)))
    b, w = mat(37)
    assert close(orc.dmv(b, 37, k, x, nw, eps), w @ xn)
    (bq, wq), (bk, wk), (bv, wv) = mat(32), mat(16), mat(16)
    got = orc.dmv_qkv(bq, bk, bv, 32, 16, k, x, nw, eps)
    assert close(got, np.concatenate([wq @ xn, wk @ xn, wv @ xn]))
    (bg, wg), (bu, wu) = mat(37), mat(37)
    gg, uu = wg @ xn, wu @ xn
    assert close(orc.dmv_ffn(bg, bu, 37, k, x, nw, eps), gg / (1 + np.exp(-gg)) * uu)


def test_rms_norm_matches_fp64():
    x = orc.Lcg(2).f32(3 * 1024, 4.0)
    w = norm_vec(1024, 3)
    got = orc.rms_norm(x, w, 3, 1024, 1e-6)
    assert rel_l2(got, np_rms(x.reshape(3, 1024), w, 1e-6).ravel()) < 1e-6


def test_rope_table_matches_fp64():
    """text.rs:768-792: f32 θ at positions ~1000 is good to ~1e-4 rad"""
    t = orc.rope_table(1e6, 128, 1100).reshape(1100, 64, 2)
    pos = np.arange(1100)[:, None]
    th = pos * 1e6 ** (-(2.0 * np.arange(64)) / 128.0)
    assert np.abs(t[..., 0] - np.cos(th)).max() < 5e-4 and np.abs(t[..., 1] - np.sin(th)).max() < 5e-4
    assert t[0, :, 0].tolist() == [1.0] * 64 and t[0, :, 1].tolist() == [0.0] * 64


def test_qkv_post_matches_fp64():
    """text.rs:926-972: q normed + roped in place, k within f16 rounding, v bit-equal to RNE f16"""
    n_head, n_kv, pos, eps = 4, 2, 5, 1e-6
    g = orc.Lcg(43)
    raw = g.f32((n_head + 2 * n_kv) * 128, 3.0)
    qn, kn = g.f32(128), g.f32(128)
    cs = orc.rope_table(1e6, 128, 7)
    q, kr, vr = orc.qkv_post(raw, qn, kn, cs, n_head, n_kv, pos, eps)
    heads = raw.reshape(-1, 128).astype(np.float64)
    wq = np_rope(np_rms(heads[:n_head], qn, eps), pos)
    assert np.abs(q[: n_head * 128] - wq.ravel()).max() < 1e-3 * (1 + np.abs(wq).max())
    wk = np_rope(np_rms(heads[n_head:n_head + n_kv], kn, eps), pos).ravel()
    kf = kr.view(np.float16).astype(np.float64)
    assert np.all(np.abs(kf - wk) <= 1e-3 * (1 + np.abs(wk)))
    assert np.array_equal(vr, raw[(n_head + n_kv) * 128:].astype(np.float16).view(np.uint16))


# ---- attention ------------------------------------------------------------------------------------------------------

def _kv(g, n, n_kv, ks=2.0):
    kf = g.f32(n * n_kv * 128, ks)
    vf = g.f32(n * n_kv * 128)
    return orc.f16_bits(kf), orc.f16_bits(vf)


def test_decode_attention_matches_fp64():
    """text.rs:1264-1292: 300 keys (3 chunks), 4 q heads on 2 kv heads; the reference's bar is rel-L2 < 1e-5"""
    n_head, n_kv, n = 4, 2, 300
    g = orc.Lcg(31)
    k, v = _kv(g, n, n_kv)
    q = g.f32(n_head * 128, 2.0)
    sc = 1 / np.sqrt(128)
    want = np_attention(q.reshape(n_head, 128).astype(np.float64),
                        k.view(np.float16).astype(np.float64).reshape(n, n_kv, 128),
                        v.view(np.float16).astype(np.float64).reshape(n, n_kv, 128), sc)
    assert rel_l2(orc.attn_decode(q, k, v, n_kv * 128, n, n_head, n_kv, np.float32(sc)), want.ravel()) < 1e-5
    assert rel_l2(orc.attn_f64(q, k, v, n_kv * 128, n, n_head, n_kv, sc), want.ravel()) < 1e-12


@pytest.mark.parametrize("n_head,n_kv,n", [(4, 2, 300), (16, 8, 600), (2, 1, 1)])
def test_decode_attention_f32_path_matches_fp64(n_head, n_kv, n):
    """the F32 path's three-kernel decode attention (attn_scores / attn_softmax / attn_values, text.rs:567-569) at the
    reference's bar (rel-L2 < 1e-5, text.rs:1290-1291): key counts over one and several of attn_softmax's 256-lane
    strides and attn_values' 8-lane strides, GQA groups of 2; and within f32 rounding of the split-K form"""
    g = orc.Lcg(41 + n)
    k, v = _kv(g, n, n_kv)
    q = g.f32(n_head * 128, 2.0)
    sc = np.float32(1 / np.sqrt(128))
    want = np_attention(q.reshape(n_head, 128).astype(np.float64),
                        k.view(np.float16).astype(np.float64).reshape(n, n_kv, 128),
                        v.view(np.float16).astype(np.float64).reshape(n, n_kv, 128), float(sc))
    got = orc.attn_decode_f32(q, k, v, n_kv * 128, n, n_head, n_kv, sc)
    assert rel_l2(got, want.ravel()) < 1e-5
    assert rel_l2(got, orc.attn_decode(q, k, v, n_kv * 128, n, n_head, n_kv, sc)) < 1e-6


def test_causal_attention_matches_fp64():
    """text.rs:797-830: a batch of 70 queries at pos0 = 9 over the f16 cache, 1e-4 abs"""
    n_head, n_kv, pos0, n_q = 4, 2, 9, 70
    n = pos0 + n_q
    g = orc.Lcg(21)
    k, v = _kv(g, n, n_kv)
    q = g.f32(n_q * n_head * 128, 2.0)
    sc = 1 / np.sqrt(128)
    out = orc.attn_causal(q, k, v, n_kv * 128, n_q, pos0, n_head, n_kv, np.float32(sc)).reshape(n_q, n_head, 128)
    kf = k.view(np.float16).astype(np.float64).reshape(n, n_kv, 128)
    vf = v.view(np.float16).astype(np.float64).reshape(n, n_kv, 128)
    for t in (0, 1, 37, 63, 64, n_q - 1):
        want = np_attention(q.reshape(n_q, n_head, 128)[t].astype(np.float64), kf[: pos0 + t + 1], vf[: pos0 + t + 1], sc)
        assert np.abs(out[t] - want).max() < 1e-4, t
    # the head-major layout helper round-trips
    assert np.array_equal(kv_head_major(k.reshape(n, n_kv * 128), n_kv)[1, 5], k.reshape(n, n_kv, 128)[5, 1])


# ---- token choice ---------------------------------------------------------------------------------------------------

def test_choose_reference_unit_cases():
    for c in GOLD["sampling"]:
        l = np.array(c["logits"], np.float32)
        counts = {int(t): n for t, n in c["counts"].items()}
        assert orc.choose(l, c["rp"], c["window"], c["fp"], c["history"], counts) == c["token"], c["source"]
        if "logit1_after" in c:
            assert abs(l[1] - c["logit1_after"]) < c["tol"]


def test_choose_penalty_is_ieee_exact():
    """text.rs:1061-1099: 8192 distinct window tokens over logits of every magnitude, bit for bit against IEEE
    float32 multiply / divide (numpy), subnormal products included"""
    c = GOLD["choose_pen_exact"]
    n = c["n"]
    bits = orc.Lcg(c["seed"]).bits(n).astype(np.uint64)
    raw = np.where(np.arange(n) % 3 == 2, (0x0D800000 + bits % (0x7F000000 - 0x0D800000)) | 0x80000000,
                   bits % 0x7F800000).astype(np.uint32)
    raw[:6] = c["special_bits"]
    l0 = raw.view(np.float32)
    hist = np.arange(n, dtype=np.int32)
    for rp in c["rp"]:
        l = l0.copy()
        orc.choose(l, rp, n, 0.0, hist)
        r = np.float32(rp)
        with np.errstate(under="ignore", over="ignore"):
            want = np.where(l0 < 0, l0 * r, l0 / r)
        assert np.array_equal(l.view(np.uint32), want.view(np.uint32)), rp


def _matrix_logits(g, n_vocab, mode, i, last):
    """text.rs:1021-1035: the mode's values in the reference's draw order (the oracle's restatement, pinned below
    against a Python loop of the same draws), all −inf at step 7, the last chosen token made the maximum + 0.05"""
    l = g.choice_matrix(mode, n_vocab)
    if i == 7:
        l[:] = -np.inf
    if last is not None:
        l[last] = l.max() + np.float32(0.05)
    return l


def gpu_choice_matrix_inputs(case, steps=None):
    """The inputs of gpu_choice_matches_choose (text.rs:1001-1054) for one case, with the reference's own sequence of
    choices computed by the numpy restatement: yields (logits, history, counts, want) per step"""
    n_vocab, rp, window, fp, seed_hist = case
    g = orc.Lcg(GOLD["gpu_choice_matrix"]["seed"])
    history = list(seed_hist)
    counts: dict = {}
    for i in range(steps or GOLD["gpu_choice_matrix"]["steps"]):
        l = _matrix_logits(g, n_vocab, i % 4, i, history[-1] if history else None)
        want, _ = np_choose(l, rp, window, fp, history, counts)
        yield l, list(history), dict(counts), want
        history.append(want)
        counts[want] = counts.get(want, 0) + 1


def test_choice_matrix_logits_follow_the_reference_draws():
    """text.rs:1021-1027 restated in Python from the reference LCG (text.rs:670-673) one draw at a time: mode 0 rounds
    half away from zero (2.5 → 3, −2.5 → −3, as Rust's f32::round), mode 2 draws its second value only when the first
    is ≤ 0.9; the oracle's generator gives the same f32 values and leaves the LCG in the same state"""
    def lcg(s):
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        return s, np.float32(np.float32(s >> 40) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0)

    def rnd(x):  # half away from zero, in f64 on the f32 value
        x = float(x)
        return np.float32(np.copysign(np.floor(abs(x) + 0.5), x))

    for mode in range(4):
        s = 12345 + mode
        want = []
        for _ in range(3000):
            s, u = lcg(s)
            if mode == 0:
                want.append(rnd(u * np.float32(3.0)))
            elif mode == 1:
                want.append(u * np.float32(20.0))
            elif mode == 2:
                if u > np.float32(0.9):
                    want.append(np.float32(-np.inf))
                else:
                    s, v = lcg(s)
                    want.append(rnd(v * np.float32(2.0)) - np.float32(1.0))
            else:
                want.append(u * np.float32(1e-3))
        g = orc.Lcg(12345 + mode)
        got = g.choice_matrix(mode, 3000)
        assert np.array_equal(got.view(np.uint32), np.array(want, np.float32).view(np.uint32)), mode
        assert g.s.value == s, mode
    assert rnd(np.float32(2.5)) == 3.0 and rnd(np.float32(-2.5)) == -3.0 and np.round(2.5) == 2.0


def test_choose_matches_numpy_restatement_on_reference_matrix():
    for case in GOLD["gpu_choice_matrix"]["cases"][2:]:  # the small vocabularies (the 151936 ones run on the GPU)
        n_vocab, rp, window, fp, _ = case
        for l, hist, counts, want in gpu_choice_matrix_inputs(case, steps=12):
            assert orc.choose(l.copy(), rp, window, fp, hist, counts) == want, case


def test_choose_nan_and_all_neg_inf():
    l = np.array([np.nan, 3.0, 5.0], np.float32)
    assert orc.choose(l, 1.0, 1, 0.0, []) == 0  # NaN at 0: the CPU loop never moves
    l = np.array([1.0, np.nan, 5.0], np.float32)
    assert orc.choose(l, 1.0, 1, 0.0, []) == 2
    assert orc.choose(np.full(5, -np.inf, np.float32), 1.0, 1, 0.0, []) == 0


# ---- the decoder ----------------------------------------------------------------------------------------------------

def np_forward(cfg, tok_embd, output_norm, layers, ids, r16=False):
    """An fp64 forward of the Qwen3 graph (text.rs:1-19) over `ids`, K / V rounded to f16 like the cache:
    → logits of every position. r16: every layer GEMM's operands (X and the dequantised W) rounded to f16 first, the
    f16 compute paths' prefill (matmul_coop_q8_0); the LM head stays exact (a matvec on every path)"""
    d, nh, nkv, f, V, eps = cfg["dim"], cfg["n_head"], cfg["n_kv"], cfg["n_ff"], cfg["n_vocab"], cfg["eps"]
    E = np_dequant(tok_embd, V, d)
    x = E[np.asarray(ids)]
    n = x.shape[0]

    def mm(a, w, rows, cols):
        W = np_dequant(w, rows, cols)
        if r16:
            a, W = a.astype(np.float16).astype(np.float64), W.astype(np.float16).astype(np.float64)
        return a @ W.T

    for ly in layers:
        h = np_rms(x, ly["attn_norm"], eps)
        q = mm(h, ly["q"], nh * 128, d)
        k = mm(h, ly["k"], nkv * 128, d)
        v = mm(h, ly["v"], nkv * 128, d)
        q = np_rms(q.reshape(n, nh, 128), ly["q_norm"], eps)
        k = np_rms(k.reshape(n, nkv, 128), ly["k_norm"], eps)
        pos = np.arange(n)[:, None, None]
        i = np.arange(64)
        th = pos * 1e6 ** (-(2.0 * i) / 128.0)
        rot = lambda z: np.concatenate([z[..., :64] * np.cos(th) - z[..., 64:] * np.sin(th),
                                        z[..., :64] * np.sin(th) + z[..., 64:] * np.cos(th)], axis=-1)
        q, k = rot(q), rot(k)
        k = k.astype(np.float16).astype(np.float64)
        v = v.reshape(n, nkv, 128).astype(np.float16).astype(np.float64)
        a = np.zeros((n, nh, 128))
        for t in range(n):
            a[t] = np_attention(q[t], k[: t + 1], v[: t + 1], 1 / np.sqrt(128))
        x = x + mm(a.reshape(n, -1), ly["o"], d, nh * 128)
        h = np_rms(x, ly["ffn_norm"], eps)
        g = mm(h, ly["gate"], f, d)
        u = mm(h, ly["up"], f, d)
        x = x + mm(g / (1 + np.exp(-g)) * u, ly["down"], d, f)
    return np_rms(x, output_norm, eps) @ E.T


@pytest.mark.parametrize("step_f32", [True, False])
def test_oracle_decoder_matches_fp64_forward(step_f32):
    """the oracle's prefill (F32-path kernels) and steps — the F32 path's step (text.rs:555-576) and the fused step of
    the f16 paths (layers_fused, text.rs:630-647) — against the independent fp64 forward on the reference's tiny model
    (text.rs:1297-1323) and its 20-token prompt"""
    cfg, te, on, layers = tiny_text_model()
    prompt = tiny_prompt()
    extra = [int(t) for t in orc.Lcg(9).bits(6) % cfg["n_vocab"]]
    want = np_forward(cfg, te, on, layers, list(prompt) + extra)
    s = orc.Session(cfg, te, on, layers, 64, step_f32=step_f32)
    got = [s.prefill(prompt)]
    for t in extra:
        got.append(s.step(t))
    assert s.n_past == len(prompt) + len(extra)
    for i, lg in enumerate(got):
        w = want[len(prompt) - 1 + i]
        assert rel_l2(lg, w) < 1e-3, i
        assert int(np.argmax(lg)) == int(np.argmax(w)), i


@pytest.mark.parametrize("m,n,k", [(7, 96, 256), (33, 64, 1024)])
def test_oracle_matmul_q8_0_both_paths_match_numpy(m, n, k):
    """Batch::matmul with a q8_0 weight (gpu.rs:1963-2014): the F32 path against the fp64 product of the exact
    dequant, the f16 paths (matmul_coop_q8_0 / matmul128h: X and q·d rounded to f16 by numpy's own conversion) against
    the fp64 product of the rounded operands — f32 summation bar 1e-6; the two paths differ by ~3e-4, so a dropped or
    misplaced rounding fails"""
    rng = np.random.default_rng(m * n + k)
    blocks, _ = orc.q8_0_quantize(rng.normal(0, 0.3, n * k).astype(np.float32))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    W = np_dequant(blocks, n, k)
    ref32 = x.astype(np.float64) @ W.T
    ref16 = x.astype(np.float16).astype(np.float64) @ W.astype(np.float16).astype(np.float64).T
    y32, y16 = orc.matmul_q8_0(x, blocks, n), orc.matmul_q8_0(x, blocks, n, r16=True)
    assert rel_l2(y32, ref32) < 1e-6 and rel_l2(y16, ref16) < 1e-6
    assert rel_l2(ref16, ref32) > 1e-4
    base = rng.normal(0, 1, (m, n)).astype(np.float32)
    assert rel_l2(orc.matmul_q8_0(x, blocks, n, y=base, r16=True) - base, ref16) < 1e-5


def test_oracle_f16_prefill_matches_fp64_forward_with_rounded_operands():
    """the oracle's f16-path prefill against the fp64 forward whose layer GEMMs take f16-rounded X and W, on the
    reference's tiny model. The bar (5e-3) is the path's own sensitivity: a 1e-7 relative nudge of the embeddings moves
    that fp64 forward by 1.0e-3 (its f32-path twin: 3.7e-6), so two correct f16-path results differ at that level;
    the F32 path's prefill stays pinned at 1e-3 above and matches its forward to 3e-5"""
    cfg, te, on, layers = tiny_text_model()
    prompt = tiny_prompt()
    want16 = np_forward(cfg, te, on, layers, list(prompt), r16=True)[-1]
    got = orc.Session(cfg, te, on, layers, 32, f16=True).prefill(prompt)
    assert rel_l2(got, want16) < 5e-3
    assert int(np.argmax(got)) == int(np.argmax(want16))


def test_oracle_step_equals_prefill_row():
    """prefill of n tokens then one step = the last logits of a prefill of n + 1 tokens (up to f32 order)"""
    cfg, te, on, layers = tiny_text_model()
    prompt = tiny_prompt()
    a = orc.Session(cfg, te, on, layers, 32)
    a.prefill(prompt[:-1])
    la = a.step(int(prompt[-1]))
    b = orc.Session(cfg, te, on, layers, 32)
    lb = b.prefill(prompt)
    assert rel_l2(la, lb) < 1e-5
    with pytest.raises(ValueError):
        b.step(cfg["n_vocab"])


def test_oracle_step_forms_agree_and_kv_rows_round_trip():
    """the F32 path's step and the fused step are the same function in two f32 orders: rel-L2 ≤ 5e-5 over 6 steps
    (measured 0.5–1.6e-5 — each step stores its K / V row in f16, where the two orders' last bits now and then round
    to neighbouring f16 values, 2^-11 apart; the prompt's rows are the same in both);
    cache rows handed from one session to another (get_kv → set_kv) make the receiver step exactly as the giver; the
    rows a prefill stores for layer 0 are the f16 of the closed-form K / V (per-head RMS norm + RoPE NEOX of
    rms_norm(embed)·Wkᵀ; V = rms_norm(embed)·Wvᵀ) within one f16 rounding"""
    cfg, te, on, layers = tiny_text_model()
    prompt = tiny_prompt()
    extra = [int(t) for t in orc.Lcg(9).bits(6) % cfg["n_vocab"]]
    a = orc.Session(cfg, te, on, layers, 64, step_f32=True)
    b = orc.Session(cfg, te, on, layers, 64, step_f32=False)
    a.prefill(prompt)
    b.prefill(prompt)
    for t in extra:
        assert rel_l2(a.step(t), b.step(t)) < 5e-5
    # the hand-over: a third session gets a's rows and steps bit-identically with a
    c = orc.Session(cfg, te, on, layers, 64, step_f32=True)
    n = a.n_past
    for li in range(cfg["n_layer"]):
        k, v = a.get_kv(li, 0, n)
        c.set_kv(li, 0, k, v)
        k2, v2 = c.get_kv(li, 0, n)
        assert np.array_equal(k, k2) and np.array_equal(v, v2)
    c.rewind(n)
    assert np.array_equal(a.step(7), c.step(7))
    with pytest.raises(ValueError):
        c.get_kv(cfg["n_layer"], 0, 1)
    with pytest.raises(ValueError):
        c.get_kv(0, 60, 5)
    # layer 0's rows against the closed form
    d, nkv = cfg["dim"], cfg["n_kv"]
    E = np_dequant(te, cfg["n_vocab"], d)
    x = E[np.asarray(prompt)]
    h = np_rms(x, layers[0]["attn_norm"], cfg["eps"])
    kr = (h @ np_dequant(layers[0]["k"], nkv * 128, d).T).reshape(len(prompt), nkv, 128)
    vr = (h @ np_dequant(layers[0]["v"], nkv * 128, d).T).reshape(len(prompt), nkv * 128)
    kw = np.stack([np_rope(np_rms(kr[t], layers[0]["k_norm"], cfg["eps"]), t) for t in range(len(prompt))])
    k0, v0 = a.get_kv(0, 0, len(prompt))
    kf = k0.view(np.float16).astype(np.float64).reshape(len(prompt), nkv, 128)
    vf = v0.view(np.float16).astype(np.float64)
    assert np.all(np.abs(kf - kw) <= 1e-3 * (1 + np.abs(kw)))
    assert np.all(np.abs(vf - vr) <= 1e-3 * (1 + np.abs(vr)))
