"""qkv_post and the split-K GQA decode attention on the GPU against the oracle and fp64 softmax attention."""
import numpy as np
import pytest

import htr
import oracle as orc
from helpers import kv_head_major, rel_l2

pytestmark = pytest.mark.gpu


def test_qkv_post_reference_shape(dev):
    """text.rs:926-972: 4 q heads, 2 kv heads, position 5 of a 7-row cache"""
    n_head, n_kv, pos, n_ctx, eps = 4, 2, 5, 7, 1e-6
    g = orc.Lcg(43)
    raw = g.f32((n_head + 2 * n_kv) * 128, 3.0)
    qn, kn = g.f32(128), g.f32(128)
    cs = orc.rope_table(1e6, 128, n_ctx)
    q_want, k_want, v_want = orc.qkv_post(raw, qn, kn, cs, n_head, n_kv, pos, eps)
    qkv = dev.upload(raw)
    kc, vc = dev.alloc(n_kv * n_ctx * 128 * 2), dev.alloc(n_kv * n_ctx * 128 * 2)
    htr.qkv_post(dev, qkv, dev.upload(qn), dev.upload(kn), dev.upload(cs), n_head, n_kv, pos, n_ctx, eps, kc, vc)
    q = qkv.download(np.float32)
    assert np.all(np.abs(q[: n_head * 128] - q_want[: n_head * 128]) < 1e-5 * (1 + np.abs(q_want[: n_head * 128])))
    k = kc.download(np.uint16).reshape(n_kv, n_ctx, 128)[:, pos].ravel()
    v = vc.download(np.uint16).reshape(n_kv, n_ctx, 128)[:, pos].ravel()
    assert np.array_equal(v, v_want)  # the V store is RNE f16 of the raw value, bit for bit
    kf, kw = k.view(np.float16).astype(np.float64), k_want.view(np.float16).astype(np.float64)
    assert np.all(np.abs(kf - kw) <= 2.0 ** -10 * np.abs(kw) + 1e-7)  # within one f16 step
    # the other cache rows stay untouched
    assert not kc.download(np.uint16).reshape(n_kv, n_ctx, 128)[:, :pos].any()


def _attention_case(dev, n_head, n_kv, n_keys, n_ctx, q, k_rows, v_rows):
    kc = dev.upload(kv_head_major(np.pad(k_rows, ((0, n_ctx - n_keys), (0, 0))), n_kv))
    vc = dev.upload(kv_head_major(np.pad(v_rows, ((0, n_ctx - n_keys), (0, 0))), n_kv))
    out = dev.alloc(n_head * 128 * 4)
    sc = np.float32(1 / np.sqrt(128))
    htr.decode_attention(dev, dev.upload(q), kc, vc, n_head, n_kv, n_ctx, n_keys, float(sc), out)
    return out.download(np.float32)


def test_decode_attention_reference_shape(dev):
    """text.rs:1264-1292: 300 keys (several chunks), 4 q heads on 2 kv heads, rel-L2 < 1e-5"""
    n_head, n_kv, n = 4, 2, 300
    g = orc.Lcg(31)
    k = orc.f16_bits(g.f32(n * n_kv * 128, 2.0)).reshape(n, -1)
    v = orc.f16_bits(g.f32(n * n_kv * 128)).reshape(n, -1)
    q = g.f32(n_head * 128, 2.0)
    got = _attention_case(dev, n_head, n_kv, n, n + 3, q, k, v)
    want = orc.attn_f64(q, k, v, n_kv * 128, n, n_head, n_kv, 1 / np.sqrt(128))
    assert rel_l2(got, want) < 1e-5
    assert rel_l2(got, orc.attn_decode(q, k, v, n_kv * 128, n, n_head, n_kv, np.float32(1 / np.sqrt(128)))) < 1e-5


@pytest.mark.parametrize("n_keys", [1, 2, 63, 64, 65, 129, 1537])
def test_decode_attention_edge_lengths(dev, n_keys):
    n_head, n_kv = 16, 8
    g = orc.Lcg(n_keys)
    k = orc.f16_bits(g.f32(n_keys * n_kv * 128, 2.0)).reshape(n_keys, -1)
    v = orc.f16_bits(g.f32(n_keys * n_kv * 128)).reshape(n_keys, -1)
    q = g.f32(n_head * 128, 2.0)
    got = _attention_case(dev, n_head, n_kv, n_keys, n_keys + 5, q, k, v)
    assert rel_l2(got, orc.attn_f64(q, k, v, n_kv * 128, n_keys, n_head, n_kv, 1 / np.sqrt(128))) < 1e-5


def test_decode_attention_merge_across_launches_and_scopes(dev):
    """one launch after another on the same device scratch: 8 KV heads (a head's chunks on one XCD, the partials and
    the ticket in its L2) at chunk counts that rise and fall (1 … 32 chunks a head), 2 KV heads (the merge through the
    coherence point) in between, and the allocation-free entry point — every output against fp64, so a ticket left
    off zero by any launch would show in the next"""
    cases = []
    for n_keys in (300, 17, 2048, 16, 1537, 8192, 33, 513):
        cases.append((16, 8, n_keys))
        if n_keys in (17, 1537):
            cases.append((4, 2, n_keys))
    sc = 1 / np.sqrt(128)
    for i, (n_head, n_kv, n_keys) in enumerate(cases):
        g = orc.Lcg(700 + i)
        k = orc.f16_bits(g.f32(n_keys * n_kv * 128, 2.0)).reshape(n_keys, -1)
        v = orc.f16_bits(g.f32(n_keys * n_kv * 128)).reshape(n_keys, -1)
        q = g.f32(n_head * 128, 2.0)
        want = orc.attn_f64(q, k, v, n_kv * 128, n_keys, n_head, n_kv, sc)
        got = _attention_case(dev, n_head, n_kv, n_keys, n_keys + 3, q, k, v)
        assert rel_l2(got, want) < 1e-5, (n_head, n_kv, n_keys)
        if n_kv == 8 and n_keys <= 2048:
            n_ctx = n_keys + 3
            kc = dev.upload(kv_head_major(np.pad(k, ((0, 3), (0, 0))), n_kv))
            vc = dev.upload(kv_head_major(np.pad(v, ((0, 3), (0, 0))), n_kv))
            qb, out = dev.upload(q), dev.alloc(n_head * 128 * 4)
            rc = htr.lib().htr_decode_attention_static(dev.h, qb.ptr, kc.ptr, vc.ptr, n_head, n_kv, n_ctx, n_keys,
                                                       float(np.float32(sc)), out.ptr)
            assert rc == 0, htr.last_error()
            assert rel_l2(out.download(np.float32), want) < 1e-5, ("static", n_keys)
            for b in (kc, vc, qb, out):
                b.free()


@pytest.mark.parametrize("L", [512, 2048, 8192])
def test_config2_attention(dev, L):
    """16 q / 8 kv heads × 128, K / V ~ N(0,1) f16, q ~ N(0,1) → per-head RMSNorm (ε 1e-6, weights
    1 + N(0, 0.02)) → RoPE θ = 1e6 at position L; n_keys = L; scale 1/√128; rel-L2 ≤ 1e-3 against fp64"""
    n_head, n_kv, eps = 16, 8, 1e-6
    k = orc.f16_bits(htr.synth_normal(10 + L, L * n_kv * 128)).reshape(L, -1)
    v = orc.f16_bits(htr.synth_normal(20 + L, L * n_kv * 128)).reshape(L, -1)
    qraw = np.concatenate([htr.synth_normal(30 + L, n_head * 128), np.zeros(2 * n_kv * 128, np.float32)])
    qn = htr.synth_normal(40, 128, 1.0, 0.02)
    kn = htr.synth_normal(41, 128, 1.0, 0.02)
    cs = orc.rope_table(1e6, 128, L + 1)
    n_ctx = L + 1
    kc = dev.upload(kv_head_major(np.pad(k, ((0, 1), (0, 0))), n_kv))
    vc = dev.upload(kv_head_major(np.pad(v, ((0, 1), (0, 0))), n_kv))
    qkv = dev.upload(qraw)
    htr.qkv_post(dev, qkv, dev.upload(qn), dev.upload(kn), dev.upload(cs), n_head, n_kv, L, n_ctx, eps, kc, vc)
    q_gpu = qkv.download(np.float32)[: n_head * 128]
    q_or = orc.qkv_post(qraw, qn, kn, cs, n_head, n_kv, L, eps)[0][: n_head * 128]
    assert rel_l2(q_gpu, q_or) < 1e-6
    out = dev.alloc(n_head * 128 * 4)
    htr.decode_attention(dev, qkv, kc, vc, n_head, n_kv, n_ctx, L, float(np.float32(1 / np.sqrt(128))), out)
    got = out.download(np.float32)
    want = orc.attn_f64(q_gpu, k, v, n_kv * 128, L, n_head, n_kv, 1 / np.sqrt(128))
    assert rel_l2(got, want) < 1e-3
    assert rel_l2(got, want) < 1e-5  # what the kernel actually reaches (f32 throughout)


@pytest.mark.parametrize("n_q,pos0,n_head,n_kv,n_ctx", [(1, 0, 4, 2, 8), (17, 0, 4, 2, 40), (33, 5, 4, 2, 64),
                                                      (100, 37, 16, 8, 160), (1023, 0, 16, 8, 1536),
                                                      (200, 1000, 16, 8, 1536)])
def test_causal_attention_matches_oracle(dev, n_q, pos0, n_head, n_kv, n_ctx):
    """attention_causal.wgsl (text.rs:484-499): queries at positions pos0 … over the keys 0 … each one's position —
    against the oracle's f32 restatement and, for sampled queries, fp64 softmax attention (bar 1e-5: f32-grade
    products and sums on both sides). The cache rows past the last key hold large values: reading them would show."""
    n_keys = pos0 + n_q
    g = orc.Lcg(n_q * 7 + pos0)
    k = orc.f16_bits(g.f32(n_keys * n_kv * 128, 2.0)).reshape(n_keys, -1)
    v = orc.f16_bits(g.f32(n_keys * n_kv * 128)).reshape(n_keys, -1)
    q = g.f32(n_q * n_head * 128, 2.0)
    big = np.full((n_ctx - n_keys, n_kv * 128), np.float16(3.0e4).view(np.uint16), np.uint16)
    kc = dev.upload(kv_head_major(np.concatenate([k, big]), n_kv))
    vc = dev.upload(kv_head_major(np.concatenate([v, big]), n_kv))
    out = dev.alloc(n_q * n_head * 128 * 4)
    sc = float(np.float32(1 / np.sqrt(128)))
    htr.causal_attention(dev, dev.upload(q), kc, vc, n_q, pos0, n_head, n_kv, n_ctx, sc, out)
    got = out.download(np.float32).reshape(n_q, n_head * 128)
    want = orc.attn_causal(q, k, v, n_kv * 128, n_q, pos0, n_head, n_kv, sc).reshape(n_q, n_head * 128)
    e = rel_l2(got, want)
    print(f"\n[causal {n_q} queries from {pos0}] rel-L2 vs the oracle {e:.2e}")
    assert e < 1e-5
    for t in sorted({0, n_q // 2, n_q - 1}):
        row = orc.attn_f64(q[t * n_head * 128:(t + 1) * n_head * 128], k, v, n_kv * 128, pos0 + t + 1, n_head, n_kv,
                           1 / np.sqrt(128))
        assert rel_l2(got[t], row) < 1e-5, t


def test_causal_attention_rejects_bad_ranges(dev):
    q, kc, vc, out = dev.alloc(4 * 128 * 4), dev.alloc(2 * 8 * 128 * 2), dev.alloc(2 * 8 * 128 * 2), dev.alloc(4 * 128 * 4)
    with pytest.raises(htr.HtrError, match="queries from position"):
        htr.causal_attention(dev, q, kc, vc, 2, 7, 4, 2, 8, 0.1, out)
    with pytest.raises(htr.HtrError, match="groups of 2"):
        htr.causal_attention(dev, q, kc, vc, 1, 0, 6, 2, 8, 0.1, out)
