"""Shared test inputs: the reference tests' seeded generators, model builders, tolerances."""
from __future__ import annotations

import numpy as np

import oracle as orc


def rel_l2(got, want) -> float:
    """text.rs:1100-1107"""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.sqrt(np.sum((got - want) ** 2) / np.sum(want ** 2)))


def norm_vec(n: int, k: int) -> np.ndarray:
    """text.rs:1305: 1 + 0.01·((i·7 + k) mod 13)"""
    return np.array([1.0 + 0.01 * ((i * 7 + k) % 13) for i in range(n)], dtype=np.float32)


def tiny_text_model():
    """text.rs:1297-1323 tiny_text_model: 5 layers, dim 256, 2 q / 1 kv head of 128, ffn 512, vocab 1000, q8_0
    weights from the LCG (seed 31) in the reference's draw order, norms near 1. → (cfg, tok_embd, output_norm,
    layers)"""
    n_layer, dim, n_head, n_kv, d_head, n_ff, n_vocab = 5, 256, 2, 1, 128, 512, 1000
    g = orc.Lcg(31)

    def w(rows, cols, scale):
        return orc.q8_0_quantize(g.f32(rows * cols, scale))[0]

    qd, kvd = n_head * d_head, n_kv * d_head
    layers = []
    for i in range(n_layer):
        ly = {"attn_norm": norm_vec(dim, i)}
        ly["q"] = w(qd, dim, 0.2)
        ly["k"] = w(kvd, dim, 0.2)
        ly["v"] = w(kvd, dim, 0.2)
        ly["o"] = w(dim, qd, 0.1)
        ly["q_norm"] = norm_vec(d_head, i + 1)
        ly["k_norm"] = norm_vec(d_head, i + 2)
        ly["ffn_norm"] = norm_vec(dim, i + 3)
        ly["gate"] = w(n_ff, dim, 0.2)
        ly["up"] = w(n_ff, dim, 0.2)
        ly["down"] = w(dim, n_ff, 0.1)
        layers.append(ly)
    tok_embd = w(n_vocab, dim, 1.0)
    cfg = dict(n_layer=n_layer, dim=dim, n_head=n_head, n_kv=n_kv, d_head=d_head, n_ff=n_ff, n_vocab=n_vocab,
               n_ctx_train=4096, eps=1e-6, rope_base=1e6)
    return cfg, tok_embd, norm_vec(dim, 0), layers


def tiny_prompt(n: int = 20) -> np.ndarray:
    """text.rs:1333: ((lcg + 1)·499) as Token, seed 5"""
    v = orc.Lcg(5).f32(n)
    return ((v + np.float32(1.0)) * np.float32(499.0)).astype(np.int32)


def synth_text_model(n_layer=28, dim=1024, n_head=16, n_kv=8, n_ff=3072, n_vocab=151936, seed=1000):
    """The Qwen3-0.6B-shaped random decoder (htr.synth.text_model)."""
    from htr import synth

    return synth.text_model(n_layer, dim, n_head, n_kv, n_ff, n_vocab, seed)


def to_htr_cfg(cfg: dict):
    import htr

    return htr.TextConfig(**cfg)


def near_tie(logits_ref: np.ndarray, want: int, got: int, rel: float = 1e-6) -> bool:
    """A documented near-tie: the reference's logits of its choice and of ours differ by less than `rel` relative."""
    a, b = float(logits_ref[want]), float(logits_ref[got])
    return abs(a - b) <= rel * max(abs(a), abs(b), 1e-30)


def kv_head_major(rows: np.ndarray, n_kv: int) -> np.ndarray:
    """[n_keys][n_kv·128] → [n_kv][n_keys][128] (this library's cache layout)"""
    n = rows.shape[0]
    return np.ascontiguousarray(rows.reshape(n, n_kv, 128).transpose(1, 0, 2))
