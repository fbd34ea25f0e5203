"""ctypes wrapper of liboracle.so — the CPU restatement of the reference decode path (htr_oracle.h).

TEST INFRASTRUCTURE ONLY. This module is the checker: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import it; the product (historic-htr-ocr_amd/) never does. Each function names the reference lines it restates in
htr_oracle.h. Built by oracle/Makefile (`make -C oracle`).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        l = C.CDLL(LIB_PATH)
        vp, sz, i32, f32, f64 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_double
        sig = {
            "or_lcg_fill": (None, [C.POINTER(C.c_uint64), vp, sz, f32]),
            "or_lcg_bits": (None, [C.POINTER(C.c_uint64), vp, sz]),
            "or_f16_from_f32": (C.c_uint16, [f32]),
            "or_f32_from_f16": (f32, [C.c_uint16]),
            "or_f16_from_f32_n": (None, [vp, vp, sz]),
            "or_q8_0_quantize": (None, [vp, sz, vp, vp]),
            "or_q8_0_dequant": (None, [vp, sz, vp]),
            "or_matvec_q8_0": (None, [vp, sz, sz, vp, vp, i32]),
            "or_dmv": (None, [vp, sz, sz, vp, vp, f32, vp, i32]),
            "or_dmv_qkv": (None, [vp, vp, vp, sz, sz, sz, vp, vp, f32, vp]),
            "or_dmv_ffn": (None, [vp, vp, sz, sz, vp, vp, f32, vp]),
            "or_matvec_q8_0_f64": (None, [vp, sz, sz, vp, vp]),
            "or_rms_norm": (None, [vp, vp, vp, sz, sz, f32]),
            "or_rope_table": (None, [f32, sz, sz, vp]),
            "or_qkv_post": (None, [vp, vp, vp, vp, i32, i32, i32, f32, vp, vp]),
            "or_attn_decode": (None, [vp, vp, vp, sz, i32, i32, i32, f32, vp]),
            "or_attn_causal": (None, [vp, vp, vp, sz, i32, i32, i32, i32, f32, vp]),
            "or_attn_f64": (None, [vp, vp, vp, sz, i32, i32, i32, f64, vp]),
            "or_choose": (C.c_int32, [vp, sz, f64, sz, f64, vp, sz, vp, vp, sz]),
            "or_session_new": (vp, [vp, vp, vp, vp, i32]),
            "or_session_free": (None, [vp]),
            "or_session_n_past": (i32, [vp]),
            "or_session_prefill": (i32, [vp, vp, i32, vp]),
            "or_session_step": (i32, [vp, C.c_int32, vp]),
            "or_session_rewind": (None, [vp, i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


class Lcg:
    """text.rs:670-673 — the reference tests' generator."""

    def __init__(self, seed: int):
        self.s = C.c_uint64(seed)

    def f32(self, n: int, scale: float = 1.0) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().or_lcg_fill(C.byref(self.s), _p(out), n, scale)
        return out

    def bits(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint32)
        lib().or_lcg_bits(C.byref(self.s), _p(out), n)
        return out


def f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.uint16)
    lib().or_f16_from_f32_n(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return np.array([lib().or_f32_from_f16(int(v)) for v in np.asarray(h).ravel()], dtype=np.float32)


def q8_0_quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    blocks = np.empty(x.size // 32 * 34, dtype=np.uint8)
    deq = np.empty(x.size, dtype=np.float32)
    lib().or_q8_0_quantize(_p(x), x.size, _p(blocks), _p(deq))
    return blocks, deq


def q8_0_dequant(blocks: np.ndarray, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().or_q8_0_dequant(_p(blocks), n, _p(out))
    return out


def matvec_q8_0(w, rows, k, x, y=None, acc=False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(rows, np.float32) if y is None else np.array(y, dtype=np.float32)
    lib().or_matvec_q8_0(_p(w), rows, k, _p(x), _p(y), int(acc))
    return y


def dmv(w, rows, k, x, nw=None, eps=1e-6, y=None, acc=False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    nw = None if nw is None else np.ascontiguousarray(nw, dtype=np.float32)
    y = np.zeros(rows, np.float32) if y is None else np.array(y, dtype=np.float32)
    lib().or_dmv(_p(w), rows, k, _p(x), _p(nw), eps, _p(y), int(acc))
    return y


def dmv_qkv(wq, wk, wv, nq, nkv, k, x, nw, eps) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    nw = np.ascontiguousarray(nw, dtype=np.float32)
    y = np.zeros(nq + 2 * nkv, np.float32)
    lib().or_dmv_qkv(_p(wq), _p(wk), _p(wv), nq, nkv, k, _p(x), _p(nw), eps, _p(y))
    return y


def dmv_ffn(wg, wu, rows, k, x, nw, eps) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    nw = np.ascontiguousarray(nw, dtype=np.float32)
    g = np.zeros(rows, np.float32)
    lib().or_dmv_ffn(_p(wg), _p(wu), rows, k, _p(x), _p(nw), eps, _p(g))
    return g


def matvec_f64(w, rows, k, x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(rows, np.float64)
    lib().or_matvec_q8_0_f64(_p(w), rows, k, _p(x), _p(y))
    return y


def rms_norm(x, w, rows, dim, eps) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty(rows * dim, np.float32)
    lib().or_rms_norm(_p(x), _p(w), _p(y), rows, dim, eps)
    return y


def rope_table(base: float, d_head: int, n_pos: int) -> np.ndarray:
    out = np.empty(n_pos * d_head, np.float32)
    lib().or_rope_table(base, d_head, n_pos, _p(out))
    return out


def qkv_post(qkv, qn, kn, cs, n_head, n_kv, pos, eps):
    """→ (qkv with q heads normed + roped, k row f16 bits [n_kv·128], v row f16 bits)"""
    qkv = np.array(qkv, dtype=np.float32)
    kr = np.zeros(n_kv * 128, np.uint16)
    vr = np.zeros(n_kv * 128, np.uint16)
    lib().or_qkv_post(_p(qkv), _p(np.ascontiguousarray(qn, np.float32)), _p(np.ascontiguousarray(kn, np.float32)),
                      _p(np.ascontiguousarray(cs, np.float32)), n_head, n_kv, pos, eps, _p(kr), _p(vr))
    return qkv, kr, vr


def attn_decode(q, k, v, kv_stride, n_keys, n_head, n_kv, scale) -> np.ndarray:
    out = np.empty(n_head * 128, np.float32)
    lib().or_attn_decode(_p(np.ascontiguousarray(q, np.float32)), _p(k), _p(v), kv_stride, n_keys, n_head, n_kv,
                         scale, _p(out))
    return out


def attn_causal(q, k, v, kv_stride, n_q, pos0, n_head, n_kv, scale) -> np.ndarray:
    out = np.empty(n_q * n_head * 128, np.float32)
    lib().or_attn_causal(_p(np.ascontiguousarray(q, np.float32)), _p(k), _p(v), kv_stride, n_q, pos0, n_head, n_kv,
                         scale, _p(out))
    return out


def attn_f64(q, k, v, kv_stride, n_keys, n_head, n_kv, scale) -> np.ndarray:
    out = np.empty(n_head * 128, np.float64)
    lib().or_attn_f64(_p(np.ascontiguousarray(q, np.float32)), _p(k), _p(v), kv_stride, n_keys, n_head, n_kv, scale,
                      _p(out))
    return out


def choose(logits: np.ndarray, rp: float, window: int, fp: float, history, counts: dict | None = None) -> int:
    """sampling.rs:38-62 on `logits` (penalised IN PLACE, like the reference's &mut [f32])."""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    hist = np.ascontiguousarray(history, dtype=np.int32)
    counts = counts or {}
    ct = np.array(list(counts.keys()), dtype=np.int32)
    cn = np.array(list(counts.values()), dtype=np.uint32)
    return int(lib().or_choose(_p(logits), logits.size, rp, window, fp, _p(hist) if hist.size else None, hist.size,
                               _p(ct) if ct.size else None, _p(cn) if cn.size else None, ct.size))


class TextCfg(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("dim", C.c_int), ("n_head", C.c_int), ("n_kv", C.c_int), ("d_head", C.c_int),
                ("n_ff", C.c_int), ("n_vocab", C.c_int), ("eps", C.c_float), ("rope_base", C.c_float)]


class LayerC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm", "k_norm",
                                          "ffn_norm")]


class Session:
    """The decoder restated (text.rs:437-658): prefill on the F32 path's kernels, steps on the fused f16-path kernels.
    The weights are the same host tensors the library gets (dicts of q8_0 block bytes / f32 norms)."""

    def __init__(self, cfg: dict, tok_embd, output_norm, layers: list[dict], n_ctx: int):
        self._keep = [tok_embd, output_norm, layers]
        self.cfg = cfg
        c = TextCfg(cfg["n_layer"], cfg["dim"], cfg["n_head"], cfg["n_kv"], 128, cfg["n_ff"], cfg["n_vocab"],
                    cfg.get("eps", 1e-6), cfg.get("rope_base", 1e6))
        arr = (LayerC * cfg["n_layer"])()
        for i, ly in enumerate(layers):
            arr[i] = LayerC(**{k: _p(ly[k]) for k in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm",
                                                      "k_norm", "ffn_norm")})
        self._arr = arr
        self.h = lib().or_session_new(C.byref(c), _p(tok_embd), _p(output_norm), arr, n_ctx)
        if not self.h:
            raise ValueError("oracle session: unsupported shape")

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_session_free(self.h)
            self.h = None

    @property
    def n_past(self) -> int:
        return lib().or_session_n_past(self.h)

    def rewind(self, n_past: int) -> None:
        lib().or_session_rewind(self.h, n_past)

    def prefill(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.cfg["n_vocab"], np.float32)
        if lib().or_session_prefill(self.h, _p(ids), ids.size, _p(out)) != 0:
            raise ValueError("oracle prefill: bad id or overflow")
        return out

    def step(self, tok: int) -> np.ndarray:
        out = np.empty(self.cfg["n_vocab"], np.float32)
        if lib().or_session_step(self.h, int(tok), _p(out)) != 0:
            raise ValueError("oracle step: bad id or overflow")
        return out
