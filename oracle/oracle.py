"""ctypes wrapper of liboracle.so — the CPU restatement of the reference decode path (htr_oracle.h).

TEST INFRASTRUCTURE ONLY. This module checks the product and is never part of it: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
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
            "or_choice_matrix_logits": (None, [C.POINTER(C.c_uint64), i32, sz, vp]),
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
            "or_rng_next_f64": (f64, [C.POINTER(C.c_uint64)]),
            "or_choose_sampled": (C.c_int32, [vp, sz, f64, f64, f64, sz, f64, vp, sz, vp, vp, sz,
                                              C.POINTER(C.c_uint64)]),
            "or_session_new": (vp, [vp, vp, vp, vp, i32]),
            "or_session_free": (None, [vp]),
            "or_session_n_past": (i32, [vp]),
            "or_session_prefill": (i32, [vp, vp, i32, vp]),
            "or_session_step": (i32, [vp, C.c_int32, vp]),
            "or_session_rewind": (None, [vp, i32]),
            "or_session_set_f16": (None, [vp, i32]),
            "or_session_set_step_f32": (None, [vp, i32]),
            "or_session_get_kv": (i32, [vp, i32, i32, i32, vp, vp]),
            "or_session_set_kv": (i32, [vp, i32, i32, i32, vp, vp]),
            "or_attn_decode_f32": (None, [vp, vp, vp, sz, i32, i32, i32, f32, vp]),
            "or_matmul_q8_0": (None, [vp, vp, vp, sz, sz, sz, i32, i32]),
            "or_pixel_lut": (None, [vp, vp, vp]),
            "or_patchify": (None, [vp, i32, i32, i32, i32, vp, vp]),
            "or_rope2d_table": (None, [f32, i32, i32, vp]),
            "or_rope2d": (None, [vp, i32, i32, i32, i32, i32, vp]),
            "or_rms_norm_h": (None, [vp, vp, vp, sz, sz, f32]),
            "or_q8_0_to_f16": (None, [vp, sz, f32, vp]),
            "or_matmul_f16": (None, [vp, vp, vp, sz, sz, sz, i32]),
            "or_ffn_f16": (None, [vp, vp, vp, vp, sz, sz, sz, f32]),
            "or_matmul_f32": (None, [vp, vp, vp, sz, sz, sz, i32]),
            "or_attention_coop": (None, [vp, vp, vp, vp, i32, i32, f32]),
            "or_unfold2x2": (None, [vp, vp, i32, i32, i32]),
            "or_gelu": (None, [vp, sz]),
            "or_vision_encode": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
            "or_vision_encode_w16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
            "or_vision_resume": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, vp, i32, i32, i32, vp]),
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

    def choice_matrix(self, mode: int, n: int) -> np.ndarray:
        """the logits of text.rs:1021-1027 for one step's mode (0 … 3), drawn in the reference's order"""
        out = np.empty(n, dtype=np.float32)
        lib().or_choice_matrix_logits(C.byref(self.s), mode, n, _p(out))
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
    qn, kn, cs = (np.ascontiguousarray(a, np.float32) for a in (qn, kn, cs))
    lib().or_qkv_post(_p(qkv), _p(qn), _p(kn), _p(cs), n_head, n_kv, pos, eps, _p(kr), _p(vr))
    return qkv, kr, vr


def attn_decode(q, k, v, kv_stride, n_keys, n_head, n_kv, scale) -> np.ndarray:
    out = np.empty(n_head * 128, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    lib().or_attn_decode(_p(q), _p(k), _p(v), kv_stride, n_keys, n_head, n_kv, scale, _p(out))
    return out


def attn_decode_f32(q, k, v, kv_stride, n_keys, n_head, n_kv, scale) -> np.ndarray:
    """the F32 path's three-kernel decode attention (attn_scores / attn_softmax / attn_values)"""
    out = np.empty(n_head * 128, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    lib().or_attn_decode_f32(_p(q), _p(k), _p(v), kv_stride, n_keys, n_head, n_kv, scale, _p(out))
    return out


def attn_causal(q, k, v, kv_stride, n_q, pos0, n_head, n_kv, scale) -> np.ndarray:
    out = np.empty(n_q * n_head * 128, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    lib().or_attn_causal(_p(q), _p(k), _p(v), kv_stride, n_q, pos0, n_head, n_kv, scale, _p(out))
    return out


def attn_f64(q, k, v, kv_stride, n_keys, n_head, n_kv, scale) -> np.ndarray:
    out = np.empty(n_head * 128, np.float64)
    q = np.ascontiguousarray(q, np.float32)
    lib().or_attn_f64(_p(q), _p(k), _p(v), kv_stride, n_keys, n_head, n_kv, scale, _p(out))
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


class Rng:
    """sampling.rs:23-35 Rng (SplitMix64), the oracle's"""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def next_f64(self) -> float:
        return lib().or_rng_next_f64(C.byref(self.state))


def choose_sampled(logits: np.ndarray, temperature: float, top_p: float, rp: float, window: int, fp: float, history,
                   counts: dict | None, rng: Rng) -> int:
    """sampling.rs:38-89 for any preset (logits penalised IN PLACE); rng advances when the preset samples"""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    hist = np.ascontiguousarray(history, dtype=np.int32)
    counts = counts or {}
    ct = np.array(list(counts.keys()), dtype=np.int32)
    cn = np.array(list(counts.values()), dtype=np.uint32)
    return int(lib().or_choose_sampled(_p(logits), logits.size, temperature, top_p, rp, window, fp,
                                       _p(hist) if hist.size else None, hist.size, _p(ct) if ct.size else None,
                                       _p(cn) if cn.size else None, ct.size, C.byref(rng.state)))


class TextCfg(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("dim", C.c_int), ("n_head", C.c_int), ("n_kv", C.c_int), ("d_head", C.c_int),
                ("n_ff", C.c_int), ("n_vocab", C.c_int), ("eps", C.c_float), ("rope_base", C.c_float)]


class LayerC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm", "k_norm",
                                          "ffn_norm")]


class Session:
    """The decoder restated (text.rs:437-658) on one compute path: the F32 path (exact q8_0 values in the prefill
    GEMMs, the F32 step of text.rs:555-576) or, with f16, the f16 paths (X and q·d rounded to f16 in the prefill GEMMs,
    the fused step of layers_fused). The weights are the same host tensors the library gets (dicts of q8_0 block
    bytes / f32 norms)."""

    def __init__(self, cfg: dict, tok_embd, output_norm, layers: list[dict], n_ctx: int, f16: bool = False,
                 step_f32: bool | None = None):
        """f16: the f16 paths' prefill rounding and fused step; step_f32 overrides the step's form (default: the F32
        path's step exactly when f16 is off)"""
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
        lib().or_session_set_f16(self.h, int(f16))
        lib().or_session_set_step_f32(self.h, int(not f16 if step_f32 is None else step_f32))
        self.n_ctx = n_ctx

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

    def get_kv(self, layer: int, pos0: int, n: int) -> tuple[np.ndarray, np.ndarray]:
        """cache rows [pos0, pos0 + n) of a layer as f16 bits [n][n_kv·128] (K, V)"""
        kvd = self.cfg["n_kv"] * 128
        k = np.empty((n, kvd), np.uint16)
        v = np.empty((n, kvd), np.uint16)
        if lib().or_session_get_kv(self.h, layer, pos0, n, _p(k), _p(v)) != 0:
            raise ValueError("oracle get_kv: outside the session")
        return k, v

    def set_kv(self, layer: int, pos0: int, k: np.ndarray, v: np.ndarray) -> None:
        """cache rows [pos0, pos0 + n) of a layer from f16 bits [n][n_kv·128]"""
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        n = k.shape[0]
        if lib().or_session_set_kv(self.h, layer, pos0, n, _p(k), _p(v)) != 0:
            raise ValueError("oracle set_kv: outside the session")


# ---- the vision encoder (htr_vision_oracle.c) ----------------------------------------------------------------------

def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def pixel_lut(mean, std) -> np.ndarray:
    out = np.empty(768, np.float32)
    mean, std = _f32(mean), _f32(std)
    lib().or_pixel_lut(_p(mean), _p(std), _p(out))
    return out


def patchify(rgb: np.ndarray, side: int, lut: np.ndarray) -> np.ndarray:
    """rgb u8 [h][w][3] → P [n][3·side²]"""
    h, w, _ = rgb.shape
    px, py = w // side, h // side
    out = np.empty((px * py, 3 * side * side), np.float32)
    rgb, lut = np.ascontiguousarray(rgb, np.uint8), _f32(lut)
    lib().or_patchify(_p(rgb), w, px, px * py, side, _p(lut), _p(out))
    return out


def rope2d_table(theta: float, d_head: int, max_pos: int) -> np.ndarray:
    """[2][max_pos][d/4][2] (cos, sin)"""
    out = np.empty((2, max_pos, d_head // 4, 2), np.float32)
    lib().or_rope2d_table(theta, d_head, max_pos, _p(out))
    return out


def rope2d(q: np.ndarray, n_head: int, d_head: int, px: int, max_pos: int, cs: np.ndarray) -> np.ndarray:
    q = np.array(q, dtype=np.float32)
    cs = _f32(cs)
    lib().or_rope2d(_p(q), q.shape[0], n_head, d_head, px, max_pos, _p(cs))
    return q


def rms_norm_h(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty(x.shape, np.float16)
    lib().or_rms_norm_h(_p(x), _p(w), _p(out), x.shape[0], x.shape[1], eps)
    return out


def q8_0_to_f16(blocks: np.ndarray, rows: int, cols: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty((rows, cols), np.float16)
    blocks = np.ascontiguousarray(blocks, np.uint8)
    lib().or_q8_0_to_f16(_p(blocks), rows * cols, scale, _p(out))
    return out


def matmul_q8_0(x: np.ndarray, w_blocks: np.ndarray, n: int, y=None, r16: bool = False) -> np.ndarray:
    """Batch::matmul with a q8_0 weight (gpu.rs:1963-2014): y (+)= x·Wᵀ, W [n][k] as q8_0 block bytes; r16: the f16
    paths' rounding of X and W"""
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    w_blocks = np.ascontiguousarray(w_blocks, np.uint8)
    assert w_blocks.size == n * (k // 32) * 34
    acc = y is not None
    y = np.zeros((m, n), np.float32) if y is None else np.ascontiguousarray(y, np.float32).copy()
    lib().or_matmul_q8_0(_p(x), _p(w_blocks), _p(y), m, n, k, int(acc), int(r16))
    return y


def matmul_f16(x16: np.ndarray, w16: np.ndarray, y=None) -> np.ndarray:
    x16 = np.ascontiguousarray(x16, np.float16)
    w16 = np.ascontiguousarray(w16, np.float16)
    m, k = x16.shape
    n = w16.shape[0]
    acc = y is not None
    y = np.zeros((m, n), np.float32) if y is None else np.array(y, dtype=np.float32)
    lib().or_matmul_f16(_p(x16), _p(w16), _p(y), m, n, k, int(acc))
    return y


def ffn_f16(x16, wg16, wu16, scale: float) -> np.ndarray:
    x16 = np.ascontiguousarray(x16, np.float16)
    m, k = x16.shape
    n = wg16.shape[0]
    out = np.empty((m, n), np.float16)
    wg16, wu16 = np.ascontiguousarray(wg16, np.float16), np.ascontiguousarray(wu16, np.float16)
    lib().or_ffn_f16(_p(x16), _p(wg16), _p(wu16), _p(out), m, n, k, scale)
    return out


def matmul_f32(x, w, y=None) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    acc = y is not None
    y = np.zeros((x.shape[0], w.shape[0]), np.float32) if y is None else np.array(y, dtype=np.float32)
    lib().or_matmul_f32(_p(x), _p(w), _p(y), x.shape[0], w.shape[0], x.shape[1], int(acc))
    return y


def attention_coop(q, k, v, n_head: int, scale: float) -> np.ndarray:
    """q / k / v f32 [n][n_head·64] → f16 [n][n_head·64]"""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty(q.shape, np.float16)
    lib().or_attention_coop(_p(q), _p(k), _p(v), _p(out), q.shape[0], n_head, scale)
    return out


def unfold2x2(x: np.ndarray, px: int, py: int) -> np.ndarray:
    x = _f32(x)
    out = np.empty(((px // 2) * (py // 2), 4 * x.shape[1]), np.float32)
    lib().or_unfold2x2(_p(x), _p(out), px, py, x.shape[1])
    return out


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().or_gelu(_p(x), x.size)
    return x


class VisionCfg(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("dim", C.c_int), ("n_head", C.c_int), ("d_head", C.c_int), ("n_ff", C.c_int),
                ("patch", C.c_int), ("merge", C.c_int), ("proj_dim", C.c_int), ("eps", C.c_float),
                ("rope_theta", C.c_float), ("mean", C.c_float * 3), ("std", C.c_float * 3)]


class VisionLayerC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("ln1", "ln2", "q", "k", "v", "o", "gate", "up", "down")]


def _vision_cfg_layers(cfg: dict, t: dict):
    c = VisionCfg(cfg["n_layer"], cfg["dim"], cfg["n_head"], 64, cfg["n_ff"], cfg["patch"], 2, cfg["proj_dim"],
                  cfg["eps"], cfg["rope_theta"], (C.c_float * 3)(*cfg["mean"]), (C.c_float * 3)(*cfg["std"]))
    arr = (VisionLayerC * cfg["n_layer"])()
    for i, ly in enumerate(t["layers"]):
        arr[i] = VisionLayerC(**{k: _p(ly[k]) for k in ("ln1", "ln2", "q", "k", "v", "o", "gate", "up", "down")})
    return c, arr


def vision_resume(cfg: dict, t: dict, x: np.ndarray, px: int, py: int, first: int, count: int,
                  project: bool = False) -> np.ndarray:
    """the encoder resumed from the residual x [px·py][dim] before layer `first`: layers first … first + count − 1,
    then (project) the projector (q8_0 host tensors, as vision_encode)"""
    c, arr = _vision_cfg_layers(cfg, t)
    x = np.ascontiguousarray(x, np.float32)
    n = px * py
    out = np.empty((n // 4, cfg["proj_dim"]) if project else (n, cfg["dim"]), np.float32)
    rc = lib().or_vision_resume(C.byref(c), arr, _p(t["input_norm"]), _p(t["merger"]), _p(t["mm1"]), _p(t["mm2"]),
                                px, py, _p(x), first, count, int(project), _p(out))
    if rc != 0:
        raise ValueError("oracle vision_resume: unsupported size")
    return out


def vision_encode(cfg: dict, t: dict, rgb: np.ndarray, n_layers: int = -1, w16: bool = False) -> np.ndarray:
    """vision.rs run_f16 + project on the host tensors `t` (q8_0 blocks / f32): n_layers < 0 → the projected
    embeddings [n/4][proj_dim]; else the residual after n_layers layers [n][dim]. w16: the layer and projector
    weights are f16 planes (uint16 [rows][cols], the down projection already × 64), as an mmproj's bf16 weights are
    converted at load (vision.rs:124-142)"""
    c = VisionCfg(cfg["n_layer"], cfg["dim"], cfg["n_head"], 64, cfg["n_ff"], cfg["patch"], 2, cfg["proj_dim"],
                  cfg["eps"], cfg["rope_theta"], (C.c_float * 3)(*cfg["mean"]), (C.c_float * 3)(*cfg["std"]))
    arr = (VisionLayerC * cfg["n_layer"])()
    for i, ly in enumerate(t["layers"]):
        arr[i] = VisionLayerC(**{k: _p(ly[k]) for k in ("ln1", "ln2", "q", "k", "v", "o", "gate", "up", "down")})
    h, w, _ = rgb.shape
    n = (h // cfg["patch"]) * (w // cfg["patch"])
    out = np.empty((n, cfg["dim"]) if n_layers >= 0 else (n // 4, cfg["proj_dim"]), np.float32)
    rgb = np.ascontiguousarray(rgb, np.uint8)
    fn = lib().or_vision_encode_w16 if w16 else lib().or_vision_encode
    rc = fn(C.byref(c), _p(t["patch_embd"]), _p(t["pre_ln"]), arr, _p(t["input_norm"]),
            _p(t["merger"]), _p(t["mm1"]), _p(t["mm2"]), _p(rgb), w, h, n_layers, _p(out))
    if rc != 0:
        raise ValueError("oracle vision_encode: unsupported size")
    return out
