"""ctypes binding of libhtr.so — the gfx950 LightOnOCR decode path behind include/htr.h.

The classes mirror the reference engine's types on this path (app/crates/ocr-wgpu/src): ``Device`` ≙ ``Gpu``
(gpu.rs:1101-1485), ``Weight`` ≙ ``Weight`` (gpu.rs, WeightType::Q8_0), ``TextModel`` / ``Session`` / ``Choice`` ≙
text.rs's ``TextModel`` / ``Session`` / ``Choice``, ``Session.decode_gpu`` ≙ ``TextModel::decode_gpu``. Errors raise
``HtrError`` with the library's message (the reference's anyhow messages carry the same numbers).

There is no fallback: without the built library every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhtr.so")

MEM_WEIGHTS, MEM_KV_CACHE, MEM_WORK, MEM_READBACK = 0, 1, 2, 3
COMPUTE_F32, COMPUTE_F16 = 0, 1

# every symbol include/htr.h declares
SYMBOLS = [
    "htr_last_error", "htr_device_open", "htr_device_close", "htr_alive", "htr_set_fatal_hook", "htr_debug_mark_lost",
    "htr_sync", "htr_device_set_compute", "htr_device_compute", "htr_device_info", "htr_timer_begin", "htr_timer_end", "htr_mem_live", "htr_alloc", "htr_free",
    "htr_upload", "htr_download", "htr_copy", "htr_debug_read", "htr_phase",
    "htr_weight_q8_0", "htr_weight_q8_0_f16", "htr_weight_free", "htr_weight_shape", "htr_matvec_q8_0",
    "htr_matvec_q8_0_many", "htr_matvec_qkv", "htr_matvec_ffn", "htr_qkv_post", "htr_decode_attention", "htr_causal_attention", "htr_choose",
    "htr_choose_many", "htr_matmul_q8_0", "htr_gemm_f16", "htr_gemm_ffn_f16", "htr_vision_create", "htr_vision_free",
    "htr_vision_get_config", "htr_vision_load_gguf", "htr_vision_out_shape", "htr_vision_encode", "htr_gguf_open", "htr_gguf_open_source", "htr_gguf_close",
    "htr_gguf_header", "htr_gguf_tensor", "htr_gguf_u32", "htr_gguf_f32", "htr_gguf_str", "htr_gguf_f32_array",
    "htr_gguf_read_small", "htr_text_model_create", "htr_text_model_free", "htr_text_model_load_gguf",
    "htr_text_model_config", "htr_session_create", "htr_session_create_grown", "htr_session_kv_rows",
    "htr_session_free",
    "htr_session_n_past", "htr_prefill", "htr_step", "htr_session_logits", "htr_session_rewind", "htr_choice_create", "htr_choice_free",
    "htr_decode_gpu", "htr_choose_host", "htr_generate", "htr_synth_q8_0", "htr_synth_normal",
    "htr_session_kv_cache", "htr_debug_last_kernel", "htr_capture_begin", "htr_capture_end", "htr_graph_launch",
    "htr_graph_free", "htr_decode_attention_static", "htr_session_profile_step", "htr_session_set_fused_step",
    "htr_session_fused_step", "htr_session_profile_fused_step", "htr_debug_handover", "htr_session_set_wait_limit",
]
STEP_EMBED, STEP_QKV, STEP_ATTENTION, STEP_O, STEP_FFN, STEP_DOWN, STEP_HEAD, STEP_ALL = 1, 2, 4, 8, 16, 32, 64, 127


class HtrError(RuntimeError):
    pass


class GpuBytes(C.Structure):
    _fields_ = [("weights", C.c_uint64), ("kv_cache", C.c_uint64), ("work", C.c_uint64), ("readback", C.c_uint64)]


class TextConfigC(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("dim", C.c_int), ("n_head", C.c_int), ("n_kv", C.c_int), ("d_head", C.c_int),
                ("n_ff", C.c_int), ("n_vocab", C.c_int), ("n_ctx_train", C.c_int), ("eps", C.c_float),
                ("rope_base", C.c_float)]


class LayerTensorsC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm", "q_norm", "k_norm",
                                          "ffn_norm")]


class GgufTensorC(C.Structure):
    _fields_ = [("name", C.c_char * 128), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("shape", C.c_uint64 * 4),
                ("n_elements", C.c_uint64), ("n_bytes", C.c_uint64), ("offset", C.c_uint64),
                ("file_offset", C.c_uint64)]


READ_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint64, C.c_void_p, C.c_size_t)


class KvViewC(C.Structure):
    _fields_ = [("d_k", C.c_void_p), ("d_v", C.c_void_p), ("n_layer", C.c_int), ("n_kv", C.c_int),
                ("n_ctx", C.c_int), ("d_head", C.c_int), ("layer_stride", C.c_size_t)]


class PresetC(C.Structure):
    _fields_ = [("temperature", C.c_double), ("top_p", C.c_double), ("repetition_penalty", C.c_double),
                ("frequency_penalty", C.c_double), ("repetition_window", C.c_size_t),
                ("max_new_tokens", C.c_size_t)]


class VisionConfigC(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("dim", C.c_int), ("n_head", C.c_int), ("d_head", C.c_int), ("n_ff", C.c_int),
                ("patch", C.c_int), ("merge", C.c_int), ("image_size", C.c_int), ("proj_dim", C.c_int),
                ("eps", C.c_float), ("rope_theta", C.c_float), ("mean", C.c_float * 3), ("std", C.c_float * 3)]


class VisionLayerC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("ln1", "ln2", "q", "k", "v", "o", "gate", "up", "down")]


FATAL_HOOK = C.CFUNCTYPE(None, C.c_char_p, C.c_char_p, C.c_void_p)
TOKEN_CB = C.CFUNCTYPE(C.c_int, C.c_int32, C.c_void_p)

_lib = None


def lib() -> C.CDLL:
    """The loaded libhtr.so (raises if it is not built: there is no other implementation)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HtrError(f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C historic-htr-ocr_amd)")
        l = C.CDLL(LIB_PATH)
        vp, sz, i32, f32 = C.c_void_p, C.c_size_t, C.c_int, C.c_float
        pp = C.POINTER(C.c_void_p)
        sig = {
            "htr_last_error": (C.c_char_p, []),
            "htr_device_open": (i32, [i32, pp]),
            "htr_device_close": (i32, [vp]),
            "htr_alive": (i32, [vp]),
            "htr_set_fatal_hook": (i32, [vp, FATAL_HOOK, vp]),
            "htr_debug_mark_lost": (i32, [vp, C.c_char_p]),
            "htr_sync": (i32, [vp]),
            "htr_device_set_compute": (i32, [vp, i32]),
            "htr_device_compute": (i32, [vp, C.POINTER(i32)]),
            "htr_device_info": (i32, [vp, C.c_char_p, sz, C.POINTER(i32)]),
            "htr_timer_begin": (i32, [vp]),
            "htr_timer_end": (i32, [vp, C.POINTER(f32)]),
            "htr_mem_live": (i32, [vp, C.POINTER(GpuBytes)]),
            "htr_alloc": (i32, [vp, sz, i32, pp]),
            "htr_free": (i32, [vp, vp]),
            "htr_upload": (i32, [vp, vp, vp, sz]),
            "htr_download": (i32, [vp, vp, vp, sz]),
            "htr_copy": (i32, [vp, vp, vp, sz]),
            "htr_debug_read": (i32, [vp, vp, sz, i32, i32, vp]),
            "htr_phase": (i32, [vp, C.c_char_p]),
            "htr_weight_q8_0": (i32, [vp, vp, sz, sz, pp]),
            "htr_weight_q8_0_f16": (i32, [vp, vp, sz, sz, f32, pp]),
            "htr_weight_free": (i32, [vp]),
            "htr_weight_shape": (i32, [vp, C.POINTER(sz), C.POINTER(sz)]),
            "htr_matvec_q8_0": (i32, [vp, vp, vp, vp, f32, vp, i32]),
            "htr_matvec_q8_0_many": (i32, [vp, C.POINTER(vp), sz, vp, vp]),
            "htr_matvec_qkv": (i32, [vp, vp, vp, vp, vp, vp, f32, vp]),
            "htr_matvec_ffn": (i32, [vp, vp, vp, vp, vp, f32, vp]),
            "htr_qkv_post": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, f32, vp, vp]),
            "htr_decode_attention": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, f32, vp]),
            "htr_decode_attention_static": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, f32, vp]),
            "htr_causal_attention": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, vp]),
            "htr_choose": (i32, [vp, vp, i32, vp, i32, i32, f32, f32, vp, vp, vp]),
            "htr_choose_many": (i32, [vp, vp, i32, i32, vp, i32, i32, i32, f32, vp]),
            "htr_matmul_q8_0": (i32, [vp, vp, sz, vp, vp, i32]),
            "htr_gemm_f16": (i32, [vp, vp, sz, vp, vp, i32]),
            "htr_gemm_ffn_f16": (i32, [vp, vp, sz, vp, vp, f32, vp]),
            "htr_vision_create": (i32, [vp, C.POINTER(VisionConfigC), vp, vp, C.POINTER(VisionLayerC), vp, vp, vp, vp,
                                        pp]),
            "htr_vision_free": (i32, [vp]),
            "htr_vision_get_config": (i32, [vp, C.POINTER(VisionConfigC)]),
            "htr_vision_load_gguf": (i32, [vp, vp, pp]),
            "htr_vision_out_shape": (i32, [vp, i32, i32, i32, C.POINTER(sz), C.POINTER(sz)]),
            "htr_vision_encode": (i32, [vp, vp, i32, i32, i32, vp]),
            "htr_gguf_open": (i32, [C.c_char_p, pp]),
            "htr_gguf_open_source": (i32, [C.c_uint64, READ_FN, vp, pp]),
            "htr_gguf_close": (i32, [vp]),
            "htr_gguf_header": (i32, [vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                      C.POINTER(sz)]),
            "htr_gguf_tensor": (i32, [vp, C.c_char_p, sz, C.POINTER(GgufTensorC)]),
            "htr_gguf_u32": (i32, [vp, C.c_char_p, C.POINTER(C.c_uint32)]),
            "htr_gguf_f32": (i32, [vp, C.c_char_p, C.POINTER(f32)]),
            "htr_gguf_str": (i32, [vp, C.c_char_p, C.c_char_p, sz, C.POINTER(sz)]),
            "htr_gguf_f32_array": (i32, [vp, C.c_char_p, vp, sz, C.POINTER(sz)]),
            "htr_gguf_read_small": (i32, [vp, C.c_char_p, vp, sz]),
            "htr_text_model_create": (i32, [vp, C.POINTER(TextConfigC), vp, vp, C.POINTER(LayerTensorsC), pp]),
            "htr_text_model_free": (i32, [vp]),
            "htr_text_model_load_gguf": (i32, [vp, vp, pp]),
            "htr_text_model_config": (i32, [vp, C.POINTER(TextConfigC)]),
            "htr_session_create": (i32, [vp, sz, pp]),
            "htr_session_create_grown": (i32, [vp, sz, sz, pp]),
            "htr_session_kv_rows": (i32, [vp, C.POINTER(C.c_size_t)]),
            "htr_session_free": (i32, [vp]),
            "htr_session_n_past": (i32, [vp, C.POINTER(sz)]),
            "htr_prefill": (i32, [vp, vp, sz, vp]),
            "htr_step": (i32, [vp, C.c_int32, vp]),
            "htr_session_logits": (i32, [vp, vp]),
            "htr_session_rewind": (i32, [vp, sz]),
            "htr_session_kv_cache": (i32, [vp, C.POINTER(KvViewC)]),
            "htr_session_profile_step": (i32, [vp, C.c_uint, i32, i32, C.POINTER(f32)]),
            "htr_session_set_fused_step": (i32, [vp, i32]),
            "htr_session_fused_step": (i32, [vp, C.POINTER(i32), C.POINTER(C.c_char_p)]),
            "htr_session_profile_fused_step": (i32, [vp, i32, C.POINTER(C.c_double), i32]),
            "htr_session_set_wait_limit": (i32, [vp, C.c_double]),
            "htr_debug_last_kernel": (i32, [vp, C.c_char_p, sz]),
            "htr_debug_handover": (i32, [vp, i32, i32, i32, i32, i32, i32, i32, C.POINTER(C.c_double), C.POINTER(i32)]),
            "htr_capture_begin": (i32, [vp]),
            "htr_capture_end": (i32, [vp, pp]),
            "htr_graph_launch": (i32, [vp]),
            "htr_graph_free": (i32, [vp]),
            "htr_choice_create": (i32, [vp, C.POINTER(PresetC), vp, sz, sz, sz, pp]),
            "htr_choice_free": (i32, [vp]),
            "htr_decode_gpu": (i32, [vp, vp, sz, TOKEN_CB, vp]),
            "htr_synth_q8_0": (i32, [C.c_uint64, sz, sz, vp]),
            "htr_synth_normal": (i32, [C.c_uint64, sz, f32, f32, vp]),
            "htr_choose_host": (i32, [vp, sz, C.POINTER(PresetC), vp, sz, vp, vp, sz, C.POINTER(C.c_uint64),
                                      C.POINTER(C.c_int32)]),
            "htr_generate": (i32, [vp, C.POINTER(PresetC), C.c_uint64, vp, sz, TOKEN_CB, vp, C.POINTER(sz)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _check(rc: int) -> None:
    if rc < 0:
        raise HtrError(lib().htr_last_error().decode(errors="replace"))


def last_error() -> str:
    return lib().htr_last_error().decode(errors="replace")


def _ptr(a: np.ndarray) -> int:
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data


# ---- synthetic inputs ----------------------------------------------------------------------------------------------

def synth_q8_0(seed: int, rows: int, cols: int) -> np.ndarray:
    """GGUF q8_0 block bytes [rows·cols/32·34]: quants uniform in [−127, 127], d = f16(|N(0,1)|·0.002)."""
    out = np.empty(rows * cols // 32 * 34, dtype=np.uint8)
    _check(lib().htr_synth_q8_0(seed, rows, cols, _ptr(out)))
    return out


def synth_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _check(lib().htr_synth_normal(seed, n, mean, std, _ptr(out)))
    return out


# ---- device and memory ---------------------------------------------------------------------------------------------

class Buffer:
    """Device memory (gpu.rs Buf): ``ptr`` is the device address."""

    def __init__(self, dev: "Device", nbytes: int, kind: int = MEM_WORK):
        self.dev, self.nbytes = dev, nbytes
        p = C.c_void_p()
        _check(lib().htr_alloc(dev.h, nbytes, kind, C.byref(p)))
        self.ptr = p.value

    def upload(self, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError(f"{a.nbytes} bytes into a {self.nbytes}-byte buffer")
        _check(lib().htr_upload(self.dev.h, self.ptr, _ptr(a), a.nbytes))
        return self

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        _check(lib().htr_download(self.dev.h, _ptr(out), self.ptr, out.nbytes))
        return out

    def copy_from(self, src: "Buffer", nbytes: int | None = None) -> "Buffer":
        """device → device copy (gpu.rs Batch::copy)"""
        n = min(self.nbytes, src.nbytes) if nbytes is None else nbytes
        _check(lib().htr_copy(self.dev.h, self.ptr, src.ptr, n))
        return self

    def read_through(self, sink: "Buffer", nontemporal: bool = True, kb_per_workgroup: int = 16) -> "Buffer":
        """the whole buffer read on the device and nothing else (htr_debug_read: the read rate of a streaming kernel;
        at most one u32 of `sink` is written)"""
        _check(lib().htr_debug_read(self.dev.h, self.ptr, self.nbytes - self.nbytes % 16, 1 if nontemporal else 0,
                                    kb_per_workgroup, sink.ptr))
        return self

    def free(self) -> None:
        if self.ptr:
            _check(lib().htr_free(self.dev.h, self.ptr))
            self.ptr = None


class Device:
    """One GPU (gpu.rs Gpu): the stream, the ledger, the sticky health."""

    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        _check(lib().htr_device_open(ordinal, C.byref(h)))
        self.h = h.value
        self._hook = None

    def close(self) -> None:
        if self.h:
            lib().htr_device_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def alive(self) -> None:
        _check(lib().htr_alive(self.h))

    def sync(self) -> None:
        _check(lib().htr_sync(self.h))

    @property
    def compute(self) -> int:
        """the compute path (COMPUTE_F16 by default, as the reference picks on a device with matrix units;
        OCR_WGPU_COMPUTE=f32 at open or a set forces COMPUTE_F32); models keep the path of their creation"""
        c = C.c_int()
        _check(lib().htr_device_compute(self.h, C.byref(c)))
        return c.value

    @compute.setter
    def compute(self, value: int) -> None:
        _check(lib().htr_device_set_compute(self.h, int(value)))

    def info(self) -> tuple[str, int]:
        name = C.create_string_buffer(256)
        n_cu = C.c_int()
        _check(lib().htr_device_info(self.h, name, 256, C.byref(n_cu)))
        return name.value.decode(), n_cu.value

    def timer_begin(self) -> None:
        _check(lib().htr_timer_begin(self.h))

    def timer_end(self) -> float:
        """milliseconds since timer_begin, by HIP events on the library's stream"""
        ms = C.c_float()
        _check(lib().htr_timer_end(self.h, C.byref(ms)))
        return ms.value

    def mem_live(self) -> dict:
        b = GpuBytes()
        _check(lib().htr_mem_live(self.h, C.byref(b)))
        return {"weights": b.weights, "kv_cache": b.kv_cache, "work": b.work, "readback": b.readback}

    def set_fatal_hook(self, fn) -> None:
        self._hook = FATAL_HOOK(lambda k, m, u: fn(k.decode(), m.decode()))
        _check(lib().htr_set_fatal_hook(self.h, self._hook, None))

    def mark_lost(self, why: str = "") -> None:
        _check(lib().htr_debug_mark_lost(self.h, why.encode()))

    def phase(self, name: str) -> None:
        """Gpu::phase: the label of the following work (a roctx range; "-" ends it)"""
        _check(lib().htr_phase(self.h, name.encode()))

    def last_kernel(self) -> str:
        """the instance name of the last kernel this device launched (e.g. 'k_dmv_full<4,1,qkv>')"""
        buf = C.create_string_buffer(96)
        _check(lib().htr_debug_last_kernel(self.h, buf, 96))
        return buf.value.decode()

    def handover(self, kind: int, a: int = 0, b: int = 8, words: int = 1024, pause: int = 16, iters: int = 1000,
                 max_polls: int = 1 << 20) -> tuple[float, bool]:
        """tagged words handed between the workgroups of one 256-workgroup launch (htr_debug_handover): kind 0 / 1, a
        word back and forth between workgroups a and b stored at workgroup / agent scope; kind 2, an all-to-all of
        `words` words with the first poll `pause` × 64 clocks after a workgroup's own. (µs a round trip or an
        exchange, whether every wait saw its word)"""
        us, seen = C.c_double(), C.c_int32()
        _check(lib().htr_debug_handover(self.h, kind, a, b, words, pause, iters, max_polls, C.byref(us), C.byref(seen)))
        return us.value, bool(seen.value)

    def capture_begin(self) -> None:
        _check(lib().htr_capture_begin(self.h))

    def capture_end(self) -> "Graph":
        g = C.c_void_p()
        _check(lib().htr_capture_end(self.h, C.byref(g)))
        return Graph(self, g.value)

    def alloc(self, nbytes: int, kind: int = MEM_WORK) -> Buffer:
        return Buffer(self, nbytes, kind)

    def upload(self, a: np.ndarray, kind: int = MEM_WORK) -> Buffer:
        a = np.ascontiguousarray(a)
        return Buffer(self, max(a.nbytes, 4), kind).upload(a)


class Graph:
    """a recorded HIP graph of the device's stream (Device.capture_begin … capture_end), replayed by launch()"""

    def __init__(self, dev: "Device", h: int):
        self.dev, self.h = dev, h

    def launch(self) -> None:
        _check(lib().htr_graph_launch(self.h))

    def free(self) -> None:
        if self.h:
            lib().htr_graph_free(self.h)
            self.h = None


class Weight:
    """A q8_0 weight [rows × cols] repacked on the device (or dequantised to f16 with ``f16=True``)."""

    def __init__(self, dev: Device, blocks: np.ndarray, rows: int, cols: int, f16: bool = False, scale: float = 1.0):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        if blocks.size != rows * cols // 32 * 34:
            raise ValueError(f"{blocks.size} bytes for a [{rows} x {cols}] q8_0 tensor")
        h = C.c_void_p()
        if f16:
            _check(lib().htr_weight_q8_0_f16(dev.h, _ptr(blocks), rows, cols, scale, C.byref(h)))
        else:
            _check(lib().htr_weight_q8_0(dev.h, _ptr(blocks), rows, cols, C.byref(h)))
        self.dev, self.h, self.rows, self.cols = dev, h.value, rows, cols

    def free(self) -> None:
        if self.h:
            lib().htr_weight_free(self.h)
            self.h = None


# ---- kernels on device buffers -------------------------------------------------------------------------------------

def _p(b) -> int | None:
    return None if b is None else b.ptr


def matvec_q8_0(dev: Device, w: Weight, x: Buffer, y: Buffer, norm_w: Buffer | None = None, eps: float = 1e-6,
                acc: bool = False) -> None:
    _check(lib().htr_matvec_q8_0(dev.h, w.h, x.ptr, _p(norm_w), eps, y.ptr, int(acc)))


def matvec_q8_0_many(dev: Device, ws: list[Weight], x: Buffer, y: Buffer) -> None:
    arr = (C.c_void_p * len(ws))(*[w.h for w in ws])
    _check(lib().htr_matvec_q8_0_many(dev.h, arr, len(ws), x.ptr, y.ptr))


def matvec_qkv(dev: Device, wq: Weight, wk: Weight, wv: Weight, x: Buffer, norm_w: Buffer, eps: float,
               qkv: Buffer) -> None:
    _check(lib().htr_matvec_qkv(dev.h, wq.h, wk.h, wv.h, x.ptr, norm_w.ptr, eps, qkv.ptr))


def matvec_ffn(dev: Device, wg: Weight, wu: Weight, x: Buffer, norm_w: Buffer, eps: float, g: Buffer) -> None:
    _check(lib().htr_matvec_ffn(dev.h, wg.h, wu.h, x.ptr, norm_w.ptr, eps, g.ptr))


def qkv_post(dev: Device, qkv: Buffer, q_norm: Buffer, k_norm: Buffer, rope: Buffer, n_head: int, n_kv: int, pos: int,
             n_ctx: int, eps: float, kc: Buffer, vc: Buffer) -> None:
    _check(lib().htr_qkv_post(dev.h, qkv.ptr, q_norm.ptr, k_norm.ptr, rope.ptr, n_head, n_kv, pos, n_ctx, eps, kc.ptr,
                              vc.ptr))


def decode_attention(dev: Device, q: Buffer, kc: Buffer, vc: Buffer, n_head: int, n_kv: int, n_ctx: int, n_keys: int,
                     scale: float, out: Buffer) -> None:
    _check(lib().htr_decode_attention(dev.h, q.ptr, kc.ptr, vc.ptr, n_head, n_kv, n_ctx, n_keys, scale, out.ptr))


def causal_attention(dev: Device, q: Buffer, kc: Buffer, vc: Buffer, n_q: int, pos0: int, n_head: int, n_kv: int,
                     n_ctx: int, scale: float, out: Buffer) -> None:
    _check(lib().htr_causal_attention(dev.h, q.ptr, kc.ptr, vc.ptr, n_q, pos0, n_head, n_kv, n_ctx, scale, out.ptr))


def choose(dev: Device, logits: Buffer, n_vocab: int, hist: Buffer, length: int, window: int, rp: float, tok: Buffer,
           fp: float = 0.0, counts: Buffer | None = None, fpen: Buffer | None = None) -> None:
    _check(lib().htr_choose(dev.h, logits.ptr, n_vocab, hist.ptr, length, window, rp, fp, _p(counts), _p(fpen),
                            tok.ptr))


def choose_many(dev: Device, logits: Buffer, n_vocab: int, n: int, hist: Buffer, hist_stride: int, length: int,
                window: int, rp: float, tok: Buffer) -> None:
    _check(lib().htr_choose_many(dev.h, logits.ptr, n_vocab, n, hist.ptr, hist_stride, length, window, rp, tok.ptr))


def matmul_q8_0(dev: Device, x: Buffer, m: int, w: Weight, y: Buffer, acc: bool = False) -> None:
    """y[m][N] (+)= x·Wᵀ (x f32 [m][K], w q8_0) on the device's compute path: F32 exact, F16 operands rounded to f16"""
    _check(lib().htr_matmul_q8_0(dev.h, x.ptr, m, w.h, y.ptr, int(acc)))


def choose_host(logits: np.ndarray, preset: Preset, history, counts: dict | None, rng_state: list) -> int:
    """sampling.rs:38-89 choose on host logits (penalised IN PLACE); rng_state is a one-element list holding the
    SplitMix64 state, advanced when the preset samples"""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    hist = np.ascontiguousarray(history, dtype=np.int32)
    counts = counts or {}
    ct = np.array(list(counts.keys()), dtype=np.int32)
    cn = np.array(list(counts.values()), dtype=np.uint32)
    st = C.c_uint64(rng_state[0])
    out = C.c_int32()
    p = preset.c()
    _check(lib().htr_choose_host(_ptr(logits), logits.size, C.byref(p), _ptr(hist) if hist.size else None, hist.size,
                                 _ptr(ct) if ct.size else None, _ptr(cn) if cn.size else None, ct.size, C.byref(st),
                                 C.byref(out)))
    rng_state[0] = st.value
    return out.value


def gemm_f16(dev: Device, x16: Buffer, m: int, w: Weight, y: Buffer, acc: bool = False) -> None:
    """y[m][N] (+)= x16·Wᵀ on the matrix cores (x16: f16 [m][K]; w: an f16 weight)"""
    _check(lib().htr_gemm_f16(dev.h, x16.ptr, m, w.h, y.ptr, int(acc)))


def gemm_ffn_f16(dev: Device, x16: Buffer, m: int, w_gate: Weight, w_up: Weight, scale: float, g16: Buffer) -> None:
    """g16[m][N] = f16(silu(x16·Wgᵀ)·(x16·Wuᵀ)·scale)"""
    _check(lib().htr_gemm_ffn_f16(dev.h, x16.ptr, m, w_gate.h, w_up.h, scale, g16.ptr))


# ---- the text decoder ----------------------------------------------------------------------------------------------

@dataclass
class TextConfig:
    """text.rs:30-42 TextConfig."""
    n_layer: int
    dim: int
    n_head: int
    n_kv: int
    d_head: int
    n_ff: int
    n_vocab: int
    n_ctx_train: int = 0
    eps: float = 1e-6
    rope_base: float = 1e6

    def c(self) -> TextConfigC:
        return TextConfigC(self.n_layer, self.dim, self.n_head, self.n_kv, self.d_head, self.n_ff, self.n_vocab,
                           self.n_ctx_train, self.eps, self.rope_base)


def seed_for_stem(stem: str) -> int:
    """presets.rs:114-117 seed_for_stem: a page's sampled-read seed, the first 4 bytes of md5(stem) big-endian (the
    presets' seedRule int(md5(stem).hexdigest()[:8], 16)); it is the seed Session.generate takes"""
    import hashlib

    return int.from_bytes(hashlib.md5(stem.encode()).digest()[:4], "big")


@dataclass
class Preset:
    """ocr-decode presets.rs:17-29 (the fields the token choice reads)."""
    repetition_penalty: float = 1.1
    repetition_window: int = 64
    frequency_penalty: float = 0.0
    max_new_tokens: int = 512
    temperature: float = 0.0
    top_p: float = 1.0

    def c(self) -> PresetC:
        return PresetC(self.temperature, self.top_p, self.repetition_penalty, self.frequency_penalty,
                       self.repetition_window, self.max_new_tokens)


GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


class Gguf:
    """ocr-gguf Gguf (lib.rs:1-401): the parsed header of a GGUF file (or of bytes in memory, read through the
    TensorSource callback); the tensors' bytes are read on demand."""

    def __init__(self, path=None, data: bytes | None = None):
        h = C.c_void_p()
        if data is not None:
            self._data = bytes(data)

            def read(_user, off, buf, n):
                if off + n > len(self._data):
                    return 1
                C.memmove(buf, self._data[off:off + n], n)
                return 0

            self._read = READ_FN(read)
            _check(lib().htr_gguf_open_source(len(self._data), self._read, None, C.byref(h)))
        else:
            _check(lib().htr_gguf_open(str(path).encode(), C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().htr_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def header(self) -> dict:
        v, al, off, n = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_size_t()
        _check(lib().htr_gguf_header(self.h, C.byref(v), C.byref(al), C.byref(off), C.byref(n)))
        return {"version": v.value, "alignment": al.value, "data_offset": off.value, "n_tensors": n.value}

    def info(self, name: str | None = None, index: int = 0) -> dict:
        t = GgufTensorC()
        _check(lib().htr_gguf_tensor(self.h, None if name is None else name.encode(), index, C.byref(t)))
        return {"name": t.name.decode(), "type": t.type, "shape": list(t.shape[: t.n_dims]), "n_bytes": t.n_bytes,
                "offset": t.offset, "file_offset": t.file_offset}

    def u32(self, key: str) -> int:
        v = C.c_uint32()
        _check(lib().htr_gguf_u32(self.h, key.encode(), C.byref(v)))
        return v.value

    def f32(self, key: str) -> float:
        v = C.c_float()
        _check(lib().htr_gguf_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def str(self, key: str) -> str:
        n = C.c_size_t()
        _check(lib().htr_gguf_str(self.h, key.encode(), None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        _check(lib().htr_gguf_str(self.h, key.encode(), buf, n.value + 1, None))
        return buf.raw[: n.value].decode()

    def f32_array(self, key: str) -> np.ndarray:
        n = C.c_size_t()
        _check(lib().htr_gguf_f32_array(self.h, key.encode(), None, 0, C.byref(n)))
        out = np.empty(n.value, np.float32)
        _check(lib().htr_gguf_f32_array(self.h, key.encode(), _ptr(out), n.value, None))
        return out

    def read_small(self, name: str) -> np.ndarray:
        nb = self.info(name)["n_bytes"]
        out = np.empty(nb, np.uint8)
        _check(lib().htr_gguf_read_small(self.h, name.encode(), _ptr(out), nb))
        return out


class TextModel:
    """TextModel::load (text.rs:332-375) from host tensors: ``layers`` is a list of dicts with the q8_0 block bytes
    (q, k, v, o, gate, up, down) and f32 norms (attn_norm, q_norm, k_norm, ffn_norm). ``TextModel.from_gguf`` loads
    one from a GGUF file instead."""

    @classmethod
    def from_gguf(cls, dev: Device, g: Gguf) -> "TextModel":
        self = cls.__new__(cls)
        h = C.c_void_p()
        _check(lib().htr_text_model_load_gguf(dev.h, g.h, C.byref(h)))
        self.dev, self.h = dev, h.value
        c = TextConfigC()
        _check(lib().htr_text_model_config(self.h, C.byref(c)))
        self.cfg = TextConfig(c.n_layer, c.dim, c.n_head, c.n_kv, c.d_head, c.n_ff, c.n_vocab, c.n_ctx_train, c.eps,
                              c.rope_base)
        return self

    def __init__(self, dev: Device, cfg: TextConfig, tok_embd: np.ndarray, output_norm: np.ndarray,
                 layers: list[dict]):
        self.dev, self.cfg = dev, cfg
        keep = []
        arr = (LayerTensorsC * cfg.n_layer)()
        for i, ly in enumerate(layers):
            vals = {}
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                a = np.ascontiguousarray(ly[name], dtype=np.uint8)
                keep.append(a)
                vals[name] = _ptr(a)
            for name in ("attn_norm", "q_norm", "k_norm", "ffn_norm"):
                a = np.ascontiguousarray(ly[name], dtype=np.float32)
                keep.append(a)
                vals[name] = _ptr(a)
            arr[i] = LayerTensorsC(**vals)
        te = np.ascontiguousarray(tok_embd, dtype=np.uint8)
        on = np.ascontiguousarray(output_norm, dtype=np.float32)
        h = C.c_void_p()
        cfg_c = cfg.c()
        _check(lib().htr_text_model_create(dev.h, C.byref(cfg_c), _ptr(te), _ptr(on), arr, C.byref(h)))
        self.h = h.value

    def free(self) -> None:
        if self.h:
            lib().htr_text_model_free(self.h)
            self.h = None

    def session(self, n_ctx: int, kv_grow: int | None = None) -> "Session":
        """a session for n_ctx positions: its KV cache sized to n_ctx at once, or (kv_grow) grown with the read"""
        return Session(self, n_ctx, kv_grow)


class Session:
    """text.rs Session: the KV cache for n_ctx positions (allocated at once, or grown by kv_grow rows past the need:
    Session::reserve) and the decode step's buffers."""

    def __init__(self, m: TextModel, n_ctx: int, kv_grow: int | None = None):
        h = C.c_void_p()
        if kv_grow is None:
            _check(lib().htr_session_create(m.h, n_ctx, C.byref(h)))
        else:
            _check(lib().htr_session_create_grown(m.h, n_ctx, kv_grow, C.byref(h)))
        self.m, self.h, self.n_ctx = m, h.value, n_ctx

    @property
    def reserved_rows(self) -> int:
        """the KV cache rows allocated now (Session::kv_rows)"""
        v = C.c_size_t()
        _check(lib().htr_session_kv_rows(self.h, C.byref(v)))
        return v.value

    def free(self) -> None:
        if self.h:
            lib().htr_session_free(self.h)
            self.h = None

    @property
    def n_past(self) -> int:
        v = C.c_size_t()
        _check(lib().htr_session_n_past(self.h, C.byref(v)))
        return v.value

    def prefill(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.m.cfg.n_vocab, dtype=np.float32)
        _check(lib().htr_prefill(self.h, _ptr(ids), ids.size, _ptr(out)))
        return out

    def step(self, tok: int) -> np.ndarray:
        out = np.empty(self.m.cfg.n_vocab, dtype=np.float32)
        _check(lib().htr_step(self.h, int(tok), _ptr(out)))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty(self.m.cfg.n_vocab, dtype=np.float32)
        _check(lib().htr_session_logits(self.h, _ptr(out)))
        return out

    def rewind(self, n_past: int) -> None:
        _check(lib().htr_session_rewind(self.h, n_past))

    def profile_step(self, classes: int, n_steps: int = 16, reps: int = 20) -> float:
        """milliseconds per decode step of the kernels of `classes` (STEP_* bits) alone, in a graph, at n_past"""
        ms = C.c_float()
        _check(lib().htr_session_profile_step(self.h, classes, n_steps, reps, C.byref(ms)))
        return ms.value

    @property
    def fused_step(self) -> bool:
        """whether the decode step runs as one launch per token (the 1024 / 2048 / 3072 decoder on the f16 paths)"""
        on, why = C.c_int(), C.c_char_p()
        _check(lib().htr_session_fused_step(self.h, C.byref(on), C.byref(why)))
        return bool(on.value)

    @fused_step.setter
    def fused_step(self, on: bool) -> None:
        _check(lib().htr_session_set_fused_step(self.h, 1 if on else 0))

    def fused_step_unavailable(self) -> str | None:
        """why the one-launch step is not available to this session (None when it is)"""
        on, why = C.c_int(), C.c_char_p()
        _check(lib().htr_session_fused_step(self.h, C.byref(on), C.byref(why)))
        return why.value.decode() if why.value else None

    def set_wait_limit(self, us: float | None) -> None:
        """the one-launch step's bound on each of its waits, in µs (None: the default 0.2 s): the launches recorded
        from now on carry it (tests of the error path make every wait run out from the host)"""
        _check(lib().htr_session_set_wait_limit(self.h, float(us) if us else 0.0))

    def profile_fused_step(self, tok: int) -> np.ndarray:
        """one one-launch step of `tok` at n_past (not advanced): workgroup 0's stamps in µs after the embed,
        [1 + 12·n_layer + 3] (per layer: each phase's input taken and output written — qkv, attention, merge, o,
        ffn, down; then the LM head's input taken, its rows done, the end)"""
        n = 1 + 12 * self.m.cfg.n_layer + 3
        us = np.zeros(n, np.float64)
        _check(lib().htr_session_profile_fused_step(self.h, int(tok), us.ctypes.data_as(C.POINTER(C.c_double)), n))
        return us

    def kv_view(self) -> KvViewC:
        v = KvViewC()
        _check(lib().htr_session_kv_cache(self.h, C.byref(v)))
        return v

    def kv_rows(self, layer: int, pos0: int, n: int) -> tuple[np.ndarray, np.ndarray]:
        """cache rows [pos0, pos0 + n) of a layer as f16 bits in the reference's layout [n][n_kv·128] (K, V)"""
        v = self.kv_view()
        out = []
        for base in (v.d_k, v.d_v):
            a = np.empty((v.n_kv, n, v.d_head), np.uint16)
            for h in range(v.n_kv):
                off = 2 * (layer * v.layer_stride + (h * v.n_ctx + pos0) * v.d_head)
                _check(lib().htr_download(self.m.dev.h, _ptr(a[h]), base + off, n * v.d_head * 2))
            out.append(np.ascontiguousarray(a.transpose(1, 0, 2).reshape(n, v.n_kv * v.d_head)))
        return out[0], out[1]

    def set_kv_rows(self, layer: int, pos0: int, k: np.ndarray, v_rows: np.ndarray) -> None:
        """write cache rows [pos0, pos0 + n) of a layer from f16 bits [n][n_kv·128] (tests that plant rows)"""
        v = self.kv_view()
        n = k.shape[0]
        for base, rows in ((v.d_k, k), (v.d_v, v_rows)):
            a = np.ascontiguousarray(np.asarray(rows, np.uint16).reshape(n, v.n_kv, v.d_head).transpose(1, 0, 2))
            for h in range(v.n_kv):
                off = 2 * (layer * v.layer_stride + (h * v.n_ctx + pos0) * v.d_head)
                _check(lib().htr_upload(self.m.dev.h, base + off, _ptr(a[h]), n * v.d_head * 2))

    def choice(self, preset: Preset, history, chunk: int = 4, depth: int = 2) -> "Choice":
        return Choice(self, preset, history, chunk, depth)

    def decode_gpu(self, ch: "Choice", max_tokens: int, on_token=None) -> list[int]:
        toks: list[int] = []

        def cb(t, _u):
            toks.append(int(t))
            return 1 if on_token is None else int(bool(on_token(int(t))))

        fn = TOKEN_CB(cb)
        _check(lib().htr_decode_gpu(self.h, ch.h, max_tokens, fn, None))
        return toks

    def generate(self, preset: Preset, seed: int, history, on_token=None) -> list[int]:
        """sampling.rs:252-278 generate: the CPU-choice read (any preset, sampled ones included), each token stepped
        on the device; on_token returning False ends the read before the token is stepped"""
        toks: list[int] = []

        def cb(t, _u):
            toks.append(int(t))
            return 1 if on_token is None else int(bool(on_token(int(t))))

        fn = TOKEN_CB(cb)
        hist = np.ascontiguousarray(history, dtype=np.int32)
        p = preset.c()
        n = C.c_size_t()
        _check(lib().htr_generate(self.h, C.byref(p), seed, _ptr(hist) if hist.size else None, hist.size, fn, None,
                                  C.byref(n)))
        assert n.value == len(toks)
        return toks


class Choice:
    """text.rs Choice::new: the GPU token choice of a greedy preset."""

    def __init__(self, s: Session, preset: Preset, history, chunk: int = 4, depth: int = 2):
        hist = np.ascontiguousarray(history, dtype=np.int32)
        h = C.c_void_p()
        p = preset.c()
        _check(lib().htr_choice_create(s.h, C.byref(p), _ptr(hist) if hist.size else None, hist.size, chunk, depth,
                                       C.byref(h)))
        self.s, self.h = s, h.value

    def free(self) -> None:
        if self.h:
            lib().htr_choice_free(self.h)
            self.h = None


# ---- the vision encoder --------------------------------------------------------------------------------------------

class Vision:
    """Vision::from_gguf (vision.rs:177-233) from host tensors. ``cfg``: n_layer, dim, n_head, n_ff, patch,
    image_size, proj_dim, eps, rope_theta, mean, std; ``t``: patch_embd (f32), pre_ln, input_norm (f32), merger, mm1,
    mm2 (q8_0 blocks) and ``layers`` (dicts with ln1, ln2 f32 and q, k, v, o, gate, up, down q8_0 blocks).
    ``Vision.from_gguf`` loads one from an mmproj GGUF (BF16 / F32 weights) instead."""

    @classmethod
    def from_gguf(cls, dev: Device, g: Gguf) -> "Vision":
        self = cls.__new__(cls)
        h = C.c_void_p()
        _check(lib().htr_vision_load_gguf(dev.h, g.h, C.byref(h)))
        self.dev, self.h = dev, h.value
        c = VisionConfigC()
        _check(lib().htr_vision_get_config(self.h, C.byref(c)))
        self.cfg = dict(n_layer=c.n_layer, dim=c.dim, n_head=c.n_head, n_ff=c.n_ff, patch=c.patch, merge=c.merge,
                        image_size=c.image_size, proj_dim=c.proj_dim, eps=c.eps, rope_theta=c.rope_theta,
                        mean=list(c.mean), std=list(c.std))
        return self

    def __init__(self, dev: Device, cfg: dict, t: dict):
        self.dev, self.cfg = dev, cfg
        keep = []

        def f32(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            keep.append(a)
            return _ptr(a)

        def u8(a):
            a = np.ascontiguousarray(a, dtype=np.uint8)
            keep.append(a)
            return _ptr(a)

        arr = (VisionLayerC * cfg["n_layer"])()
        for i, ly in enumerate(t["layers"]):
            arr[i] = VisionLayerC(ln1=f32(ly["ln1"]), ln2=f32(ly["ln2"]),
                                  **{k: u8(ly[k]) for k in ("q", "k", "v", "o", "gate", "up", "down")})
        c = VisionConfigC(cfg["n_layer"], cfg["dim"], cfg["n_head"], 64, cfg["n_ff"], cfg["patch"], 2,
                          cfg.get("image_size", 1540), cfg["proj_dim"], cfg["eps"], cfg["rope_theta"],
                          (C.c_float * 3)(*cfg["mean"]), (C.c_float * 3)(*cfg["std"]))
        h = C.c_void_p()
        _check(lib().htr_vision_create(dev.h, C.byref(c), f32(t["patch_embd"]), f32(t["pre_ln"]), arr,
                                       f32(t["input_norm"]), u8(t["merger"]), u8(t["mm1"]), u8(t["mm2"]), C.byref(h)))
        self.h = h.value

    def free(self) -> None:
        if self.h:
            lib().htr_vision_free(self.h)
            self.h = None

    def out_shape(self, width: int, height: int, n_layers: int = -1) -> tuple[int, int]:
        n, d = C.c_size_t(), C.c_size_t()
        _check(lib().htr_vision_out_shape(self.h, width, height, n_layers, C.byref(n), C.byref(d)))
        return n.value, d.value

    def encode_gpu(self, rgb: np.ndarray, n_layers: int = -1, out: Buffer | None = None) -> tuple[Buffer, int, int]:
        """Vision::encode_gpu: the result left on the device → (buffer, rows, width)"""
        rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
        h, w, _ = rgb.shape
        n, d = self.out_shape(w, h, n_layers)
        out = out or self.dev.alloc(n * d * 4)
        _check(lib().htr_vision_encode(self.h, _ptr(rgb), w, h, n_layers, out.ptr))
        return out, n, d

    def encode(self, rgb: np.ndarray, n_layers: int = -1) -> np.ndarray:
        """Vision::encode: the embeddings [n/4][proj_dim] (or the residual [n][dim] after n_layers layers)"""
        buf, n, d = self.encode_gpu(rgb, n_layers)
        out = buf.download(np.float32, n * d).reshape(n, d)
        buf.free()
        return out
