"""A GGUF v3 writer for the tests: ggml's gguf.cpp layout (the same the reader restates, ocr-gguf lib.rs:1-401).

header = magic "GGUF", u32 version, u64 tensor count, u64 KV count; KVs = key (u64 length + bytes), u32 value type,
value; tensor infos = name, u32 n_dims, u64 dims (ggml order: dims[0] contiguous), u32 ggml type, u64 offset; the data
section starts at the header's end rounded up to the alignment, each tensor at an aligned offset, zero padding
between tensors (none after the last). Written here from the format description, and pinned against the reference test's hand-built bytes
(lib.rs:498-548) by tests/test_gguf.py."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}


def _s(v: str) -> bytes:
    b = v.encode()
    return struct.pack("<Q", len(b)) + b


def _value(ty: int, v) -> bytes:
    if ty == STR:
        return _s(v)
    if ty == ARR:
        ety, items = v
        return struct.pack("<IQ", ety, len(items)) + b"".join(_value(ety, x) for x in items)
    return struct.pack(_SCALAR[ty], v)


def gguf_bytes(kvs, tensors, alignment=None, version=3) -> bytes:
    """kvs: [(key, type, value)] (arrays: (ARR, (element type, [values]))); tensors: [(name, ggml type, dims, data
    bytes)] in file order; alignment: written as general.alignment (u32) when given, else the default 32"""
    al = 32 if alignment is None else alignment
    kvs = list(kvs) + ([("general.alignment", U32, alignment)] if alignment is not None else [])
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for key, ty, v in kvs:
        out += _s(key) + struct.pack("<I", ty) + _value(ty, v)
    off = 0
    offsets = []
    for name, ty, dims, data in tensors:
        offsets.append(off)
        out += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, off)
        off = (off + len(data) + al - 1) // al * al
    while len(out) % al:
        out.append(0)
    for k, ((name, ty, dims, data), o) in enumerate(zip(tensors, offsets)):
        out += bytes(data)
        while k + 1 < len(tensors) and len(out) % al:  # padding between tensors, none after the last
            out.append(0)
    return bytes(out)


def text_model_gguf(cfg: dict, tok_embd, output_norm, layers, extra_kvs=(), extra_tensors=(), skip=()) -> bytes:
    """a qwen3 text GGUF of the test models (q8_0 projections and token_embd, f32 norms) with the metadata keys
    TextConfig::from_gguf reads (text.rs:43-76); ``skip``: tensor names left out (before ``extra_tensors`` are added, so
    one can be replaced), ``extra_*``: added"""
    d, qd, kvd, f = cfg["dim"], cfg["n_head"] * 128, cfg["n_kv"] * 128, cfg["n_ff"]
    kvs = [("general.architecture", STR, "qwen3"), ("qwen3.block_count", U32, cfg["n_layer"]),
           ("qwen3.context_length", U32, cfg.get("n_ctx_train", 4096)), ("qwen3.embedding_length", U32, d),
           ("qwen3.feed_forward_length", U32, f), ("qwen3.attention.head_count", U32, cfg["n_head"]),
           ("qwen3.attention.head_count_kv", U32, cfg["n_kv"]), ("qwen3.attention.key_length", U32, 128),
           ("qwen3.attention.value_length", U32, 128),
           ("qwen3.attention.layer_norm_rms_epsilon", F32, cfg.get("eps", 1e-6)),
           ("qwen3.rope.freq_base", F32, cfg.get("rope_base", 1e6))]
    kvs += list(extra_kvs)
    q8 = lambda a: np.ascontiguousarray(a, np.uint8).tobytes()
    f32 = lambda a: np.ascontiguousarray(a, np.float32).tobytes()
    ts = [("token_embd.weight", GGML_Q8_0, [d, cfg["n_vocab"]], q8(tok_embd))]
    for i, ly in enumerate(layers):
        p = f"blk.{i}."
        ts += [(p + "attn_norm.weight", GGML_F32, [d], f32(ly["attn_norm"])),
               (p + "attn_q.weight", GGML_Q8_0, [d, qd], q8(ly["q"])),
               (p + "attn_k.weight", GGML_Q8_0, [d, kvd], q8(ly["k"])),
               (p + "attn_v.weight", GGML_Q8_0, [d, kvd], q8(ly["v"])),
               (p + "attn_output.weight", GGML_Q8_0, [qd, d], q8(ly["o"])),
               (p + "attn_q_norm.weight", GGML_F32, [128], f32(ly["q_norm"])),
               (p + "attn_k_norm.weight", GGML_F32, [128], f32(ly["k_norm"])),
               (p + "ffn_norm.weight", GGML_F32, [d], f32(ly["ffn_norm"])),
               (p + "ffn_gate.weight", GGML_Q8_0, [d, f], q8(ly["gate"])),
               (p + "ffn_up.weight", GGML_Q8_0, [d, f], q8(ly["up"])),
               (p + "ffn_down.weight", GGML_Q8_0, [f, d], q8(ly["down"]))]
    ts.append(("output_norm.weight", GGML_F32, [d], f32(output_norm)))
    ts = [t for t in ts if t[0] not in skip] + list(extra_tensors)
    return gguf_bytes(kvs, ts)


def bf16_bits(a) -> np.ndarray:
    """float32 values → bf16 bit patterns (round to nearest even)"""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(b) -> np.ndarray:
    """bf16 bit patterns → their float32 values (exact)"""
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def vision_model_gguf(cfg: dict, t: dict, kvs_over=None, extra_tensors=(), skip=()) -> bytes:
    """an mmproj GGUF of a LightOnOCR-shaped encoder with the clip.* keys VisionConfig::from_gguf reads
    (vision.rs:55-84). ``t`` as the host-array encoder takes it, but each weight a uint16 array (BF16 bits) or a
    float32 array (F32), [rows][cols]; norms float32. The patch embedding is written [p, p, 3, dim] as an mmproj holds
    it. ``kvs_over``: {key: (type, value)} replacing or adding keys (value None drops the key)"""
    d, f, pd, p = cfg["dim"], cfg["n_ff"], cfg["proj_dim"], cfg["patch"]
    kvs = {"general.architecture": (STR, "clip"), "clip.projector_type": (STR, "lightonocr"),
           "clip.use_silu": (BOOL, 1), "clip.vision.embedding_length": (U32, d),
           "clip.vision.attention.head_count": (U32, cfg["n_head"]), "clip.vision.block_count": (U32, cfg["n_layer"]),
           "clip.vision.feed_forward_length": (U32, f), "clip.vision.patch_size": (U32, p),
           "clip.vision.spatial_merge_size": (U32, 2), "clip.vision.image_size": (U32, cfg.get("image_size", 1540)),
           "clip.vision.projection_dim": (U32, pd),
           "clip.vision.attention.layer_norm_epsilon": (F32, cfg["eps"]),
           "clip.vision.image_mean": (ARR, (F32, list(cfg["mean"]))),
           "clip.vision.image_std": (ARR, (F32, list(cfg["std"])))}
    for k, v in (kvs_over or {}).items():
        if v is None:
            kvs.pop(k, None)
        else:
            kvs[k] = v

    def w(name, a, dims):
        a = np.ascontiguousarray(a)
        ty = GGML_BF16 if a.dtype == np.uint16 else GGML_F32
        assert a.dtype in (np.uint16, np.float32) and a.size == int(np.prod(dims)), name
        return (name, ty, dims, a.tobytes())

    vec = lambda name, a: (name, GGML_F32, [a.size], np.ascontiguousarray(a, np.float32).tobytes())
    ts = []
    for i, ly in enumerate(t["layers"]):
        b = f"v.blk.{i}."
        ts += [vec(b + "ln1.weight", ly["ln1"]), vec(b + "ln2.weight", ly["ln2"]),
               w(b + "attn_q.weight", ly["q"], [d, d]), w(b + "attn_k.weight", ly["k"], [d, d]),
               w(b + "attn_v.weight", ly["v"], [d, d]), w(b + "attn_out.weight", ly["o"], [d, d]),
               w(b + "ffn_gate.weight", ly["gate"], [d, f]), w(b + "ffn_up.weight", ly["up"], [d, f]),
               w(b + "ffn_down.weight", ly["down"], [f, d])]
    ts += [w("v.patch_embd.weight", t["patch_embd"], [p, p, 3, d]), vec("v.pre_ln.weight", t["pre_ln"]),
           vec("mm.input_norm.weight", t["input_norm"]), w("mm.patch_merger.weight", t["merger"], [4 * d, d]),
           w("mm.1.weight", t["mm1"], [d, pd]), w("mm.2.weight", t["mm2"], [pd, pd])]
    ts = [x for x in ts if x[0] not in skip] + list(extra_tensors)
    return gguf_bytes([(k, ty, v) for k, (ty, v) in kvs.items()], ts)
