"""The GGUF reader (ocr-gguf lib.rs:1-401) on the host: no GPU involved.

The reference's own test file (lib.rs:498-607) is rebuilt byte by byte here — three KVs (u32 a.n = 7, a string array,
an f32 array), an optional general.alignment, a bf16 [3, 2] tensor and a q8_0 [32] tensor (d = 0.5, quants −16 … 15)
— with its expectations: the values, the dequantised −8.0 / 7.5, an aligned data section; and its rejections (an
unknown ggml type, a truncated file, a wrong magic)."""
import struct

import numpy as np
import pytest

import htr
from gguf_writer import (ARR, F32, GGML_BF16, GGML_F32, GGML_Q8_0, STR, U32, bf16_bits, bf16_value, gguf_bytes,
                         text_model_gguf, vision_model_gguf)
from helpers import tiny_text_model


def _s(v: str) -> bytes:
    return struct.pack("<Q", len(v)) + v.encode()


def reference_tiny(alignment=None) -> bytes:
    """lib.rs:505-548 tiny(): the bytes in the order the reference test appends them"""
    b = bytearray(b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", 2) + struct.pack("<Q", 3 + (alignment is not None)))
    b += _s("a.n") + struct.pack("<I", 4) + struct.pack("<I", 7)
    b += _s("a.names") + struct.pack("<I", 9) + struct.pack("<I", 8) + struct.pack("<Q", 2) + _s("x") + _s("yz")
    b += _s("a.mean") + struct.pack("<I", 9) + struct.pack("<I", 6) + struct.pack("<Q", 3)
    b += struct.pack("<3f", 0.5, 0.25, -1.0)
    if alignment is not None:
        b += _s("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", alignment)
    al = alignment or 32
    b += _s("w") + struct.pack("<I", 2) + struct.pack("<QQ", 3, 2) + struct.pack("<I", 30) + struct.pack("<Q", 0)
    b += _s("q") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<I", 8) + struct.pack("<Q", al)
    while len(b) % al:
        b.append(0)
    b += np.array([1.0, -2.0, 0.5, 3.0, 0.0, 1.5], np.float32).view(np.uint32).__rshift__(16).astype("<u2").tobytes()
    while len(b) % al:
        b.append(0)
    b += np.float16(0.5).tobytes() + bytes((i - 16) & 0xFF for i in range(32))
    return bytes(b)


def bf16_to_f32(raw: np.ndarray) -> np.ndarray:
    return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("al", [None, 64])
def test_reference_tiny_file_parses(al):
    with htr.Gguf(data=reference_tiny(al)) as g:
        h = g.header()
        assert h["version"] == 3 and h["n_tensors"] == 2
        assert h["alignment"] == (al or 32) and h["data_offset"] % (al or 32) == 0
        assert g.u32("a.n") == 7
        assert list(g.f32_array("a.mean")) == [0.5, 0.25, -1.0]
        w = g.info("w")
        assert (w["shape"], w["type"]) == ([3, 2], GGML_BF16)
        assert list(bf16_to_f32(g.read_small("w"))) == [1.0, -2.0, 0.5, 3.0, 0.0, 1.5]
        q = g.info("q")
        assert (q["shape"], q["type"], q["n_bytes"]) == ([32], GGML_Q8_0, 34)
        raw = g.read_small("q")
        d = float(raw[:2].view(np.float16)[0])
        deq = raw[2:].view(np.int8).astype(np.float32) * d
        assert (deq[0], deq[31]) == (-8.0, 7.5)
        assert g.info(index=1)["name"] == "q"
        with pytest.raises(htr.HtrError, match="not a string"):
            g.str("a.names")
        with pytest.raises(htr.HtrError, match="no metadata key"):
            g.u32("a.missing")
        with pytest.raises(htr.HtrError, match="no tensor"):
            g.info("nope")


@pytest.mark.parametrize("al", [None, 64])
def test_writer_matches_the_reference_layout(al):
    """the test-side writer reproduces the reference test's bytes exactly (so files it writes are GGUF as the
    reference's reader sees them)"""
    w = np.array([1.0, -2.0, 0.5, 3.0, 0.0, 1.5], np.float32).view(np.uint32).__rshift__(16).astype("<u2").tobytes()
    q = np.float16(0.5).tobytes() + bytes((i - 16) & 0xFF for i in range(32))
    got = gguf_bytes([("a.n", U32, 7), ("a.names", ARR, (STR, ["x", "yz"])), ("a.mean", ARR, (F32, [0.5, 0.25, -1.0]))],
                     [("w", GGML_BF16, [3, 2], w), ("q", GGML_Q8_0, [32], q)], alignment=al)
    assert got == reference_tiny(al)


def test_rejects_unknown_type_truncation_and_bad_magic():
    b = bytearray(reference_tiny())
    # the q tensor's type field: Q8_0 (8) → Q4_K (12), as lib.rs:594-598 patches it
    pos = bytes(b).index(bytes([1, 0, 0, 0, 32, 0, 0, 0, 0, 0, 0, 0])) + 12
    b[pos] = 12
    with pytest.raises(htr.HtrError, match="not supported"):
        htr.Gguf(data=bytes(b))
    with pytest.raises(htr.HtrError, match="ends at byte"):
        htr.Gguf(data=reference_tiny()[:-1])
    with pytest.raises(htr.HtrError, match="no GGUF magic"):
        htr.Gguf(data=b"GGUX")
    with pytest.raises(htr.HtrError, match="truncated"):
        htr.Gguf(data=reference_tiny()[:40])


def test_rejects_malformed_headers():
    base = [("a.n", U32, 7)]
    t = [("q", GGML_Q8_0, [32], bytes(34))]
    with pytest.raises(htr.HtrError, match="version 1"):
        htr.Gguf(data=gguf_bytes(base, t, version=1))
    with pytest.raises(htr.HtrError, match="duplicate metadata key"):
        htr.Gguf(data=gguf_bytes(base + base, t))
    with pytest.raises(htr.HtrError, match="not a power of two"):
        htr.Gguf(data=gguf_bytes(base, t, alignment=48))
    with pytest.raises(htr.HtrError, match="duplicate tensor"):
        htr.Gguf(data=gguf_bytes(base, t + t))
    with pytest.raises(htr.HtrError, match="whole number of blocks"):
        htr.Gguf(data=gguf_bytes(base, [("q", GGML_Q8_0, [16], bytes(34))]))
    bad_bool = bytearray(gguf_bytes([("a.b", 7, 1)], t))
    bad_bool[bytes(bad_bool).index(_s("a.b")) + len(_s("a.b")) + 4] = 2
    with pytest.raises(htr.HtrError, match="bool value 2"):
        htr.Gguf(data=bytes(bad_bool))
    nested = gguf_bytes([("a.x", ARR, (ARR, []))], t)
    with pytest.raises(htr.HtrError, match="nested arrays"):
        htr.Gguf(data=nested.replace(struct.pack("<IQ", 9, 0), struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 4, 0), 1))


def test_long_header_and_file_source(tmp_path):
    """a header of 2.4 MB (a 200k-entry string array, like the text GGUF's tokenizer) is read through the doubling
    prefix; a file on disk and the same bytes through the read callback parse alike"""
    vocab = [f"tok{i}" for i in range(200_000)]
    data = gguf_bytes([("tokenizer.ggml.tokens", ARR, (STR, vocab)), ("a.n", U32, 11)],
                      [("q", GGML_Q8_0, [64], np.arange(68, dtype=np.uint8).tobytes())])
    assert len(data) > 2 * (1 << 20)
    p = tmp_path / "long.gguf"
    p.write_bytes(data)
    with htr.Gguf(p) as g1, htr.Gguf(data=data) as g2:
        assert g1.header() == g2.header()
        assert g1.u32("a.n") == 11 == g2.u32("a.n")
        assert np.array_equal(g1.read_small("q"), np.arange(68, dtype=np.uint8))
        assert g1.info("q") == g2.info("q")
    with pytest.raises(htr.HtrError, match="cannot open"):
        htr.Gguf(tmp_path / "missing.gguf")


def test_text_model_file_metadata():
    """a qwen3 text GGUF of the reference's tiny model: the keys TextConfig::from_gguf reads and the tensor table"""
    cfg, te, on, layers = tiny_text_model()
    with htr.Gguf(data=text_model_gguf(cfg, te, on, layers)) as g:
        assert g.str("general.architecture") == "qwen3"
        assert g.u32("qwen3.block_count") == 5 and g.u32("qwen3.embedding_length") == 256
        assert g.f32("qwen3.rope.freq_base") == 1e6
        t = g.info("blk.4.ffn_down.weight")
        assert (t["shape"], t["type"], t["n_bytes"]) == ([512, 256], GGML_Q8_0, 256 * 512 // 32 * 34)
        assert g.info("token_embd.weight")["shape"] == [256, 1000]
        assert g.header()["n_tensors"] == 2 + 5 * 11
        assert g.read_small("blk.0.attn_norm.weight").view(np.float32).tolist() == layers[0]["attn_norm"].tolist()


def test_bf16_bits_round_to_nearest_even():
    """the writer's f32 → bf16 (the mmproj tensors of the tests): ties to even, the exact values kept, 65504 (no
    bf16) to 65536, subnormals kept; bf16_value is exact"""
    a = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 1 + 2 ** -7, -3.0, 65504.0, 2.0 ** -130], np.float32)
    b = bf16_bits(a)
    assert b.tolist() == [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC040, 0x4780, 0x0008]
    assert bf16_value(b).tolist() == [1.0, 1.0, 1 + 2 ** -6, 1 + 2 ** -7, -3.0, 65536.0, 2.0 ** -130]


def test_vision_model_file_metadata():
    """an mmproj GGUF of the tiny encoder: the clip.* keys VisionConfig::from_gguf reads and the tensor table (BF16
    weights [cols, rows], the patch embedding [p, p, 3, dim], F32 norms)"""
    from test_vision_oracle import tiny_vision_cfg

    cfg = tiny_vision_cfg()
    d, f, pp = cfg["dim"], cfg["n_ff"], 3 * cfg["patch"] ** 2
    r = np.random.default_rng(0)
    w = lambda rows, cols: bf16_bits(r.normal(0, 0.05, (rows, cols)))
    nv = lambda n: np.ones(n, np.float32)
    layers = [dict(ln1=nv(d), ln2=nv(d), q=w(d, d), k=w(d, d), v=w(d, d), o=w(d, d), gate=w(f, d), up=w(f, d),
                   down=w(d, f)) for _ in range(cfg["n_layer"])]
    t = dict(patch_embd=w(d, pp), pre_ln=nv(d), layers=layers, input_norm=nv(d), merger=w(d, 4 * d),
             mm1=w(cfg["proj_dim"], d), mm2=w(cfg["proj_dim"], cfg["proj_dim"]))
    with htr.Gguf(data=vision_model_gguf(cfg, t)) as g:
        assert g.str("clip.projector_type") == "lightonocr"
        assert g.u32("clip.vision.embedding_length") == d and g.u32("clip.vision.block_count") == 2
        assert np.array_equal(np.float32(g.f32_array("clip.vision.image_std")), np.float32(cfg["std"]))
        ti = g.info("v.blk.1.ffn_down.weight")
        assert (ti["shape"], ti["type"], ti["n_bytes"]) == ([f, d], GGML_BF16, 2 * d * f)
        assert g.info("v.patch_embd.weight")["shape"] == [14, 14, 3, d]
        assert g.info("mm.patch_merger.weight")["shape"] == [4 * d, d]
        assert g.info("v.pre_ln.weight")["type"] == GGML_F32
        assert g.header()["n_tensors"] == 2 * 9 + 6
        assert np.array_equal(g.read_small("v.blk.0.attn_q.weight").view(np.uint16), layers[0]["q"].ravel())


def test_read_small_refuses_large_tensors():
    big = bytes(34 * 40_000)  # 1.36 MB of q8_0 blocks
    with htr.Gguf(data=gguf_bytes([], [("big", GGML_Q8_0, [32 * 40_000], big)])) as g:
        with pytest.raises(htr.HtrError, match="not small"):
            g.read_small("big")


def test_hostile_counts_and_offsets_are_errors():
    """a header whose numbers would overflow or ask for absurd memory ends in the reader's error, not in a crash: an
    array count far beyond the bytes left (2^62 elements), and a tensor offset near 2^64 (offset + bytes wraps)"""
    base = [("a.n", U32, 7)]
    t = [("q", GGML_Q8_0, [32], bytes(34))]
    b = bytearray(gguf_bytes(base + [("a.arr", ARR, (U32, [1, 2, 3]))], t))
    # the array's count (u64 after its element type u32 = 4) → 2^62
    key = b"a.arr"
    pos = bytes(b).index(key) + len(key) + 4 + 4  # key, value type ARR (u32), element type (u32)
    b[pos:pos + 8] = (1 << 62).to_bytes(8, "little")
    with pytest.raises(htr.HtrError, match="truncated"):
        htr.Gguf(data=bytes(b))
    # the tensor's offset (u64 after name, n_dims, dims, type) → 2^64 − 64 (aligned): data offset + offset wraps
    b = bytearray(gguf_bytes(base, t))
    pos = bytes(b).index(b"\x01\x00\x00\x00\x20\x00\x00\x00\x00\x00\x00\x00\x08\x00\x00\x00") + 16
    b[pos:pos + 8] = ((1 << 64) - 64).to_bytes(8, "little")
    with pytest.raises(htr.HtrError, match="ends past byte 2\\^64"):
        htr.Gguf(data=bytes(b))
