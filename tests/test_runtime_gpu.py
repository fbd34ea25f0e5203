"""Device runtime on the GPU: the device copy (gpu.rs:2102-2110 Batch::copy → copy_words.wgsl), the read measurement
(htr_debug_read), the memory ledger per kind (gpu.rs:509-561), and the copy's argument checks."""
import numpy as np
import pytest

import htr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 48, 1000, 4096 + 7, (3 << 20) + 5])
def test_copy_is_exact(dev, nbytes):
    """bit-exact copies, whole 16-byte units and a ragged tail; the byte after the copy stays untouched"""
    rng = np.random.default_rng(nbytes)
    src_h = rng.integers(0, 256, nbytes, dtype=np.uint8)
    src = dev.upload(src_h)
    dst = dev.upload(np.full(nbytes + 16, 0xA5, dtype=np.uint8))
    dst.copy_from(src, nbytes)
    got = dst.download(np.uint8)
    assert np.array_equal(got[:nbytes], src_h)
    assert np.all(got[nbytes:] == 0xA5)
    src.free()
    dst.free()


def test_copy_rejects_overlap_and_misalignment(dev):
    b = dev.alloc(4096)
    with pytest.raises(htr.HtrError, match="overlap"):
        htr._check(htr.lib().htr_copy(dev.h, b.ptr + 16, b.ptr, 256))
    with pytest.raises(htr.HtrError, match="aligned"):
        htr._check(htr.lib().htr_copy(dev.h, b.ptr + 4, b.ptr + 1024, 256))
    b.free()


def test_read_measurement_reads_and_leaves_memory_alone(dev):
    """htr_debug_read (the bench's read leg): every launch shape over a buffer whose size is not a multiple of a
    workgroup's share leaves the buffer and the 4-byte sink's neighbours as they were (the fold of these bytes is not
    the stored value, so the sink keeps its word too); misaligned or odd sizes and other shares are refused"""
    n = (5 << 20) + 48
    data = np.random.default_rng(5).integers(0, 256, n, dtype=np.uint8)
    data[:16] = 0  # not a fold of 0x7fffffff for any launch shape: checked below on the host
    buf = dev.upload(data)
    sink = dev.upload(np.array([0x12345678, 0xA5A5A5A5], np.uint32))
    for nt in (True, False):
        for kb in (16, 32, 64):
            buf.read_through(sink, nt, kb)
    dev.sync()
    assert np.array_equal(buf.download(np.uint8), data)
    words = data.view(np.int32).reshape(-1, 4)
    for kb in (16, 32, 64):  # no workgroup's fold equals the value that would be stored
        per = kb * 1024 // 16
        for g in range(0, words.shape[0], per):
            f = np.bitwise_xor.reduce(words[g:g + per].reshape(-1))
            assert f != 0x7FFFFFFF
    assert sink.download(np.uint32).tolist() == [0x12345678, 0xA5A5A5A5]
    with pytest.raises(htr.HtrError, match="multiple of 16"):
        htr._check(htr.lib().htr_debug_read(dev.h, buf.ptr + 4, 1024, 1, 16, sink.ptr))
    with pytest.raises(htr.HtrError, match="multiple of 16"):
        htr._check(htr.lib().htr_debug_read(dev.h, buf.ptr, 1000, 1, 16, sink.ptr))
    with pytest.raises(htr.HtrError, match="KB a workgroup"):
        htr._check(htr.lib().htr_debug_read(dev.h, buf.ptr, 4096, 1, 8, sink.ptr))
    buf.free()
    sink.free()


def test_memory_ledger_counts_per_kind(dev):
    before = dev.mem_live()
    a = dev.alloc(1 << 20, htr.MEM_KV_CACHE)
    b = dev.alloc(3 << 20, htr.MEM_WORK)
    mid = dev.mem_live()
    assert mid["kv_cache"] - before["kv_cache"] == 1 << 20
    assert mid["work"] - before["work"] == 3 << 20
    a.free()
    b.free()
    assert dev.mem_live() == before


def test_phase_ranges(dev):
    """gpu.rs:1349-1358 Gpu::phase: each name opens a roctx range on this thread and ends the previous one ("-" ends
    it); on a dead device the call fails with the sticky reason"""
    for name in ("vision", "prefill", "decode", "-", "-", "decode"):
        dev.phase(name)
    dev.phase("-")
    d = htr.Device(0)
    d.phase("prefill")
    d.mark_lost("test: device.destroy()")
    with pytest.raises(htr.HtrError, match="device.destroy"):
        d.phase("decode")
    d.close()
