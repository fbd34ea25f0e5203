"""Device runtime on the GPU: the device copy (gpu.rs:2102-2110 Batch::copy → copy_words.wgsl), the memory ledger per
kind (gpu.rs:509-561), and the copy's argument checks."""
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
