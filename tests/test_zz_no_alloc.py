"""htr_decode_attention_static, the decode attention entry point that allocates nothing: its split-K partials and
tickets live in a file-scope device array. Checked through the C ABI against htr_decode_attention (the same kernel
with library-allocated scratch) bit for bit, on two calls in a row — the second with a smaller input, so it runs over
what the first left in the shared array — and recorded into a graph with no call before it at that size."""
import ctypes as C

import numpy as np
import pytest

import htr

pytestmark = pytest.mark.gpu


def _inputs(seed, n_head, n_kv, n_ctx):
    q = htr.synth_normal(seed, n_head * 128)
    k = htr.synth_normal(seed + 1, n_kv * n_ctx * 128).astype(np.float16).view(np.uint16)
    v = htr.synth_normal(seed + 2, n_kv * n_ctx * 128).astype(np.float16).view(np.uint16)
    return q, k, v


def _run(dev, fn, q, k, v, n_head, n_kv, n_ctx, n_keys, scale):
    out = dev.alloc(n_head * 128 * 4)
    rc = fn(dev.h, q.ptr, k.ptr, v.ptr, n_head, n_kv, n_ctx, n_keys, scale, out.ptr)
    if rc < 0:
        raise htr.HtrError(htr.last_error())
    got = out.download(np.float32)
    out.free()
    return got


def test_static_attention_equals_the_allocating_one(dev):
    L = htr.lib()
    sc = float(np.float32(1 / np.sqrt(128)))
    # 1: a long cache (32 chunks of 256 keys: partials of 16 heads x 32 chunks through the array, merged by the last
    # workgroup of each KV head); 2: a smaller one right after (10 chunks of 32 keys) over the first call's leftovers
    for seed, n_head, n_kv, n_ctx, n_keys in ((11, 16, 8, 8192, 8000), (12, 16, 8, 600, 300)):
        qh, kh, vh = _inputs(seed, n_head, n_kv, n_ctx)
        q, k, v = dev.upload(qh), dev.upload(kh), dev.upload(vh)
        want = _run(dev, L.htr_decode_attention, q, k, v, n_head, n_kv, n_ctx, n_keys, sc)
        live = dev.mem_live()
        got = _run(dev, L.htr_decode_attention_static, q, k, v, n_head, n_kv, n_ctx, n_keys, sc)
        assert dev.mem_live() == live  # the static call added nothing to the ledger (its output buffer was freed)
        print(f"\n[static attention] {n_head} / {n_kv} heads, {n_keys} of {n_ctx} keys: equal "
              f"{np.array_equal(got, want)}", flush=True)
        assert np.all(np.isfinite(got)) and np.array_equal(got, want)
        for b in (q, k, v):
            b.free()


def test_static_attention_records_into_a_graph_and_refuses_oversize(dev):
    L = htr.lib()
    sc = float(np.float32(1 / np.sqrt(128)))
    n_head, n_kv, n_ctx, n_keys = 16, 8, 2048, 1500
    qh, kh, vh = _inputs(21, n_head, n_kv, n_ctx)
    q, k, v = dev.upload(qh), dev.upload(kh), dev.upload(vh)
    out = dev.alloc(n_head * 128 * 4)
    dev.capture_begin()
    rc = L.htr_decode_attention_static(dev.h, q.ptr, k.ptr, v.ptr, n_head, n_kv, n_ctx, n_keys, sc, out.ptr)
    g = dev.capture_end()
    assert rc == 0, htr.last_error()
    want = _run(dev, L.htr_decode_attention, q, k, v, n_head, n_kv, n_ctx, n_keys, sc)
    poison = np.full(n_head * 128, np.nan, np.float32)
    for _ in range(3):
        out.upload(poison)
        g.launch()
        dev.sync()
        assert np.array_equal(out.download(np.float32), want)
    g.free()
    # partials of 32 heads x 256 chunks (a 65536-row cache) exceed the 4 MiB array: a clear error, nothing launched
    rc = L.htr_decode_attention_static(dev.h, q.ptr, k.ptr, v.ptr, 32, 16, 65536, 10, sc, out.ptr)
    assert rc < 0 and "static scratch" in htr.last_error()
    rc = L.htr_decode_attention_static(dev.h, q.ptr, k.ptr, v.ptr, 130, 65, 1024, 10, sc, out.ptr)
    assert rc < 0 and "KV heads" in htr.last_error()
    dev.alive()
    for b in (q, k, v, out):
        b.free()
