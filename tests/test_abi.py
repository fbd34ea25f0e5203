"""The C ABI library: it loads, exports every symbol include/htr.h declares, and its host-side logic (errors, seeded
inputs) behaves — no GPU needed."""
import os
import re

import numpy as np
import pytest

import htr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "htr.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(htr_[a-z0-9_]+)\s*\(", src)) - {"htr_fatal_hook", "htr_token_cb"})


def test_library_exports_every_declared_symbol():
    lib = htr.lib()
    names = declared_symbols()
    assert len(names) >= 35
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(htr.SYMBOLS) == names


def test_no_device_is_a_clean_error():
    try:
        d = htr.Device(0)
    except htr.HtrError as e:
        assert "device" in str(e).lower()
        return
    d.close()  # a GPU is present (the box): opening worked


def test_synth_inputs_are_seeded_and_shaped():
    a = htr.synth_q8_0(7, 64, 1024)
    assert a.size == 64 * 1024 // 32 * 34
    assert np.array_equal(a, htr.synth_q8_0(7, 64, 1024))
    assert not np.array_equal(a, htr.synth_q8_0(8, 64, 1024))
    b = a.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    q = b[:, 2:].view(np.int8).astype(np.int64)
    assert q.min() == -127 and q.max() == 127
    assert abs(q.mean()) < 1.0 and abs(q.std() - 255 / np.sqrt(12)) < 1.0
    # d = |N(0,1)|·0.002: mean 0.002·√(2/π)
    assert np.all(d >= 0) and abs(d.mean() - 0.002 * np.sqrt(2 / np.pi)) < 5e-5
    x = htr.synth_normal(3, 200000, 1.0, 0.02)
    assert abs(x.mean() - 1.0) < 1e-3 and abs(x.std() - 0.02) < 1e-3
    # a prefix of a longer draw is the shorter draw (counter-based)
    assert np.array_equal(htr.synth_normal(3, 1000), htr.synth_normal(3, 5000)[:1000])


def test_weight_shape_errors_need_no_gpu():
    with pytest.raises(htr.HtrError):
        htr.synth_q8_0(1, 2, 33)
