"""The bench line's contract on the CPU: one GPU only, and the roofline arithmetic of roofline_by_config."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused_with_a_reason():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_roofline_by_config_fractions():
    import bench

    r = {
        "decode": {"achieved_GBs": 2000.0, "frac": 0.25, "bytes_per_token": 781569024.0, "mean_keys": 1279.5},
        "matvec": {"graph_node_128_copies_GBs": 1200.0, "graph_node_128_copies_frac": 0.15,
                   "batched_launch_GBs": 6900.0, "batched_frac": 6900.0 / 8000.0, "batched_launch_us": 62.0,
                   "batched_bytes_per_launch": 429916160},
        "read": {"best_GBs": 7000.0},
        "choose": {"graph_node_GBs": 100.0, "graph_node_frac": 0.0125, "batched_GBs": 4000.0, "batched_frac": 0.5},
        "attention": {"512": {"graph_node_GBs": 400.0, "graph_node_frac": 0.05}},
        "vision_gemm": {"tflops": 850.0, "frac_mfma_peak": 0.34},
    }
    out = bench.roofline_by_config(r)
    assert set(out) == {"config3_decode", "config0_matvec_graph_node", "config0_matvec_batched",
                        "config1_choice_graph_node", "config1_choice_batched", "config2_attention_512",
                        "config4_vision_gemm"}
    assert out["config0_matvec_batched"]["frac_of_read_ceiling"] == pytest.approx(6900.0 / 7000.0)
    assert out["config0_matvec_batched"]["frac"] == pytest.approx(0.8625)
    assert out["config4_vision_gemm"]["bound"] == "mfma"
    assert all(v["bound"] == "hbm" for k, v in out.items() if k != "config4_vision_gemm")
    assert "frac_of_read_ceiling" not in bench.roofline_by_config({k: v for k, v in r.items() if k != "read"})[
        "config0_matvec_batched"]


def test_no_nan_turns_non_finite_values_into_null():
    import bench

    assert bench.no_nan({"a": float("nan"), "b": [1.0, float("inf")], "c": {"d": 2}}) == {"a": None, "b": [1.0, None],
                                                                                          "c": {"d": 2}}
