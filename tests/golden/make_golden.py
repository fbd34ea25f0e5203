"""Writes tests/golden/reference_cases.json: the known-answer values the reference's own tests state for this path.

Every value below is copied from a reference test as data (inputs and expected outputs), with its file:line:
  - the q8_0 block of the tiny GGUF and its dequantised ends      ocr-gguf/src/lib.rs:584-591
  - the windowed-penalty and frequency-penalty unit cases         ocr-decode/src/sampling.rs:297-321
  - choose_pen_is_exact's special logits and penalty sweep        ocr-wgpu/src/text.rs:1074-1082
  - gpu_choice_matches_choose's case matrix                       ocr-wgpu/src/text.rs:1006-1014
  - the LCG (text.rs:670-673) evaluated in Python integers for seed 11 (an independent restatement of the
    generator the reference tests seed every input with)
Run: python tests/golden/make_golden.py
"""
import json
import os
import struct

import numpy as np


def lcg_values(seed, n):
    out = []
    s = seed
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        out.append(float(np.float32(np.float32(np.float32(s >> 40) / np.float32(1 << 24)) * np.float32(2.0)) - np.float32(1.0)))
    return out


def main():
    block = list(struct.pack("<e", 0.5)) + [(i - 16) & 0xFF for i in range(32)]
    cases = {
        "gguf_q8_0_block": {"source": "ocr-gguf/src/lib.rs:584-591", "bytes": block, "first": -8.0, "last": 7.5},
        "sampling": [
            {"source": "ocr-decode/src/sampling.rs:297-304", "logits": [2.0, 2.2, -1.0], "rp": 1.1, "window": 2,
             "fp": 0.0, "history": [0, 1, 1], "counts": {}, "token": 0, "logit1_after": 2.0, "tol": 1e-6},
            {"source": "ocr-decode/src/sampling.rs:316-321", "logits": [1.0, 1.05], "rp": 1.0, "window": 2,
             "fp": 0.1, "history": [], "counts": {"1": 2}, "token": 0},
        ],
        "choose_pen_exact": {
            "source": "ocr-wgpu/src/text.rs:1074-1082",
            "n": 8192,
            "seed": 3,
            "special_bits": [0x00000000, 0x80000000, 0x7F800000, 0x7F7FFFFF, 0x00000001, 0x00800000],
            "rp": [1.1, 0.9, 1.0000001, 3.0, 1e-3, 1e3, 1.7e-30, 6.0e29],
        },
        "gpu_choice_matrix": {
            "source": "ocr-wgpu/src/text.rs:1006-1014",
            "seed": 77,
            "steps": 40,
            "cases": [
                [151936, 1.1, 20, 0.0, [5] * 30],
                [151936, 1.1, 20, 0.1, [3, 3, 9]],
                [1000, 1.0, 20, 0.0, []],
                [1000, 1.3, 1, 0.0, [1, 2]],
                [1000, 0.7, 7, 0.37, [0, 999, 0, 4, 4, 4, 17, 999]],
                [1000, 1.1, 64, 0.1, [(i * 7) % 13 for i in range(100)]],
                [257, 2.5, 3, 1.5, [256]],
            ],
        },
        "lcg_seed11": {"source": "ocr-wgpu/src/text.rs:670-673", "seed": 11, "values": lcg_values(11, 8)},
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_cases.json")
    with open(path, "w") as f:
        json.dump(cases, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
