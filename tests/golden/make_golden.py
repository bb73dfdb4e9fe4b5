#!/usr/bin/env python3
"""Write golden vectors from the COMPILED REFERENCE kernels (oracle/_ref).

Each fixture holds a seeded weight matrix, fp32 activations, the Q8_K blocks
and GEMM outputs the reference's own q38_quantize_q8_k / q38_tensor_gemm_q8_k
produced (built from its sources by oracle/Makefile).  The fixtures are data;
the tests compare the oracle and the HIP kernels against them on hosts where
the reference is not available.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "qwen3.8-27b-in-c_amd"))

from oracle import IQ1_M, Q4_K, Q6_K, Reference  # noqa: E402
from q38hip import synth  # noqa: E402

CASES = [
    # (name, type, rows, width, tokens, weight seed, activation seed)
    ("q4k_r8_w512_m3", Q4_K, 8, 512, 3, 101, 201),
    ("q4k_r5_w1280_m1", Q4_K, 5, 1280, 1, 102, 202),
    ("q4k_r3_w4352_m5", Q4_K, 3, 4352, 5, 103, 203),
    ("iq1m_r8_w512_m3", IQ1_M, 8, 512, 3, 111, 211),
    ("iq1m_r5_w1280_m1", IQ1_M, 5, 1280, 1, 112, 212),
    ("iq1m_r3_w4352_m5", IQ1_M, 3, 4352, 5, 113, 213),
    ("q6k_r8_w512_m3", Q6_K, 8, 512, 3, 121, 221),
    ("q6k_r5_w1280_m1", Q6_K, 5, 1280, 1, 122, 222),
    ("q6k_r3_w4352_m4", Q6_K, 3, 4352, 4, 123, 223),
]


def main():
    ref = Reference()
    out_dir = os.path.dirname(os.path.abspath(__file__))
    for name, qtype, rows, width, tokens, wseed, xseed in CASES:
        w = synth.matrix(qtype, rows, width, seed=wseed)
        x = synth.activations(width, seed=xseed, count=tokens).reshape(-1)
        q = ref.quantize(x)
        y = ref.gemm(qtype, w, rows, q, tokens)
        np.savez_compressed(os.path.join(out_dir, name + ".npz"), meta=np.array([qtype, rows, width, tokens]),
                            w=w, x=x, q8k=q.view(np.uint8), y=y)
        print("wrote", name)


if __name__ == "__main__":
    main()
