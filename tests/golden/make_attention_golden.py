#!/usr/bin/env python3
"""Golden outputs of the reference's full-attention core, q38_full_core
(src/qwen38/qwen38_model.c:816-885), compiled from its own source through
oracle/ref_attention_shim.c into oracle/_ref/libq38ref.so.

For each case of tests/attention_cases.py (one decode row at positions 0, 1,
31, 32, 33, 2047 and 4100, where the output kernel's 32-position batches
and the score kernel's 64-position chunks start and end), the fixture keeps
the SHA-256 of the gated attention output [6144] and of the K row written to
the cache, plus the first 64 output values.

Run from the repository root:  python tests/golden/make_attention_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import attention_cases as ac  # noqa: E402
from oracle import Reference  # noqa: E402

POSITIONS = (0, 1, 31, 32, 33, 2047, 4100)


def main():
    ref = Reference()
    out = {"positions": np.array(POSITIONS, dtype=np.uint32)}
    digests, key_digests, heads = [], [], []
    for position in POSITIONS:
        context = position + 1
        rows_in, qn, kn, kc, vc = ac.inputs(context, position, 1)
        att = ac.run_rows(ref.full_core, rows_in, qn, kn, kc, vc, position)[0]
        digests.append(ac.digest(att))
        key_digests.append(ac.digest(kc[position]))
        heads.append(att[:64])
        print("position %d: %s" % (position, digests[-1]), flush=True)
    out["digests"] = np.array(digests)
    out["key_digests"] = np.array(key_digests)
    out["first64"] = np.stack(heads)
    dest = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attention_ref.npz")
    np.savez_compressed(dest, **out)
    print("wrote", dest)


if __name__ == "__main__":
    main()
