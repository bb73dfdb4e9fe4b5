#!/usr/bin/env python3
"""Full-size decode fixtures of the COMPILED REFERENCE engine
(oracle/_ref/libq38ref.so, the reference's own C sources) on the synthetic
27B-shaped models, at the sizes the benchmark runs:

  q4km  Q4_K_M layout: a 512-token prompt (bench.py's prompt ids, seed 11),
        then 256 greedy tokens (forward_token) and, from a reset, the same
        prompt followed by speculative_greedy(k=3, no stop token) until 256
        tokens are produced.
  iq1m  IQ1_M layout: a 4096-token prompt (seed 11) prefilled as one batch,
        then speculative_greedy(k=3) until 1024 tokens are produced and, from
        a reset, the same prompt followed by 1024 greedy tokens (context
        4097-5120, the benchmark's IQ1_M decode).

Stored per scenario: the token ids, the accepted counts, and the SHA-256 of
every returned logits row (prefill included), plus a strided sample of the
prefill logits.  The reference's own invariant is asserted as the fixture is
written: its speculative tokens equal its greedy tokens
(src/cli/qwen38_spec_bench.c:100-119).

Run from the repository root (about 10 min for q4km and 5.5 h for iq1m on
8 cores):
  python tests/golden/make_decode_golden.py q4km|iq1m [GGUF_PATH]
"""
import hashlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "qwen3.8-27b-in-c_amd"))

SEED = 1
PROMPT_SEED = 11
NO_STOP = 0xFFFFFFFF
DRAFT = 3
SAMPLE_STRIDE = 1009
# variant: (prompt tokens, speculative tokens, greedy tokens)
SIZES = {"q4km": (512, 256, 256), "iq1m": (4096, 1024, 1024)}


def prompt_ids(count, seed=PROMPT_SEED):
    """bench.py's prompt: uniform token ids from PCG64(seed)"""
    return np.random.Generator(np.random.PCG64(seed)).integers(0, 248320, count).astype(np.uint32)


def digest(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


def argmax(logits):
    return int(np.argmax(logits))  # first index of the maximum, as q38_argmax


def run(model, variant, log):
    prompt_len, spec_len, greedy_len = SIZES[variant]
    prompt = prompt_ids(prompt_len)
    out = {"prompt_len": np.array([prompt_len, PROMPT_SEED], dtype=np.uint32)}

    model.reset()
    logits = model.prefill(prompt)
    log("prefill done")
    out["prefill_digest"] = np.array([digest(logits)])
    out["prefill_sample"] = logits[::SAMPLE_STRIDE].copy()
    produced = [argmax(logits)]
    counts, digests = [], []
    while len(produced) < spec_len:
        accepted, logits = model.speculative_greedy(produced[-1], NO_STOP, DRAFT)
        counts.append(len(accepted))
        digests.append(digest(logits))
        produced.extend(int(t) for t in accepted)
        if len(counts) % 32 == 0:
            log("speculative: %d transactions, %d tokens" % (len(counts), len(produced)))
    out["spec_tokens"] = np.array(produced, dtype=np.uint32)
    out["spec_counts"] = np.array(counts, dtype=np.uint32)
    out["spec_digests"] = np.array(digests)
    log("speculative done: %d tokens in %d transactions" % (len(produced), len(counts)))

    model.reset()
    logits = model.prefill(prompt)
    tokens, greedy_digests = [argmax(logits)], []
    while len(tokens) < greedy_len:
        logits = model.forward_token(tokens[-1])
        greedy_digests.append(digest(logits))
        tokens.append(argmax(logits))
        if len(tokens) % 128 == 0:
            log("greedy: %d tokens" % len(tokens))
    out["greedy_tokens"] = np.array(tokens, dtype=np.uint32)
    out["greedy_digests"] = np.array(greedy_digests)
    log("greedy done")
    n = min(len(tokens), len(produced))
    if tokens[:n] != produced[:n]:
        raise AssertionError("reference speculative decode differs from its greedy decode")
    return out


def main():
    from oracle import reference_model
    from q38hip import synth
    variant = sys.argv[1] if len(sys.argv) > 1 else "q4km"
    if variant not in SIZES:
        raise SystemExit("variant must be one of %s" % ", ".join(SIZES))
    path = sys.argv[2] if len(sys.argv) > 2 else synth.model_path(SEED, variant)
    synth.write_model_gguf(path, SEED, variant)
    prompt_len, spec_len, _ = SIZES[variant]
    t0 = time.time()
    log = lambda msg: print("[%7.1f s] %s" % (time.time() - t0, msg), flush=True)  # noqa: E731
    model = reference_model().open(path, prompt_len + spec_len + 4 * DRAFT)
    model.enable_mtp()
    out = run(model, variant, log)
    model.close()
    dest = os.path.join(os.path.dirname(os.path.abspath(__file__)), "decode_%s_s%d.npz" % (variant, SEED))
    np.savez_compressed(dest, seed=np.array([SEED, DRAFT]), **out)
    log("wrote " + dest)


if __name__ == "__main__":
    main()
