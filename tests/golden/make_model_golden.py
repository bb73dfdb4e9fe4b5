#!/usr/bin/env python3
"""Golden token sequences and logits digests of the COMPILED REFERENCE engine
(oracle/_ref/libq38ref.so, the reference's own C sources) on the synthetic
27B-shaped models written by qwen3.8-27b-in-c_amd/synth/q38_synth_gguf: the
Q4_K_M layout (variant q4km), the IQ1_M layout (variant iq1m: IQ1_M layer
matrices, Q4_K embedding, Q6_K LM head) and the mixed layout (variant mixed:
every other matrix format the reference accepts, a Q8_0 embedding and a Q5_K
LM head).

The GGUF is a pure function of its seed (about 15.7 GB, not committed); this
script writes it when missing, runs the reference's model API
(include/qwen38/qwen38_model.h) through the scenarios below, and stores the
results as a small fixture: the token ids, SHA-256 digests of every logits
row, top-5 ids/values, a strided sample of the first logits row, and the
hidden state after the first 1 and 4 layers.

Scenarios (context 256, MTP enabled, prompt of 12 seeded ids):
  layers   fresh model, forward_token_layers(prompt[0], 1) and (.., 4)
  greedy   prefill(prompt) then 12 forward_token steps, argmax each
  mtp      prefill(prompt) then 3 chained mtp_forward drafts
  spec     prefill(prompt) then speculative_greedy(k=3) until 12 tokens

Run from the repository root:
  python tests/golden/make_model_golden.py [q4km|iq1m|mixed [GGUF_PATH]]
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
CONTEXT = 256
PROMPT_SEED = 7
PROMPT_LEN = 12
DECODE = 12
DRAFT = 3
NO_STOP = 0xFFFFFFFF
SAMPLE_STRIDE = 1009


def prompt_ids():
    return np.random.Generator(np.random.PCG64(PROMPT_SEED)).integers(0, 248320, PROMPT_LEN).astype(np.uint32)


def digest(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


def top5(logits):
    order = np.argsort(-logits, kind="stable")[:5]
    return order.astype(np.uint32), logits[order].astype(np.float32)


def argmax(logits):
    return int(np.argmax(logits))  # first index of the maximum, as q38_argmax


def run(model, log):
    out = {}
    prompt = prompt_ids()
    out["prompt"] = prompt

    model.reset()
    out["hidden_l1"] = model.forward_token_layers(int(prompt[0]), 1)
    model.reset()
    out["hidden_l4"] = model.forward_token_layers(int(prompt[0]), 4)
    log("layers done")

    model.reset()
    logits = model.prefill(prompt)
    out["prefill_sample"] = logits[::SAMPLE_STRIDE].copy()
    out["prefill_top5_ids"], out["prefill_top5_values"] = top5(logits)
    digests, tokens = [digest(logits)], [argmax(logits)]
    log("prefill done")
    for _ in range(DECODE - 1):
        logits = model.forward_token(tokens[-1])
        digests.append(digest(logits))
        tokens.append(argmax(logits))
    out["greedy_tokens"] = np.array(tokens, dtype=np.uint32)
    out["greedy_digests"] = np.array(digests)
    log("greedy done: %s" % tokens)

    model.reset()
    logits = model.prefill(prompt)
    first = argmax(logits)
    drafts, mtp_digests, token = [], [], first
    for _ in range(DRAFT):
        mlog = model.mtp_forward(token)
        mtp_digests.append(digest(mlog))
        token = argmax(mlog)
        drafts.append(token)
    out["mtp_drafts"] = np.array(drafts, dtype=np.uint32)
    out["mtp_digests"] = np.array(mtp_digests)
    log("mtp done: %s" % drafts)

    model.reset()
    logits = model.prefill(prompt)
    produced = [argmax(logits)]
    batches, spec_digests = [], []
    while len(produced) < DECODE:
        requested = min(DRAFT, DECODE - len(produced))
        accepted, logits = model.speculative_greedy(produced[-1], NO_STOP, requested)
        batches.append(len(accepted))
        spec_digests.append(digest(logits))
        produced.extend(int(t) for t in accepted)
    out["spec_tokens"] = np.array(produced[:DECODE], dtype=np.uint32)
    out["spec_counts"] = np.array(batches, dtype=np.uint32)
    out["spec_digests"] = np.array(spec_digests)
    log("spec done: %s counts %s" % (produced, batches))
    if list(out["spec_tokens"]) != list(out["greedy_tokens"]):
        raise AssertionError("reference speculative decode differs from its greedy decode")
    return out


def main():
    from oracle import reference_model
    from q38hip import synth
    variant = sys.argv[1] if len(sys.argv) > 1 else "q4km"
    if variant not in ("q4km", "iq1m", "mixed"):
        raise SystemExit("variant must be q4km, iq1m or mixed")
    path = sys.argv[2] if len(sys.argv) > 2 else synth.model_path(SEED, variant)
    synth.write_model_gguf(path, SEED, variant)
    t0 = time.time()
    log = lambda msg: print("[%6.1f s] %s" % (time.time() - t0, msg), flush=True)  # noqa: E731
    model = reference_model().open(path, CONTEXT)
    model.enable_mtp()
    out = run(model, log)
    model.close()
    dest = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_%s_s%d.npz" % (variant, SEED))
    np.savez_compressed(dest, seed=np.array([SEED, CONTEXT, DRAFT]), **out)
    log("wrote " + dest)


if __name__ == "__main__":
    main()
