#!/usr/bin/env python3
"""Golden transactions of the COMPILED REFERENCE engine
(oracle/_ref/libq38ref.so, the reference's own C sources) on the synthetic
checkpoint whose drafts are ALL accepted: the "accept_all" GGUF, the 65-block
Q4_K_M file whose LM head rows all hold the bytes of row 0.  Every logit of a
row is then the same value, so the greedy token of the target and of the MTP
head is always 0, every draft matches (src/qwen38/qwen38_model.c:1665-1676)
and a transaction of k drafts consumes all k rows.  The logits still depend on
the hidden state (each is the dot product of row 0 with the normed hidden
vector), so their digests pin the state after every transaction.

This drives the paths of a real high-acceptance checkpoint that random
weights never reach: verify batches of more than 8 rows, recurrent state
after 9 or more consumed rows, the MTP catch-up over every consumed row, and
the returned logits taken from the last of many rows.

Scenarios (context 1024):
  spec     an 18-token prompt (a prompt batch whose length is a multiple of
           9), then the SCHEDULE of (draft_count, stop_token) transactions;
           stored: accepted ids, counts, positions, the SHA-256 of every
           returned logits row, then the MTP logits digest and the hidden
           state after all 64 blocks for the pending token
  greedy   reset, the same prompt and forward_token over the same length:
           the token ids (the reference's own invariant that speculative
           decoding reproduces greedy decoding is asserted here) and the
           digest of every logits row
  long     reset, a 521-token prompt (one 512-token batch and one of 9 rows
           where prompts are split into 512-token batches), its logits
           digest, 4 greedy steps' digests and the hidden state after all 64
           blocks for the next token

Run from the repository root (about 10 min on 8 cores):
  python tests/golden/make_accept_all_golden.py [GGUF_PATH]
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
CONTEXT = 1024
PROMPT_SEED = 17
PROMPT_LEN = 18
LONG_PROMPT_LEN = 521
LONG_STEPS = 4
NO_STOP = 0xFFFFFFFF
# (draft_count, stop_token); stop token 0 ends the drafts at the first one
SCHEDULE = [(3, NO_STOP), (5, NO_STOP), (8, NO_STOP), (9, NO_STOP), (16, NO_STOP), (17, NO_STOP),
            (24, NO_STOP), (3, 0), (4, NO_STOP), (12, 0), (20, NO_STOP), (1, NO_STOP), (7, NO_STOP)]


def prompt_ids(count, seed=PROMPT_SEED):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, 248320, count).astype(np.uint32)


def digest(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


def argmax(logits):
    return int(np.argmax(logits))  # first index of the maximum, as q38_argmax


def run(model, log):
    out = {}
    prompt = prompt_ids(PROMPT_LEN)
    model.reset()
    logits = model.prefill(prompt)
    out["prefill_digest"] = np.array([digest(logits)])
    produced = [argmax(logits)]
    accepted_rows, counts, digests, positions = [], [], [], []
    for i, (k, stop) in enumerate(SCHEDULE):
        accepted, logits = model.speculative_greedy(produced[-1], stop, k)
        row = np.full(24, 0xFFFFFFFF, dtype=np.uint32)
        row[:len(accepted)] = accepted
        accepted_rows.append(row)
        counts.append(len(accepted))
        digests.append(digest(logits))
        positions.append(model.position())
        produced.extend(int(t) for t in accepted)
    log("transactions: counts %s" % counts)
    expected = [1 if stop == 0 else k for (k, stop) in SCHEDULE]
    if counts != expected:
        raise AssertionError("not every draft was accepted: %s" % counts)
    out["accepted"] = np.stack(accepted_rows)
    out["counts"] = np.array(counts, dtype=np.uint32)
    out["digests"] = np.array(digests)
    out["positions"] = np.array(positions, dtype=np.uint32)
    out["tokens"] = np.array(produced, dtype=np.uint32)
    pending = produced[-1]
    out["final_mtp_digest"] = np.array([digest(model.mtp_forward(pending))])
    out["final_hidden"] = model.forward_token_layers(pending, 64)
    log("final state recorded")

    model.reset()
    logits = model.prefill(prompt)
    greedy, greedy_digests = [argmax(logits)], [digest(logits)]
    while len(greedy) < len(produced):
        logits = model.forward_token(greedy[-1])
        greedy.append(argmax(logits))
        greedy_digests.append(digest(logits))
    out["greedy_tokens"] = np.array(greedy, dtype=np.uint32)
    out["greedy_digests"] = np.array(greedy_digests)
    if greedy != produced:
        raise AssertionError("reference speculative decode differs from its greedy decode")
    log("greedy equivalence holds over %d tokens" % len(greedy))

    model.reset()
    long_prompt = prompt_ids(LONG_PROMPT_LEN, PROMPT_SEED + 1)
    logits = model.prefill(long_prompt)
    long_digests, token = [digest(logits)], argmax(logits)
    for _ in range(LONG_STEPS):
        logits = model.forward_token(token)
        long_digests.append(digest(logits))
        token = argmax(logits)
    out["long_digests"] = np.array(long_digests)
    out["long_hidden"] = model.forward_token_layers(token, 64)
    log("long prompt done")
    return out


def main():
    from oracle import reference_model
    from q38hip import synth
    path = sys.argv[1] if len(sys.argv) > 1 else synth.model_path(SEED, "accept_all")
    synth.write_model_gguf(path, SEED, "accept_all")
    t0 = time.time()
    log = lambda msg: print("[%7.1f s] %s" % (time.time() - t0, msg), flush=True)  # noqa: E731
    model = reference_model().open(path, CONTEXT)
    model.enable_mtp()
    out = run(model, log)
    model.close()
    dest = os.path.join(os.path.dirname(os.path.abspath(__file__)), "accept_all_s%d.npz" % SEED)
    np.savez_compressed(dest, seed=np.array([SEED, CONTEXT, PROMPT_LEN, PROMPT_SEED, LONG_PROMPT_LEN]), **out)
    log("wrote " + dest)


if __name__ == "__main__":
    main()
