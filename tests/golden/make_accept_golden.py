#!/usr/bin/env python3
"""Golden speculative-decoding transactions of the COMPILED REFERENCE engine
(oracle/_ref/libq38ref.so) on the synthetic checkpoint pair whose drafts get
accepted: the "accept" base GGUF (64 Q4_K_M blocks, an LM head with two live
rows, so every greedy token is 0, 1 or 2) and the separate "accept_mtp" GGUF
attached with q38_model_attach_mtp_gguf (src/qwen38/qwen38_model.c:1408-1425).

Random weights make the target and the MTP head disagree on nearly every
draft; here they agree about a third of the time, so the transactions
consume 1, 2, ... k rows.  That runs the paths a real checkpoint takes
(src/qwen38/qwen38_model.c:1614-1714): accepted drafts, the restore of the
target state after `consumed` rows, the MTP catch-up over several rows, the
stop at stop_token, draft counts above the 8 rows of one verify batch, and the
refused calls (bad token, no drafts, more drafts than the context holds),
which must leave the state as it was.

Scenario (context 1024): prefill an 80-token prompt (positions cross the
attention kernels' 32- and 64-position batches), then the SCHEDULE of
(draft_count, stop_token) transactions with the refused calls in between,
then one MTP draft and the hidden state after all 64 blocks for the pending
token.  Stored: every accepted id list, count, position after, SHA-256 of
every returned logits row, the final MTP logits digest and hidden state, and
the plain greedy tokens over the same length (the reference's own invariant
that speculative decoding reproduces greedy decoding is asserted here).

Run from the repository root:
  python tests/golden/make_accept_golden.py
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
PROMPT_SEED = 13
PROMPT_LEN = 80
NO_STOP = 0xFFFFFFFF
# (draft_count, stop_token)
SCHEDULE = ([(3, NO_STOP)] * 12 + [(5, NO_STOP)] * 3 + [(8, NO_STOP)] * 3 + [(1, NO_STOP), (2, NO_STOP)] +
            [(3, 2), (3, 2), (4, 2), (4, 0), (5, 1), (8, 2), (3, 0), (6, 1)] +
            [(12, NO_STOP), (20, NO_STOP), (11, 2), (17, 1), (9, NO_STOP)] * 2 + [(3, NO_STOP)] * 6)
# refused calls made before transaction i: (i, token, draft_count)
REFUSED = [(5, 248320, 3), (5, 0, 0), (11, 1, CONTEXT)]


def prompt_ids():
    return np.random.Generator(np.random.PCG64(PROMPT_SEED)).integers(0, 248320, PROMPT_LEN).astype(np.uint32)


def digest(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


def argmax(logits):
    return int(np.argmax(logits))


def run(model, log):
    out = {}
    prompt = prompt_ids()
    logits = model.prefill(prompt)
    out["prefill_digest"] = np.array([digest(logits)])
    produced = [argmax(logits)]
    accepted_rows, counts, digests, positions, refused = [], [], [], [], []
    for i, (k, stop) in enumerate(SCHEDULE):
        for (at, token, count) in REFUSED:
            if at == i:
                ok, _, _ = model.try_speculative_greedy(token, NO_STOP, count)
                refused.append([token, count, ok, model.position()])
        ok, accepted, logits = model.try_speculative_greedy(produced[-1], stop, k)
        if not ok:
            raise AssertionError("transaction %d failed" % i)
        row = np.full(24, 0xFFFFFFFF, dtype=np.uint32)
        row[:len(accepted)] = accepted
        accepted_rows.append(row)
        counts.append(len(accepted))
        digests.append(digest(logits))
        positions.append(model.position())
        produced.extend(int(t) for t in accepted)
    log("transactions: counts %s" % counts)
    out["accepted"] = np.stack(accepted_rows)
    out["counts"] = np.array(counts, dtype=np.uint32)
    out["digests"] = np.array(digests)
    out["positions"] = np.array(positions, dtype=np.uint32)
    out["refused"] = np.array(refused, dtype=np.uint32)
    out["tokens"] = np.array(produced, dtype=np.uint32)
    pending = produced[-1]
    out["final_mtp_digest"] = np.array([digest(model.mtp_forward(pending))])
    out["final_hidden"] = model.forward_token_layers(pending, 64)
    log("final state recorded")

    model.reset()
    logits = model.prefill(prompt)
    greedy = [argmax(logits)]
    while len(greedy) < len(produced):
        greedy.append(argmax(model.forward_token(greedy[-1])))
    out["greedy_tokens"] = np.array(greedy, dtype=np.uint32)
    if greedy != produced:
        raise AssertionError("reference speculative decode differs from its greedy decode")
    log("greedy equivalence holds over %d tokens" % len(greedy))
    return out


def main():
    from oracle import reference_model
    from q38hip import synth
    base = synth.model_path(SEED, "accept")
    mtp = synth.model_path(SEED, "accept_mtp")
    synth.write_model_gguf(base, SEED, "accept")
    synth.write_model_gguf(mtp, SEED, "accept_mtp")
    t0 = time.time()
    log = lambda msg: print("[%7.1f s] %s" % (time.time() - t0, msg), flush=True)  # noqa: E731
    model = reference_model().open(base, CONTEXT)
    model.attach_mtp(mtp)
    model.enable_mtp()
    out = run(model, log)
    model.close()
    dest = os.path.join(os.path.dirname(os.path.abspath(__file__)), "accept_s%d.npz" % SEED)
    np.savez_compressed(dest, seed=np.array([SEED, CONTEXT, PROMPT_LEN, PROMPT_SEED]), **out)
    log("wrote " + dest)


if __name__ == "__main__":
    main()
