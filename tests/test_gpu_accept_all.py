"""Speculative transactions that accept EVERY draft, on the GPU, against the
compiled reference engine (tests/golden/accept_all_s1.npz, written by
tests/golden/make_accept_all_golden.py).

The checkpoint is the "accept_all" GGUF: the 65-block Q4_K_M model whose LM
head rows all hold the same bytes, so every logit of a row is equal, the
greedy token of the target and of the MTP head is always 0 and a
transaction of k drafts consumes all k rows (src/qwen38/qwen38_model.c:
1665-1676).  The logits still carry the hidden state (each is row 0's dot
product with it), so the digests pin the state after every transaction.

What this runs that random weights never reach:
* one-graph transactions consuming 4..8 rows;
* draft counts above the 8-row verify batch (9, 12, 16, 17, 20, 24): a
  second and third verify chunk, recurrent state slots wrapping around the
  slot ring after 9 or more consumed rows, the MTP catch-up over every chunk
  and the returned logits row taken from the last chunk;
* the stop token ending the drafts at the first one;
* prompt batches whose length is a multiple of 9 (18 tokens, and 521 tokens
  = one 512-token batch + one of 9 rows).

Bar: bit-identical ids, counts, positions, logits SHA-256, final MTP logits
and the hidden state after all 64 blocks."""
import hashlib
import os
import time

import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "accept_all_s1.npz")


def digest(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def golden():
    if not os.path.exists(GOLDEN):
        pytest.skip("tests/golden/accept_all_s1.npz not written")
    return dict(np.load(GOLDEN))


@pytest.fixture(scope="module")
def model(device):
    from conftest import synthetic_model
    from golden.make_accept_all_golden import CONTEXT
    from q38hip.model import Model
    path = synthetic_model("accept_all")
    t0 = time.time()
    m = Model.open(path, CONTEXT)
    m.enable_mtp()
    print("model open + upload %.1f s" % (time.time() - t0), flush=True)
    yield m
    m.close()


def test_every_draft_accepted_matches_reference(model, golden):
    from golden.make_accept_all_golden import PROMPT_LEN, SCHEDULE, prompt_ids
    model.reset()
    model.enable_mtp()
    logits = model.prefill(prompt_ids(PROMPT_LEN))
    assert digest(logits) == golden["prefill_digest"][0], "prefill of %d tokens" % PROMPT_LEN
    produced = [int(np.argmax(logits))]
    for i, (k, stop) in enumerate(SCHEDULE):
        print("transaction %d: k=%d stop=%#x" % (i, k, stop), flush=True)
        ok, accepted, logits = model.try_speculative_greedy(produced[-1], stop, k)
        assert ok, "transaction %d failed" % i
        want = golden["accepted"][i][:int(golden["counts"][i])]
        assert list(accepted) == [int(t) for t in want], "transaction %d (k=%d)" % (i, k)
        assert model.position() == int(golden["positions"][i]), "transaction %d" % i
        assert digest(logits) == golden["digests"][i], "transaction %d (k=%d) logits" % (i, k)
        produced.extend(int(t) for t in accepted)
    assert list(golden["counts"]) == [1 if stop == 0 else k for k, stop in SCHEDULE]
    assert produced == [int(t) for t in golden["tokens"]]
    pending = produced[-1]
    assert digest(model.mtp_forward(pending)) == golden["final_mtp_digest"][0]
    hidden = model.forward_token_layers(pending, 64)
    assert np.array_equal(hidden.view(np.uint32), golden["final_hidden"].view(np.uint32)), \
        "max abs diff %g" % np.abs(hidden - golden["final_hidden"]).max()


def test_greedy_logits_match_reference(model, golden):
    """Plain decoding over the same length: every logits row equals the
    reference's, and the tokens equal the speculative ones."""
    from golden.make_accept_all_golden import PROMPT_LEN, prompt_ids
    model.reset()
    model.enable_mtp()
    logits = model.prefill(prompt_ids(PROMPT_LEN))
    want = golden["greedy_digests"]
    tokens = [int(np.argmax(logits))]
    assert digest(logits) == want[0]
    for i in range(1, len(want)):
        logits = model.forward_token(tokens[-1])
        assert digest(logits) == want[i], "greedy step %d" % i
        tokens.append(int(np.argmax(logits)))
    assert tokens == [int(t) for t in golden["greedy_tokens"]]


def test_prompt_of_512_plus_9_tokens(model, golden):
    """A 521-token prompt is prefilled as a 512-token batch and a 9-row batch
    (a multiple of the 9 recurrent state slots): logits, the next greedy
    steps and the hidden state after all 64 blocks equal the reference's."""
    from golden.make_accept_all_golden import LONG_PROMPT_LEN, LONG_STEPS, PROMPT_SEED, prompt_ids
    model.reset()
    model.enable_mtp()
    logits = model.prefill(prompt_ids(LONG_PROMPT_LEN, PROMPT_SEED + 1))
    want = golden["long_digests"]
    assert digest(logits) == want[0], "prefill of %d tokens" % LONG_PROMPT_LEN
    token = int(np.argmax(logits))
    for i in range(LONG_STEPS):
        logits = model.forward_token(token)
        assert digest(logits) == want[i + 1], "step %d after the long prompt" % i
        token = int(np.argmax(logits))
    hidden = model.forward_token_layers(token, 64)
    assert np.array_equal(hidden.view(np.uint32), golden["long_hidden"].view(np.uint32)), \
        "max abs diff %g" % np.abs(hidden - golden["long_hidden"]).max()
