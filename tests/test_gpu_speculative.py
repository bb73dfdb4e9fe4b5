"""Speculative decoding with accepted drafts on the GPU, against the compiled
reference engine (tests/golden/accept_s1.npz, written by
tests/golden/make_accept_golden.py).

The checkpoint pair is the "accept" base GGUF (an LM head with two live rows,
so greedy tokens are 0, 1 or 2 and the MTP drafts are often right) and its
separate "accept_mtp" GGUF, attached with q38_model_attach_mtp_gguf.  The
transactions consume 1 .. k rows, so they run what random weights never
reach (src/qwen38/qwen38_model.c:1614-1714): accepted drafts, the target state
after `consumed` rows of the verify batch, the MTP catch-up over several
rows, the stop at stop_token and the refused calls.

Bar: bit-identical.  Every transaction's accepted ids, count, position and
logits (SHA-256) equal the reference's; refused calls return 0 and leave the
position unchanged; after the last transaction the MTP logits and the hidden
state after all 64 blocks equal the reference's."""
import hashlib
import os
import time

import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "accept_s1.npz")
NO_STOP = 0xFFFFFFFF


def digest(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def golden():
    if not os.path.exists(GOLDEN):
        pytest.skip("tests/golden/accept_s1.npz not written")
    return dict(np.load(GOLDEN))


@pytest.fixture(scope="module")
def accept_model(device):
    from conftest import synthetic_model
    from golden.make_accept_golden import CONTEXT
    from q38hip.model import Model
    base, mtp = synthetic_model("accept"), synthetic_model("accept_mtp")
    t0 = time.time()
    m = Model.open(base, CONTEXT)
    print("model open + upload %.1f s" % (time.time() - t0), flush=True)
    yield m, mtp
    m.close()


def test_mtp_calls_refused_before_attach_and_enable(accept_model):
    """Without MTP weights, enable_mtp fails (qwen38_model.c:1564-1569); with
    them attached but not enabled, MTP calls fail; attach only at position 0."""
    model, mtp = accept_model
    model.reset()
    assert model.lib.q38_model_enable_mtp(model.handle) == 0
    model.attach_mtp(mtp)
    assert model.try_speculative_greedy(1, NO_STOP, 3)[0] == 0
    import ctypes
    p = ctypes.POINTER(ctypes.c_float)()
    assert model.lib.q38_model_mtp_forward(model.handle, 1, ctypes.byref(p)) == 0
    assert model.lib.q38_model_attach_mtp_gguf(model.handle, mtp.encode()) == 0   # already attached
    model.enable_mtp()
    assert model.position() == 0


def test_accepted_drafts_match_reference(accept_model, golden):
    from golden.make_accept_golden import REFUSED, SCHEDULE, prompt_ids
    model, mtp = accept_model
    model.reset()
    model.lib.q38_model_attach_mtp_gguf(model.handle, mtp.encode())   # 0 when already attached
    model.enable_mtp()
    logits = model.prefill(prompt_ids())
    assert digest(logits) == golden["prefill_digest"][0]
    produced = [int(np.argmax(logits))]
    refused = []
    for i, (k, stop) in enumerate(SCHEDULE):
        for (at, token, count) in REFUSED:
            if at == i:
                ok, _, _ = model.try_speculative_greedy(token, NO_STOP, count)
                refused.append([token, count, ok, model.position()])
        ok, accepted, logits = model.try_speculative_greedy(produced[-1], stop, k)
        assert ok, "transaction %d failed" % i
        want = golden["accepted"][i][:int(golden["counts"][i])]
        assert list(accepted) == [int(t) for t in want], "transaction %d (k=%d, stop=%d)" % (i, k, stop)
        assert model.position() == int(golden["positions"][i]), "transaction %d" % i
        assert digest(logits) == golden["digests"][i], "transaction %d logits" % i
        produced.extend(int(t) for t in accepted)
    assert refused == golden["refused"].tolist()
    assert produced == [int(t) for t in golden["tokens"]]
    assert produced == [int(t) for t in golden["greedy_tokens"]]
    counts = golden["counts"]
    assert (counts > 1).sum() >= 5 and (counts == np.array([k for k, _ in SCHEDULE])).sum() >= 2, \
        "the fixture must contain accepted drafts"
    pending = produced[-1]
    assert digest(model.mtp_forward(pending)) == golden["final_mtp_digest"][0]
    hidden = model.forward_token_layers(pending, 64)
    assert np.array_equal(hidden.view(np.uint32), golden["final_hidden"].view(np.uint32)), \
        "max abs diff %g" % np.abs(hidden - golden["final_hidden"]).max()


def test_long_drafts_reproduce_greedy(accept_model):
    """Draft counts above the 8 rows of one verify batch (9 .. 20) run the
    verify in 8-row chunks: the accepted tokens and every returned logits
    row equal plain greedy decoding's (the reference's invariant,
    src/cli/qwen38_spec_bench.c:100-119), bit for bit."""
    from golden.make_accept_golden import prompt_ids
    model, mtp = accept_model
    model.reset()
    model.lib.q38_model_attach_mtp_gguf(model.handle, mtp.encode())
    model.enable_mtp()
    n = 48
    logits = model.prefill(prompt_ids())
    greedy, digests = [int(np.argmax(logits))], [digest(logits)]
    while len(greedy) < n + 24:
        logits = model.forward_token(greedy[-1])
        greedy.append(int(np.argmax(logits)))
        digests.append(digest(logits))
    model.reset()
    logits = model.prefill(prompt_ids())
    produced = [int(np.argmax(logits))]
    counts = []
    for k in (12, 20, 9, 17, 11, 24, 10, 16) * 4:
        if len(produced) >= n:
            break
        stop = 2 if k % 2 else NO_STOP
        ok, accepted, logits = model.try_speculative_greedy(produced[-1], stop, k)
        assert ok, "k=%d failed" % k
        produced.extend(int(t) for t in accepted)
        counts.append(len(accepted))
        assert produced == greedy[:len(produced)], "k=%d counts %s" % (k, counts)
        assert digest(logits) == digests[len(produced) - 1], "k=%d logits" % k
        assert model.position() == len(prompt_ids()) + len(produced) - 1
    print("long-draft transactions consumed", counts, flush=True)
    assert max(counts) > 1
