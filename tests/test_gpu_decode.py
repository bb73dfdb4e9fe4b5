"""Full-size decode parity on the GPU against the compiled reference engine
(tests/golden/decode_<variant>_s1.npz, written by
tests/golden/make_decode_golden.py from oracle/_ref on the same synthetic
27B-shaped GGUF and the same prompt ids as bench.py).

  q4km  512-token prompt, then speculative_greedy(k=3) until 256 tokens are
        produced, and from a reset the same prompt + 256 greedy tokens
  iq1m  4096-token prompt prefilled as one batch, 32 speculative tokens and
        16 greedy tokens (context past 4096 positions)

Bar: bit-identical.  The prefill logits, every transaction's logits and
every greedy step's logits compare by SHA-256 of their float32 bytes; the
token ids and accepted counts compare exactly.  The call sequence is the
reference's own speculative bench (src/cli/qwen38_spec_bench.c:37-83,
100-119)."""
import hashlib
import os
import time

import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
VARIANTS = [v for v in ("q4km", "iq1m") if os.path.exists(os.path.join(GOLDEN_DIR, "decode_%s_s1.npz" % v))]
NO_STOP = 0xFFFFFFFF


def digest(logits):
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


@pytest.fixture(scope="module", params=VARIANTS)
def case(request, device):
    from conftest import synthetic_model
    from golden.make_decode_golden import DRAFT, prompt_ids
    from q38hip.model import Model
    golden = dict(np.load(os.path.join(GOLDEN_DIR, "decode_%s_s1.npz" % request.param)))
    prompt_len, prompt_seed = (int(v) for v in golden["prompt_len"])
    assert int(golden["seed"][1]) == DRAFT
    path = synthetic_model(request.param)
    spec_len = len(golden["spec_tokens"])
    t0 = time.time()
    m = Model.open(path, prompt_len + spec_len + 4 * DRAFT)
    print("model open + upload %.1f s" % (time.time() - t0), flush=True)
    m.enable_mtp()
    yield golden, m, prompt_ids(prompt_len, prompt_seed), DRAFT
    m.close()


def test_speculative_decode_matches_reference(case):
    golden, model, prompt, draft = case
    model.reset()
    logits = model.prefill(prompt)
    assert digest(logits) == str(golden["prefill_digest"][0]), "prefill logits differ"
    produced = [int(np.argmax(logits))]
    want_tokens = [int(t) for t in golden["spec_tokens"]]
    want_counts = [int(c) for c in golden["spec_counts"]]
    for i, want_digest in enumerate(golden["spec_digests"]):
        accepted, logits = model.speculative_greedy(produced[-1], NO_STOP, draft)
        assert len(accepted) == want_counts[i], "transaction %d: %d accepted, reference %d" % (
            i, len(accepted), want_counts[i])
        produced.extend(int(t) for t in accepted)
        assert produced == want_tokens[:len(produced)], "transaction %d: token ids differ" % i
        assert digest(logits) == str(want_digest), "transaction %d: logits differ" % i
    assert produced == want_tokens


def test_greedy_decode_matches_reference(case):
    golden, model, prompt, _ = case
    model.reset()
    logits = model.prefill(prompt)
    assert digest(logits) == str(golden["prefill_digest"][0])
    tokens = [int(np.argmax(logits))]
    for i, want_digest in enumerate(golden["greedy_digests"]):
        logits = model.forward_token(tokens[-1])
        assert digest(logits) == str(want_digest), "step %d: logits differ" % i
        tokens.append(int(np.argmax(logits)))
    assert tokens == [int(t) for t in golden["greedy_tokens"]]
