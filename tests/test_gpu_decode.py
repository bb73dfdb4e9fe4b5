"""Full-size decode parity on the GPU against the compiled reference engine
(tests/golden/decode_<variant>_s1.npz, written by
tests/golden/make_decode_golden.py from oracle/_ref on the same synthetic
27B-shaped GGUF and the same prompt ids as bench.py).

  q4km  512-token prompt, then speculative_greedy(k=3) until 256 tokens are
        produced, and from a reset the same prompt + 256 greedy tokens
  iq1m  4096-token prompt prefilled as one batch, then speculative_greedy(k=3)
        until 1024 tokens are produced, and from a reset the same prompt +
        1024 greedy tokens (context 4097..5120)

Bar: bit-identical.  The prefill logits, every transaction's logits and
every greedy step's logits compare by SHA-256 of their float32 bytes; the
token ids and accepted counts compare exactly.  The call sequence is the
reference's own speculative bench (src/cli/qwen38_spec_bench.c:37-83,
100-119).

The device sampler entry points (q38hip_model_sample,
q38hip_model_forward_sample) are checked on the same model against
q38_sample on the host logits: same tokens, same RNG states."""
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


def test_device_sampling_matches_reference(case):
    """Sampling on the device from the model's logits, against the
    reference's q38_sample over the downloaded logits: the reference CLI's
    generation loop (src/cli/qwen38_main.c:545-553: sample, observe,
    forward) run both ways for 24 tokens with the presence penalty on, and
    single draws with several sampler settings."""
    from oracle import Oracle, Reference
    from q38hip import Sampler
    golden, model, prompt, _ = case
    checker = Reference() if Reference.available() else Oracle()
    vocab = model.lib.q38_model_vocab_size(model.handle)
    model.reset()
    logits = model.prefill(prompt[:32])
    presence = np.zeros(vocab, np.uint8)
    presence[np.argsort(-logits)[:5]] = 1
    for s in (Sampler(seed=7, temperature=0.8, top_k=40, top_p=0.9), Sampler(seed=0),
              Sampler(seed=3, temperature=0.0), Sampler(seed=5, temperature=1.0, top_k=1),
              Sampler(seed=11, temperature=1.3, top_k=256, top_p=1.0, presence_penalty=1.5, presence=presence),
              Sampler(seed=13, temperature=0.6, top_k=1024, top_p=0.99, presence_penalty=-0.5, presence=presence)):
        want = checker.sample(logits, s.state, s.temperature, s.top_p, s.presence_penalty, s.top_k, s.presence)
        got = model.sample(s)
        assert (got, s.state) == want, vars(s)

    def settings(presence):
        return Sampler(seed=21, temperature=0.9, top_k=20, top_p=0.95, presence_penalty=0.7, presence=presence)

    host = settings(np.zeros(vocab, np.uint8))
    model.reset()
    logits = model.prefill(prompt[:32])
    token, host.state = checker.sample(logits, host.state, host.temperature, host.top_p, host.presence_penalty,
                                       host.top_k, host.presence)
    want = [token]
    for _ in range(24):
        host.observe(token)
        logits = model.forward_token(token)
        token, host.state = checker.sample(logits, host.state, host.temperature, host.top_p,
                                           host.presence_penalty, host.top_k, host.presence)
        want.append(token)

    dev = settings(np.zeros(vocab, np.uint8))
    model.reset()
    model.prefill(prompt[:32])
    got = [model.sample(dev)]
    for _ in range(24):
        dev.observe(got[-1])
        got.append(model.forward_sample(got[-1], dev))
    assert got == want
    assert dev.state == host.state
