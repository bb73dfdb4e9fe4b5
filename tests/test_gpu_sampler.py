"""Device token sampler (q38hip_sample) against q38_sample.

The checker is the compiled reference (oracle/_ref, src/qwen38/
qwen38_sampler.c) when it is present, else the oracle's orc_sample, which
tests/test_sampler_oracle.py pins to it.  Bar: the same token and the same
xorshift64* state after the call, on every case of sampler_cases (greedy
and sampling paths, ties, infinities, NaN, presence penalty, vocabulary
sizes from 1 to 248320)."""
import numpy as np
import pytest

import sampler_cases as sc

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(300)]


@pytest.fixture(scope="module")
def checker(oracle):
    from oracle import Reference
    return Reference() if Reference.available() else oracle


def device_sample(case, device):
    import torch
    import q38hip
    logits = torch.from_numpy(case["logits"]).to(device)
    presence = None if case["presence"] is None else torch.from_numpy(case["presence"]).to(device)
    sampler = q38hip.Sampler(temperature=case["temperature"], top_p=case["top_p"],
                             presence_penalty=case["presence_penalty"], top_k=case["top_k"])
    sampler.state = case["state"]
    token = q38hip.sample(logits, sampler, presence)
    return int(token.cpu()[0]), sampler.state


def test_unit_answers(device):
    for case, want in sc.unit_cases():
        token, _ = device_sample(case, device)
        assert token == want, case["name"]


def test_special_values_match_reference(device, checker):
    for case in sc.special_cases(np.random.default_rng(11)):
        print(case["name"], flush=True)
        assert device_sample(case, device) == sc.call(checker, case), case["name"]


def test_random_cases_match_reference(device, checker):
    for case in sc.random_cases(np.random.default_rng(12), 160):
        assert device_sample(case, device) == sc.call(checker, case), case["name"]


def test_state_sequence(device, checker):
    """64 consecutive draws from one row: the state carried from call to
    call as the reference carries it."""
    import torch
    import q38hip
    rng = np.random.default_rng(5)
    logits = (rng.standard_normal(sc.VOCAB) * 2).astype(np.float32)
    dev = torch.from_numpy(logits).to(device)
    sampler = q38hip.Sampler(seed=2024, temperature=0.9, top_p=0.9, top_k=50)
    state = sampler.state
    for i in range(64):
        got = int(q38hip.sample(dev, sampler).cpu()[0])
        want, state = checker.sample(logits, state, 0.9, 0.9, 0.0, 50)
        assert (got, sampler.state) == (want, state), "draw %d" % i


def test_limits_are_errors(device):
    import torch
    import q38hip
    logits = torch.zeros(5000, dtype=torch.float32, device=device)
    sampler = q38hip.Sampler(seed=9, temperature=1.0, top_k=2000)
    with pytest.raises(RuntimeError, match="1024"):
        q38hip.sample(logits, sampler)
    assert sampler.state == 9   # a refused call leaves the state alone
    # greedy takes any top_k; top_k beyond a small vocabulary is that vocabulary
    sampler.temperature = 0.0
    assert int(q38hip.sample(logits, sampler).cpu()[0]) == 0
    sampler.temperature = 1.0
    q38hip.sample(logits[:700], sampler)
    assert sampler.state != 9
