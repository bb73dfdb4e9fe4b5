"""The oracle's token sampler (orc_sample) pinned on the CPU.

  - the reference's own unit test (tests/unit/test_qwen38_sampler.c) and its
    answers;
  - the compiled reference q38_sample (oracle/_ref) on every case of
    sampler_cases, tokens and RNG states equal;
  - what the mathematics fixes, independently of the reference: greedy is
    numpy's first argmax; the state sequence is Vigna's xorshift64*; the
    frequencies of many draws follow the renormalised softmax of the top-k /
    top-p candidates (a dropped temperature, a wrong sign or a shifted index
    fails it).
"""
import numpy as np
import pytest

import sampler_cases as sc

MASK = (1 << 64) - 1


def xorshift64star(state):
    """Vigna, "An experimental exploration of Marsaglia's xorshift
    generators, scrambled" (2016): shifts 12, 25, 27 and the multiplier
    2685821657736338717.  Returns (output, new state)."""
    x = state
    x ^= x >> 12
    x ^= (x << 25) & MASK
    x ^= x >> 27
    return (x * 2685821657736338717) & MASK, x


def test_unit_answers(oracle):
    for case, want in sc.unit_cases():
        token, _ = sc.call(oracle, case)
        assert token == want, case["name"]


def test_matches_reference(oracle, reference):
    rng = np.random.default_rng(7)
    cases = [c for c, _ in sc.unit_cases()] + sc.special_cases(rng) + sc.random_cases(rng, 120)
    for case in cases:
        assert sc.call(oracle, case) == sc.call(reference, case), case["name"]


def test_greedy_is_first_argmax(oracle):
    rng = np.random.default_rng(3)
    for vocab in (1, 5, 300, 5000):
        logits = (np.round(rng.standard_normal(vocab) * 2) / 2).astype(np.float32)
        state = 12345
        for temperature, top_k in ((0.0, 20), (-2.0, 40), (1.0, 1), (1.0, 0)):
            token, new_state = oracle.sample(logits, state, temperature, 0.9, 0.0, top_k)
            assert token == int(np.argmax(logits))
            assert new_state == state   # greedy draws nothing
    # a NaN at index 0 wins the reference's scan (every > is false); elsewhere it never does
    logits = np.array([np.nan, 1.0, 3.0, 2.0], np.float32)
    assert oracle.sample(logits, 1, 0.0, 0.9, 0.0, 20)[0] == 0
    logits = np.array([1.0, np.nan, 3.0, 3.0], np.float32)
    assert oracle.sample(logits, 1, 0.0, 0.9, 0.0, 20)[0] == 2


def test_state_is_xorshift64star(oracle):
    logits = np.linspace(-1, 1, 50).astype(np.float32)
    state = 0x9E3779B97F4A7C15
    for _ in range(20):
        _, new_state = oracle.sample(logits, state, 1.0, 0.95, 0.0, 20)
        assert new_state == xorshift64star(state)[1]
        state = new_state


def test_draw_frequencies_follow_softmax(oracle):
    """Empirical frequencies over 40000 draws against the closed form: the
    top_k largest logits, p_i proportional to exp((l_i - l_max) / T), the
    smallest prefix whose cumulative share reaches top_p, renormalised."""
    logits = np.array([0.3, 2.0, -1.0, 1.2, 1.9, -0.4, 0.8, 2.5, -3.0, 0.0], np.float32)
    draws = 40000
    for temperature, top_k, top_p in ((1.0, 20, 1.0), (0.5, 4, 1.0), (2.0, 6, 0.8), (0.7, 10, 0.5)):
        order = np.argsort(-logits.astype(np.float64), kind="stable")[:top_k]
        p = np.exp((logits[order].astype(np.float64) - logits[order[0]]) / temperature)
        p /= p.sum()
        keep = int(np.searchsorted(np.cumsum(p), top_p - 1e-12) + 1) if top_p < 1.0 else len(p)
        expected = np.zeros(len(logits))
        expected[order[:keep]] = p[:keep] / p[:keep].sum()
        counts = np.zeros(len(logits))
        state = 99
        for _ in range(draws):
            token, state = oracle.sample(logits, state, temperature, top_p, 0.0, top_k)
            counts[token] += 1
        freq = counts / draws
        assert np.all(counts[expected == 0] == 0), (temperature, top_k, top_p)
        sigma = np.sqrt(expected * (1 - expected) / draws)
        assert np.all(np.abs(freq - expected) <= 5 * sigma + 1e-9), (temperature, top_k, top_p, freq, expected)


def test_presence_penalty_subtracts(oracle):
    logits = np.array([1.0, 5.0, 4.5, 0.0], np.float32)
    presence = np.array([0, 1, 0, 0], np.uint8)
    assert oracle.sample(logits, 1, 0.0, 0.9, 1.0, 20, presence)[0] == 2
    assert oracle.sample(logits, 1, 0.0, 0.9, 0.25, 20, presence)[0] == 1
    # ids at or beyond presence_size are never penalised
    assert oracle.sample(logits, 1, 0.0, 0.9, 1.0, 20, presence[:1])[0] == 1
    with pytest.raises(ValueError):
        oracle.sample(np.zeros(0, np.float32), 1, 1.0, 0.9, 0.0, 20)
