"""Sampler cases shared by the CPU oracle pins and the GPU parity tests.

Each case is a dict of q38_sample's inputs (src/qwen38/qwen38_sampler.c:
51-119, the Q38Sampler fields of include/qwen38/qwen38_sampler.h:10-18):
logits, state, temperature, top_p, presence_penalty, top_k, presence.
The families cover what the reference's arithmetic distinguishes: greedy
and sampling paths, top-k at and beyond the vocabulary, top-p inside and
outside (0, 1), exact ties (order by id), the -FLT_MAX floor of the
candidate list, infinities, NaN at index 0 and elsewhere, the presence
penalty with presence arrays shorter and longer than the vocabulary, and
vocabulary sizes around the 4096-logit chunks of the device kernels up to
the model's 248320.
"""
import numpy as np

FLT_MAX = np.finfo(np.float32).max
VOCAB = 248320


def _case(logits, state, temperature=1.0, top_p=0.95, presence_penalty=0.0, top_k=20, presence=None, name=""):
    return dict(name=name, logits=np.ascontiguousarray(logits, dtype=np.float32), state=int(state),
                temperature=float(temperature), top_p=float(top_p), presence_penalty=float(presence_penalty),
                top_k=int(top_k), presence=None if presence is None else np.ascontiguousarray(presence, np.uint8))


def unit_cases():
    """tests/unit/test_qwen38_sampler.c:11-37 with the answers it asserts:
    (case, expected token)."""
    logits = np.array([-2.0, 1.0, 4.0, 3.0, 0.0], dtype=np.float32)
    presence = np.zeros(5, np.uint8)
    presence[2] = 1
    return [
        (_case(logits, 42, temperature=0.0, name="unit greedy"), 2),
        (_case(logits, 42, temperature=1.0, top_k=1, name="unit top-k one"), 2),
        (_case(logits, 42, temperature=1.0, top_k=2, top_p=0.01, name="unit top-p keeps best"), 2),
        (_case(logits, 42, temperature=0.0, top_k=20, top_p=0.01, presence_penalty=2.0, presence=presence,
               name="unit presence penalty"), 3),
    ]


def special_cases(rng):
    """Infinities, NaN, the -FLT_MAX floor and ties on small rows."""
    out = []
    base = rng.standard_normal(64).astype(np.float32)
    for temperature, top_k in ((0.0, 20), (0.8, 1), (0.8, 20), (1.3, 64), (0.5, 100)):
        def add(logits, name):
            out.append(_case(logits, rng.integers(1, 2**63), temperature=temperature, top_k=top_k,
                             top_p=0.9, name="%s T=%g k=%d" % (name, temperature, top_k)))
        v = base.copy(); v[5] = np.inf; add(v, "+inf")
        v = base.copy(); v[[3, 9, 40]] = np.inf; add(v, "three +inf")
        v = base.copy(); v[::3] = -np.inf; add(v, "-inf")
        v = base.copy(); v[::2] = -FLT_MAX; add(v, "-FLT_MAX")
        add(np.full(64, -np.inf, np.float32), "all -inf")
        add(np.full(64, -FLT_MAX, np.float32), "all -FLT_MAX")
        v = base.copy(); v[0] = np.nan; add(v, "NaN at 0")
        v = base.copy(); v[17] = np.nan; add(v, "NaN inside")
        v = base.copy(); v[[1, 30, 63]] = np.nan; add(v, "NaNs")
        add(np.full(64, np.nan, np.float32), "all NaN")
        add(np.round(base * 2) / 2, "ties")
        add(np.zeros(64, np.float32), "all equal")
        v = base.copy(); v[10] = 3e38; v[11] = -3e38; add(v, "huge")
        add(base * 1e-40, "subnormal")
        v = np.round(base * 2) / 2; v[7] = np.nan; add(v, "ties + NaN")
    return out


def random_cases(rng, count, vocab_sizes=(1, 2, 7, 64, 4095, 4096, 4097, 10000, 65536, VOCAB)):
    """Random rows and parameters over the given vocabulary sizes."""
    out = []
    temps = (0.0, -1.0, 0.1, 0.6, 0.7, 1.0, 1.5, 4.0)
    top_ks = (0, 1, 2, 5, 20, 40, 64, 256, 1024)
    top_ps = (0.0, 0.05, 0.5, 0.8, 0.95, 1.0, 1.5)
    for i in range(count):
        vocab = int(vocab_sizes[i % len(vocab_sizes)])
        kind = rng.integers(0, 4)
        if kind == 0:
            logits = rng.standard_normal(vocab).astype(np.float32) * rng.uniform(0.5, 8.0)
        elif kind == 1:   # ties at a coarse grid
            logits = (np.round(rng.standard_normal(vocab) * 3) / 4).astype(np.float32)
        elif kind == 2:   # a few dominant logits
            logits = rng.standard_normal(vocab).astype(np.float32)
            logits[rng.integers(0, vocab, size=min(vocab, 8))] += 12.0
        else:             # -inf masked rows
            logits = rng.standard_normal(vocab).astype(np.float32) * 3
            logits[rng.random(vocab) < 0.5] = -np.inf
        presence = None
        penalty = 0.0
        if rng.random() < 0.5:
            size = int(rng.choice([vocab, max(1, vocab // 2), vocab + 17]))
            presence = (rng.random(size) < 0.3).astype(np.uint8)
            penalty = float(rng.choice([0.0, 0.5, 1.5, -0.75]))
        out.append(_case(logits, rng.integers(0, 2**64, dtype=np.uint64), temperature=rng.choice(temps),
                         top_p=rng.choice(top_ps), presence_penalty=penalty, top_k=rng.choice(top_ks),
                         presence=presence, name="random %d (vocab %d, kind %d)" % (i, vocab, kind)))
    return out


def call(sampler, case):
    """sampler.sample(...) over a case dict: (token, state)."""
    return sampler.sample(case["logits"], case["state"], case["temperature"], case["top_p"],
                          case["presence_penalty"], case["top_k"], case["presence"])
