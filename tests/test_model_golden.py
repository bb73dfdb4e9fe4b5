"""Consistency of the full-model fixtures written by the compiled reference
(tests/golden/model_<variant>_s1.npz; CPU only).  The fixtures themselves are
the pin of the model path: the reference engine ran on the synthetic
checkpoints."""
import glob
import os

import numpy as np
import pytest

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_*_s1.npz")))


def test_both_layouts_have_fixtures():
    names = {os.path.basename(p) for p in GOLDEN}
    assert {"model_q4km_s1.npz", "model_iq1m_s1.npz"} <= names


@pytest.mark.parametrize("path", GOLDEN, ids=os.path.basename)
def test_fixture_is_self_consistent(path):
    g = np.load(path)
    greedy, spec = list(g["greedy_tokens"]), list(g["spec_tokens"])
    # the reference's speculative path reproduces its greedy sequence
    assert spec == greedy
    # the first greedy token is the argmax of the prefill logits (top-5 head)
    assert int(g["prefill_top5_ids"][0]) == int(greedy[0])
    assert np.all(np.diff(g["prefill_top5_values"]) <= 0)
    # with one token accepted per transaction (random weights: drafts never
    # match), the logits after transaction i are greedy decode step i + 1
    counts = list(g["spec_counts"])
    if all(c == 1 for c in counts):
        assert list(g["spec_digests"]) == list(g["greedy_digests"][1:1 + len(counts)])
    assert np.isfinite(g["hidden_l1"]).all() and np.isfinite(g["hidden_l4"]).all()
    assert len(set(greedy)) > 1
