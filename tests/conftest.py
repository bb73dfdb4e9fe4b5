import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "qwen3.8-27b-in-c_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle import Reference
    if not Reference.available():
        pytest.skip("reference library oracle/_ref not built (needs the reference sources)")
    return Reference()


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test run without a visible GPU")
    return torch.device("cuda:0")


MODEL_SEED = 1


def synthetic_model(variant):
    """Path of the synthetic 27B-shaped GGUF of `variant` (seed 1; q4km about
    15.7 GB, iq1m about 7.2 GB), written by
    qwen3.8-27b-in-c_amd/synth/q38_synth_gguf when missing."""
    from q38hip import synth
    path = synth.model_path(MODEL_SEED, variant)
    if path is None:
        pytest.skip("no directory with room for the synthetic %s model" % variant)
    print("synthetic model:", path, flush=True)
    return synth.write_model_gguf(path, MODEL_SEED, variant)

