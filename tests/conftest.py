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


@pytest.fixture(scope="session")
def model_gguf():
    """Path of the synthetic 27B-shaped Q4_K_M GGUF (seed 1), written by
    qwen3.8-27b-in-c_amd/synth/q38_synth_gguf when missing (about 15.7 GB)."""
    from q38hip import synth
    path = synth.model_path(MODEL_SEED, "q4km")
    if path is None:
        pytest.skip("no directory with 17 GB free for the synthetic model")
    print("synthetic model:", path, flush=True)
    return synth.write_model_gguf(path, MODEL_SEED, "q4km")
