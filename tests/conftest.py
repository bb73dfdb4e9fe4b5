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


def _model_dir(need_bytes):
    """A directory with room for the synthetic model: $Q38_MODEL_DIR, then
    /dev/shm, then the system temporary directory."""
    import shutil
    import tempfile
    candidates = [os.environ.get("Q38_MODEL_DIR"), "/dev/shm", tempfile.gettempdir()]
    for d in candidates:
        if d and os.path.isdir(d) and os.access(d, os.W_OK):
            existing = os.path.join(d, "q38_q4km_s%d.gguf" % MODEL_SEED)
            if os.path.exists(existing) or shutil.disk_usage(d).free > need_bytes + (2 << 30):
                return d
    return None


@pytest.fixture(scope="session")
def model_gguf():
    """Path of the synthetic 27B-shaped Q4_K_M GGUF (seed 1), written by
    qwen3.8-27b-in-c_amd/synth/q38_synth_gguf when missing (about 15.7 GB)."""
    from q38hip import synth
    need = synth.MODEL_GGUF_BYTES["q4km"]
    d = _model_dir(need)
    if d is None:
        pytest.skip("no directory with 17 GB free for the synthetic model")
    path = os.path.join(d, "q38_q4km_s%d.gguf" % MODEL_SEED)
    print("synthetic model:", path, flush=True)
    return synth.write_model_gguf(path, MODEL_SEED, "q4km")
