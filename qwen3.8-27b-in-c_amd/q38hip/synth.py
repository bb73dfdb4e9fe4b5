"""Seeded synthetic GGUF-layout weights and activations.

Every generator takes an explicit seed and uses numpy's PCG64, so the same
bytes are produced on any host.  Layouts are the GGUF block formats the
engine reads (shape[0] = input width, shape[1] = output rows):

* Q4_K  144-byte super-blocks: fp16 d @0, fp16 dmin @2, 12 bytes of packed
  6-bit scales/mins @4, 128 bytes of nibbles @16
  (third_party/ggml-common.h:327-338 of the reference).
* IQ1_M 56-byte blocks: qs[32] @0, qh[16] @32, scales[8] @48 with the fp16
  super-scale in bits 12..15 of the four u16 (ggml-common.h:431-443).
* Q6_K  210-byte blocks: ql[128] @0, qh[64] @128, int8 scales[16] @192,
  fp16 d @208 (ggml-common.h:362-368).
"""
import os

import numpy as np

Q4_K, Q6_K, IQ1_M = 12, 14, 29
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, IQ1_M: 56}


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _abs_normal_f16_bits(rng, count, sigma):
    values = np.abs(rng.normal(0.0, sigma, size=count)).astype(np.float16)
    return values.view(np.uint16)


def q4k_matrix(rows, width, seed, sigma=0.01):
    """Q4_K matrix: d, dmin = fp16(|N(0, sigma)|); scale and quant bytes uniform."""
    assert width % 256 == 0
    nb = width // 256
    rng = _rng(seed)
    blocks = rng.integers(0, 256, size=(rows * nb, 144), dtype=np.uint8)
    d = _abs_normal_f16_bits(rng, rows * nb, sigma)
    dmin = _abs_normal_f16_bits(rng, rows * nb, sigma)
    blocks[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:4] = dmin.view(np.uint8).reshape(-1, 2)
    return blocks.reshape(-1)


def iq1m_matrix(rows, width, seed, sigma=0.01):
    """IQ1_M matrix: qs, qh uniform; 3-bit sub-scales uniform; fp16 super-scale
    |N(0, sigma)| split over bits 12..15 of the four packed-scale u16."""
    assert width % 256 == 0
    nb = width // 256
    rng = _rng(seed)
    blocks = rng.integers(0, 256, size=(rows * nb, 56), dtype=np.uint8)
    sub = rng.integers(0, 1 << 12, size=(rows * nb, 4), dtype=np.uint16)
    scale = _abs_normal_f16_bits(rng, rows * nb, sigma)
    packed = np.empty((rows * nb, 4), dtype=np.uint16)
    for j in range(4):
        packed[:, j] = sub[:, j] | (((scale >> (4 * j)) & 0xF) << 12)
    blocks[:, 48:56] = packed.astype("<u2").view(np.uint8).reshape(-1, 8)
    return blocks.reshape(-1)


def q6k_matrix(rows, width, seed, sigma=0.01):
    """Q6_K matrix: quant bytes uniform, int8 sub-scales uniform, d = fp16(|N(0, sigma)|)."""
    assert width % 256 == 0
    nb = width // 256
    rng = _rng(seed)
    blocks = rng.integers(0, 256, size=(rows * nb, 210), dtype=np.uint8)
    d = _abs_normal_f16_bits(rng, rows * nb, sigma)
    blocks[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return blocks.reshape(-1)


def matrix(qtype, rows, width, seed, sigma=0.01):
    if qtype == Q4_K:
        return q4k_matrix(rows, width, seed, sigma)
    if qtype == IQ1_M:
        return iq1m_matrix(rows, width, seed, sigma)
    if qtype == Q6_K:
        return q6k_matrix(rows, width, seed, sigma)
    raise ValueError("unsupported type %r" % qtype)


def activations(width, seed, count=1):
    """fp32 rows ~ N(0, 1), shape [count, width]."""
    return _rng(seed).normal(0.0, 1.0, size=(count, width)).astype(np.float32)


SYNTH_GGUF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "synth", "q38_synth_gguf")
MODEL_GGUF_BYTES = {"q4km": 15709517280, "iq1m": 7193032160, "accept": 15470533184, "accept_mtp": 2001697184,
                    "accept_all": 15709517280, "mixed": 13757834720}


def write_model_gguf(path, seed, variant="q4km"):
    """Write the deterministic synthetic 27B-shaped GGUF (synth/q38_synth_gguf.c)
    to `path` unless a file of the expected size is already there.  Variants:
    q4km, iq1m, mixed (every other matrix format), and the checkpoint pair
    accept (64 blocks, an LM head with two live rows) + accept_mtp (its
    separate MTP block), and accept_all (the q4km file with every LM head
    row equal to row 0, so every draft is accepted)."""
    import subprocess
    expected = MODEL_GGUF_BYTES.get(variant)
    if expected and os.path.exists(path) and os.path.getsize(path) == expected:
        return path
    if not os.path.exists(SYNTH_GGUF):
        raise RuntimeError("synthetic GGUF writer not built: make -C qwen3.8-27b-in-c_amd")
    subprocess.run([SYNTH_GGUF, path, str(seed), variant], check=True)
    return path


def model_path(seed, variant="q4km"):
    """Where the synthetic model of `seed` lives (or will be written): a file
    q38_<variant>_s<seed>.gguf in $Q38_MODEL_DIR, /dev/shm or the system
    temporary directory, the first with room for it.  None if none has."""
    import shutil
    import tempfile
    need = MODEL_GGUF_BYTES.get(variant, 16 << 30)
    name = "q38_%s_s%d.gguf" % (variant, seed)
    for d in (os.environ.get("Q38_MODEL_DIR"), "/dev/shm", tempfile.gettempdir()):
        if d and os.path.isdir(d) and os.access(d, os.W_OK):
            path = os.path.join(d, name)
            if os.path.exists(path) or shutil.disk_usage(d).free > need + (2 << 30):
                return path
    return None
