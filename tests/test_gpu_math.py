"""Device math of the kernels (qwen3.8-27b-in-c_amd/csrc/q38_math.h,
q38_libm.h) on the GPU, through the test-only probe tests/native/libq38probe.so.

* q38_expf / q38_logf over all 2^32 inputs: the device checksum equals the one
  the host forms with the C library's expf / logf (tests/native/libm_check.c),
  which the reference calls (src/qwen38/qwen38_model.c:439, 444, 554, 771, 867).
* sqrt and division: correctly rounded, compared with numpy float32 (IEEE).
* sigmoid / SiLU / softplus: the reference's formulas, one rounding per step.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE = os.path.join(ROOT, "tests", "native", "libq38probe.so")
OP_EXP, OP_LOG, OP_SQRT, OP_DIV, OP_SIGMOID, OP_SILU, OP_SOFTPLUS = range(7)


@pytest.fixture(scope="module")
def probe(device):
    if not os.path.exists(PROBE):
        raise RuntimeError("tests/native/libq38probe.so not built (make -C tests/native)")
    lib = ctypes.CDLL(PROBE)
    lib.probe_eval.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
    lib.probe_checksum.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_uint64)]
    return lib


def evaluate(probe, op, x, y=None):
    import torch
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    yd = None if y is None else torch.from_numpy(np.ascontiguousarray(y, np.float32)).cuda()
    out = torch.empty_like(xd)
    assert probe.probe_eval(op, out.data_ptr(), xd.data_ptr(), 0 if yd is None else yd.data_ptr(), xd.numel())
    return out.cpu().numpy()


def host_checksums(tmp_path):
    exe = str(tmp_path / "libm_check")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off",
                    "-I", os.path.join(ROOT, "qwen3.8-27b-in-c_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "libm_check.c"), "-o", exe, "-lm"], check=True)
    out = subprocess.run([exe, "checksum"], check=True, capture_output=True, text=True).stdout.split()
    return {out[0]: int(out[2]), out[3]: int(out[5])}


def test_expf_logf_match_host_libm_on_every_input(probe, tmp_path):
    want = host_checksums(tmp_path)
    for op, name in ((OP_EXP, "expf"), (OP_LOG, "logf")):
        got = ctypes.c_uint64(0)
        assert probe.probe_checksum(op, ctypes.byref(got))
        assert got.value == want[name], name


def special_and_random(count, seed, positive=False):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 1 << 32, count, dtype=np.uint64).astype(np.uint32)
    if positive:
        bits &= 0x7fffffff
    special = np.array([0.0, -0.0, 1.0, 2.0, 0.5, 1e-45, 1e-38, 3.4e38, np.inf, -np.inf, 1e-6, 128.0, 256.0],
                       np.float32)
    return np.concatenate([special, bits.view(np.float32)])


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return np.all((a.view(np.uint32) == b.view(np.uint32)) | both_nan)


def test_sqrt_is_correctly_rounded(probe):
    x = special_and_random(1 << 22, 1, positive=True)
    with np.errstate(invalid="ignore"):
        assert same(evaluate(probe, OP_SQRT, x), np.sqrt(x))


def test_division_is_correctly_rounded(probe):
    x = special_and_random(1 << 22, 2)
    y = special_and_random(1 << 22, 3)
    with np.errstate(all="ignore"):
        assert same(evaluate(probe, OP_DIV, x, y), x / y)


def test_sigmoid_silu_softplus_follow_the_reference_formulas(probe):
    x = np.concatenate([np.linspace(-30, 30, 200001, dtype=np.float32),
                        np.random.default_rng(4).normal(0, 4, 1 << 20).astype(np.float32)])
    e_neg = evaluate(probe, OP_EXP, -x)
    e_pos = evaluate(probe, OP_EXP, x)
    one = np.float32(1.0)
    with np.errstate(all="ignore"):
        assert same(evaluate(probe, OP_SIGMOID, x), one / (one + e_neg))          # :437-440
        assert same(evaluate(probe, OP_SILU, x), x / (one + e_neg))               # :442-445
        log1p_e = evaluate(probe, OP_LOG, one + e_pos)
        assert same(evaluate(probe, OP_SOFTPLUS, x), np.where(x > 20, x, log1p_e))  # :551-555
