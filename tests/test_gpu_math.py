"""Device math of the kernels (qwen3.8-27b-in-c_amd/csrc/q38_math.h,
q38_libm.h) on the GPU, through the test-only probe tests/native/libq38probe.so.

* q38_expf / q38_logf over all 2^32 inputs: the device checksum equals the one
  the host forms with the C library's expf / logf (tests/native/libm_check.c),
  which the reference calls (src/qwen38/qwen38_model.c:439, 444, 554, 771, 867).
* sqrt and division: correctly rounded, compared with numpy float32 (IEEE).
* sigmoid / SiLU / softplus: the reference's formulas, one rounding per step.
* the RMSNorm mean of squares (q38_norm.h), including its sequential redo
  near a float rounding boundary.
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
    lib.probe_mean_square.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
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


def _mean_square(probe, x):
    import torch
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    out = torch.empty(1, dtype=torch.float32, device="cuda")
    assert probe.probe_mean_square(xd.data_ptr(), xd.numel(), out.data_ptr())
    return out.cpu().numpy()[0]


def _reference_mean_square(x):
    """The reference's RMSNorm mean: sum += (double)(x[i] * x[i]) in order,
    then (float)(sum / n) (src/qwen38/qwen38_model.c:426-435)."""
    sq = (x.astype(np.float32) * x.astype(np.float32)).astype(np.float32)
    s = 0.0
    for v in sq.tolist():
        s += v
    return np.float32(s / len(x))


def _takes_sequential_redo(x):
    """Whether the kernels' parallel sum is within 2^-36 of a float rounding
    boundary of sum / n, so that q38_norm.h redoes the sum in order (the
    constructed sums below are exact in double, so any summation order gives
    this total)."""
    sq = (x.astype(np.float32) * x.astype(np.float32)).astype(np.float64)
    total = float(np.sum(sq))
    n = float(len(x))
    return np.float32((total * (1.0 - 2.0 ** -36)) / n) != np.float32((total * (1.0 + 2.0 ** -36)) / n)


def test_rmsnorm_mean_sequential_redo(probe):
    """The RMSNorm mean of squares (q38_norm.h block_sum_squares, used by
    every norm kernel) equals the reference's sequential double sum, on
    vectors built so that sum / n lies exactly on a float rounding midpoint
    (ties to even one way and the other), which forces the kernels'
    sequential redo; on random vectors, which do not; and on a NaN."""
    xa = np.float32(1.0 + 1280 * 2.0 ** -23)   # xa * xa rounds to exactly 1 + 2560 * 2^-23
    assert np.float32(xa * xa) == np.float32(1.0 + 2560 * 2.0 ** -23)
    xb = np.float32(1.0 + 32 * 2.0 ** -23)     # xb * xb rounds to exactly 1 + 64 * 2^-23
    assert np.float32(xb * xb) == np.float32(1.0 + 64 * 2.0 ** -23)
    cases = []
    # mean = 1 + 2^-24: halfway between 1 and 1 + 2^-23, ties to 1
    a = np.ones(5120, np.float32)
    a[1234] = xa
    cases.append((a, True))
    # mean = 1 + 3 * 2^-24: halfway between 1 + 2^-23 and 1 + 2^-22, ties to 1 + 2^-22
    b = np.ones(5120, np.float32)
    b[[7, 2000, 5119]] = xa
    cases.append((b, True))
    # the same midpoint over the 128-wide L2-norm length
    c = np.ones(128, np.float32)
    c[99] = xb
    cases.append((c, True))
    # negative values square the same way
    d = -a
    cases.append((d, True))
    rng = np.random.default_rng(5)
    for n in (5120, 128, 6144):
        cases.append((rng.standard_normal(n).astype(np.float32), False))
    for x, redo in cases:
        assert _takes_sequential_redo(x) == redo
        got = _mean_square(probe, x)
        want = _reference_mean_square(x)
        assert np.float32(got).view(np.uint32) == want.view(np.uint32), (len(x), got, want)
    assert _reference_mean_square(a) == np.float32(1.0)
    assert _reference_mean_square(b) == np.float32(1.0 + 2.0 ** -22)
    nan = np.ones(5120, np.float32)
    nan[17] = np.nan
    assert np.isnan(_mean_square(probe, nan))
