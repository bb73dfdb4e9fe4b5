"""Every other matrix format of the reference model on the GPU against the
oracle (oracle/q38_oracle_formats.c, pinned to the compiled reference by
tests/test_formats_oracle.py) and, where it was built, the compiled
reference itself.  Bar: bit-identical fp32 outputs.

  - Q8_K path (q38hip_gemm_q8_k): Q2_K, Q3_K, Q5_K, IQ2_XXS, IQ2_XS, IQ2_S,
    IQ3_XXS, IQ3_S, IQ4_XS, IQ4_NL, IQ1_S at ragged row counts, widths 256 ..
    17408 and 1..12 tokens, plus the reference's known-answer blocks through
    the host drop-in q38_tensor_gemv_q8_k;
  - float path (q38hip_gemm_f32, q38_tensor_gemv_f32): F32, F16, BF16, Q8_0,
    IQ4_NL and the K-quants against fp32 input, and NaN rows for the types
    the reference's float dot does not know;
  - row decode (q38hip_row_f32, q38_tensor_row_f32).
"""
import ctypes

import numpy as np
import pytest

import format_cases as fc
from oracle import F32_FORMATS, FORMAT_NAMES, IQ1_S, IQ2_XXS, IQ4_NL, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8K_FORMATS

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

NEW_Q8K = [t for t in Q8K_FORMATS if t not in (Q4_K, Q6_K, 29)]
FLOAT_DOT = list(F32_FORMATS) + [Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def to_dev(array, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


@pytest.mark.parametrize("qtype", NEW_Q8K, ids=lambda t: FORMAT_NAMES[t])
def test_q8k_formats_match_oracle(device, oracle, qtype):
    import q38hip
    rng = np.random.default_rng(300 + qtype)
    for rows, width in ((9, 256), (77, 1280), (1000, 5120), (333, 17408)):
        data = fc.random_matrix(qtype, rows, width, rng)
        x = rng.standard_normal((12, width)).astype(np.float32)
        q8 = oracle.quantize(x.reshape(-1))
        nb = width // 256
        want = np.stack([oracle.gemv(qtype, data, rows, q8[t * nb:(t + 1) * nb]) for t in range(12)])
        w_dev = to_dev(data, device)
        q8_dev = to_dev(q8.view(np.uint8), device)
        for batch in (1, 2, 3, 5, 8, 12):
            print(FORMAT_NAMES[qtype], rows, width, batch, flush=True)
            got = q38hip.gemm_q8_k(w_dev, qtype, width, rows, q8_dev[:batch * nb * 292], batch).cpu().numpy()
            assert np.array_equal(bits(got), bits(want[:batch])), (rows, width, batch)


def test_q8k_formats_match_compiled_reference(device, oracle, reference):
    import q38hip
    rng = np.random.default_rng(17)
    for qtype in NEW_Q8K:
        rows, width = 64, 2560
        data = fc.random_matrix(qtype, rows, width, rng)
        q8 = oracle.quantize(rng.standard_normal(5 * width).astype(np.float32))
        want = reference.gemm(qtype, data, rows, q8, 5)
        got = q38hip.gemm_q8_k(to_dev(data, device), qtype, width, rows, to_dev(q8.view(np.uint8), device), 5)
        assert np.array_equal(bits(got.cpu().numpy()), bits(want)), FORMAT_NAMES[qtype]


def test_known_blocks_through_host_drop_in(device, oracle):
    import q38hip
    lib = q38hip.lib()
    q8 = oracle.quantize(np.ones(256, np.float32))
    for qtype, block, expected in fc.known_integer_blocks():
        tensor = q38hip.make_tensor(block.ctypes.data, qtype, 256, 1, block.nbytes)
        out = np.zeros(1, np.float32)
        assert lib.q38_tensor_gemv_q8_k(out.ctypes.data, q8.ctypes.data, 256, ctypes.byref(tensor)), \
            q38hip.last_error()
        assert out[0] == expected, FORMAT_NAMES[qtype]
    for qtype, block, width, expected in fc.known_float_blocks():
        tensor = q38hip.make_tensor(block.ctypes.data, qtype, width, 1, block.nbytes)
        out = np.zeros(1, np.float32)
        x = np.ones(width, np.float32)
        assert lib.q38_tensor_gemv_f32(out.ctypes.data, x.ctypes.data, ctypes.byref(tensor)), q38hip.last_error()
        assert out[0] == expected, FORMAT_NAMES[qtype]


@pytest.mark.parametrize("qtype", FLOAT_DOT, ids=lambda t: FORMAT_NAMES[t])
def test_float_path_matches_oracle(device, oracle, qtype):
    import q38hip
    rng = np.random.default_rng(400 + qtype)
    for rows, width in ((5, 256), (300, 1280), (40, 5120)):
        data = fc.random_matrix(qtype, rows, width, rng)
        x = rng.standard_normal((6, width)).astype(np.float32)
        want = np.stack([oracle.gemv_f32(qtype, data, rows, x[t]) for t in range(6)])
        print(FORMAT_NAMES[qtype], rows, width, flush=True)
        got = q38hip.gemm_f32(to_dev(data, device), qtype, width, rows, to_dev(x, device)).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), (rows, width)


@pytest.mark.parametrize("qtype", FLOAT_DOT, ids=lambda t: FORMAT_NAMES[t])
def test_row_decode_matches_oracle(device, oracle, qtype):
    import q38hip
    rng = np.random.default_rng(500 + qtype)
    rows, width = 37, 1280
    data = fc.random_matrix(qtype, rows, width, rng)
    got = q38hip.row_f32(to_dev(data, device), qtype, width, rows, 3, 30).cpu().numpy()
    for r in range(30):
        assert np.array_equal(bits(got[r]), bits(oracle.format_row_f32(qtype, data, width, 3 + r))), r


def test_row_decode_non_finite_weights(device, oracle):
    """a block with an infinite scale: its other elements' unit-basis dots
    meet inf * 0 and become NaN"""
    import q38hip
    rng = np.random.default_rng(5)
    data = fc.random_matrix(Q3_K, 2, 512, rng)
    data[108:110] = np.array([0x00, 0x7C], np.uint8)   # d = +inf in block 0 of row 0
    got = q38hip.row_f32(to_dev(data, device), Q3_K, 512, 2, 0, 2).cpu().numpy()
    for r in range(2):
        assert np.array_equal(bits(got[r]), bits(oracle.format_row_f32(Q3_K, data, 512, r)))
    assert np.isnan(got[0, :256]).any()


def test_types_without_float_dot_give_nan(device, oracle, reference):
    """q38_tensor_gemv_f32 / q38_tensor_row_f32 on an IQ type: the
    reference's float dot has no case for it and writes NaN"""
    import q38hip
    rng = np.random.default_rng(6)
    for qtype in (IQ2_XXS, IQ1_S):
        data = fc.random_matrix(qtype, 4, 256, rng)
        x = rng.standard_normal(256).astype(np.float32)
        got = q38hip.gemm_f32(to_dev(data, device), qtype, 256, 4, to_dev(x, device)).cpu().numpy()
        want = reference.gemv_f32(qtype, data, 4, x)
        assert np.array_equal(bits(got[0]), bits(want))
        row = q38hip.row_f32(to_dev(data, device), qtype, 256, 4, 1).cpu().numpy()
        assert np.array_equal(bits(row[0]), bits(reference.row_f32(qtype, data, 256, 1, 4)))
