"""Pins for the oracle's restatement of every other matrix format
(oracle/q38_oracle_formats.c), CPU only.

  (1) the reference's own known answers (tests/unit/test_qwen38_quant.c:
      467-488, 736-900), through the Q8_K GEMV and the float GEMV;
  (2) the integer definition of each format: the eight AVX2 lanes sum to
      sum_e s16[e / 16] * q[e] * a[e] over the decoded integer weights,
      and the float path's row decode equals d * s16 * q (- min) element by
      element for the K-quants;
  (3) the compiled reference (oracle/_ref) on seeded random matrices: the
      Q8_K GEMV and GEMM (its 4-token tiles), the float GEMV and the row
      decode, compared as uint32;
  (4) the grid codebooks: csrc/q38_iq_grids.inc regenerates byte for byte
      from the reference's ggml-common.h when it is present, and its
      expanded tables carry the SHA-256 recorded in its header.
"""
import hashlib
import os
import re

import numpy as np
import pytest

import format_cases as fc
from oracle import (F32_FORMATS, FORMAT_NAMES, IQ1_S, IQ4_NL, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0,
                    Q8K_FORMATS)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GRIDS_INC = os.path.join(ROOT, "qwen3.8-27b-in-c_amd", "csrc", "q38_iq_grids.inc")
NEW_Q8K = [t for t in Q8K_FORMATS if t not in (Q4_K, Q6_K, 29)]
FLOAT_DOT = list(F32_FORMATS) + [Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("case", fc.known_integer_blocks(), ids=lambda c: FORMAT_NAMES[c[0]])
def test_known_integer_blocks(oracle, case):
    qtype, block, expected = case
    q8 = oracle.quantize(np.ones(256, np.float32))
    assert oracle.gemv(qtype, block, 1, q8)[0] == expected


@pytest.mark.parametrize("case", fc.known_float_blocks(), ids=lambda c: FORMAT_NAMES[c[0]])
def test_known_float_blocks(oracle, case):
    qtype, block, width, expected = case
    assert oracle.gemv_f32(qtype, block, 1, np.ones(width, np.float32))[0] == expected
    if qtype != Q8_0:
        q8 = oracle.quantize(np.ones(256, np.float32))
        assert oracle.gemv(qtype, block, 1, q8)[0] == expected


@pytest.mark.parametrize("qtype", NEW_Q8K, ids=lambda t: FORMAT_NAMES[t])
def test_lanes_sum_to_integer_definition(oracle, qtype):
    rng = np.random.default_rng(qtype)
    for _ in range(20):
        block = fc.random_matrix(qtype, 1, 256, rng)
        q8 = oracle.quantize(rng.standard_normal(256).astype(np.float32))
        lanes, extra = oracle.block_lanes(qtype, block, q8)
        q, s16 = oracle.block_decode(qtype, block)
        a = q8["quants"][0].astype(np.int64)
        assert int(lanes.astype(np.int64).sum()) == int((np.repeat(s16, 16) * q * a).sum())
        # lane l only sees bytes 4l..4l+3 of each 32-element group
        for lane in range(8):
            idx = np.array([32 * g + 4 * lane + t for g in range(8) for t in range(4)])
            assert lanes[lane] == int((np.repeat(s16, 16)[idx] * q[idx] * a[idx]).sum())
        sums = q8["sums"][0].astype(np.int64)
        if qtype == Q2_K:
            assert extra == int(((block[:16] >> 4).astype(np.int64) * sums).sum())
        if qtype == IQ1_S:
            high = block[34:50].view(np.uint16).astype(np.int64)
            scale = 1 + 2 * ((high >> 12) & 7)
            sign = np.where(high & 0x8000, -1, 1)
            assert extra == int((scale * sign * (sums[0::2] + sums[1::2])).sum())


def test_row_decode_closed_form(oracle):
    """K-quant and Q8_0 rows decode to the weight expressions of the float
    dots: Q4_K (d*sc)*q - dmin*m, Q3_K (d*sc)*q, Q8_0 d*q."""
    rng = np.random.default_rng(9)
    q4 = fc.random_matrix(Q4_K, 1, 256, rng)
    row = oracle.format_row_f32(Q4_K, q4, 256, 0)
    assert np.array_equal(bits(row), bits(oracle.row_f32(Q4_K, q4, 256, 0)))
    q3 = fc.random_matrix(Q3_K, 1, 256, rng)
    q, s16 = oracle.block_decode(Q3_K, q3)
    d = np.float32(np.frombuffer(q3[108:110].tobytes(), np.float16)[0])
    want = (d * np.repeat(s16, 16).astype(np.float32)) * q.astype(np.float32)
    want[want == 0] = 0.0
    assert np.array_equal(bits(oracle.format_row_f32(Q3_K, q3, 256, 0)), bits(want))
    q8 = fc.random_matrix(Q8_0, 1, 64, rng)
    blocks = q8.reshape(2, 34)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(2, 1)
    want = (d * blocks[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)
    want[want == 0] = 0.0
    assert np.array_equal(bits(oracle.format_row_f32(Q8_0, q8, 64, 0)), bits(want))


@pytest.mark.parametrize("qtype", Q8K_FORMATS, ids=lambda t: FORMAT_NAMES[t])
def test_q8k_gemv_and_gemm_match_compiled_reference(oracle, reference, qtype):
    rng = np.random.default_rng(100 + qtype)
    for rows, width in ((9, 256), (5, 1280), (3, 5120)):
        data = fc.random_matrix(qtype, rows, width, rng)
        x = rng.standard_normal((6, width)).astype(np.float32)
        q8 = oracle.quantize(x.reshape(-1))
        assert np.array_equal(bits(oracle.gemv(qtype, data, rows, q8[:width // 256])),
                              bits(reference.gemv(qtype, data, rows, q8[:width // 256])))
        # the reference's GEMM runs 4-token tiles and a 2..3-token tail
        for batch in (2, 5, 6):
            got = oracle.gemm(qtype, data, rows, q8[:batch * width // 256], batch) if qtype in (Q4_K, Q6_K, 29) \
                else np.stack([oracle.gemv(qtype, data, rows, q8[t * width // 256:(t + 1) * width // 256])
                               for t in range(batch)])
            want = reference.gemm(qtype, data, rows, q8[:batch * width // 256], batch)
            assert np.array_equal(bits(got), bits(want)), (rows, width, batch)


@pytest.mark.parametrize("qtype", FLOAT_DOT, ids=lambda t: FORMAT_NAMES[t])
def test_float_gemv_and_row_match_compiled_reference(oracle, reference, qtype):
    rng = np.random.default_rng(200 + qtype)
    for rows, width in ((4, 256), (3, 1280)):
        data = fc.random_matrix(qtype, rows, width, rng)
        x = rng.standard_normal(width).astype(np.float32)
        assert np.array_equal(bits(oracle.gemv_f32(qtype, data, rows, x)),
                              bits(reference.gemv_f32(qtype, data, rows, x)))
        for row in (0, rows - 1):
            assert np.array_equal(bits(oracle.format_row_f32(qtype, data, width, row)),
                                  bits(reference.row_f32(qtype, data, width, row, rows)))


def _expand_grids(text):
    """byte tables of q38_iq_grids.inc, in its header's order"""
    tables = []
    for name, width, bits_per, levels in (("IQ2XXS", 8, 2, (8, 25, 43)), ("IQ2XS", 8, 2, (8, 25, 43)),
                                          ("IQ2S", 8, 2, (8, 25, 43)),
                                          ("IQ3XXS", 4, 3, (4, 12, 20, 28, 36, 44, 52, 62)),
                                          ("IQ3S", 4, 3, tuple(range(1, 16, 2)))):
        body = re.search(r"#define Q38_%s_CODES\(X\)(.*?)(?:\n\n|\Z)" % name, text, re.S).group(1)
        codes = [int(c, 16) for c in re.findall(r"X\(0x([0-9a-f]+)\)", body)]
        mask = (1 << bits_per) - 1
        tables.append(bytes(levels[(c >> (bits_per * k)) & mask] for c in codes for k in range(width)))
    values = [int(v) for v in re.search(r"#define Q38_IQ4NL_VALUES (.*)", text).group(1).split(",")]
    return tables, bytes(v & 0xFF for v in values)


def test_grid_tables_pinned():
    text = open(GRIDS_INC).read()
    tables, values = _expand_grids(text)
    assert [len(t) for t in tables] == [2048, 4096, 8192, 1024, 2048]
    digest = hashlib.sha256(b"".join(tables) + values).hexdigest()
    assert re.search(r"\*   ([0-9a-f]{64})", text).group(1) == digest


def test_grid_tables_regenerate_from_reference_header():
    import gen_iq_grids
    if not os.path.exists(gen_iq_grids.HEADER):
        pytest.skip("reference header not present")
    grids, values, _ = gen_iq_grids.read_reference_tables()
    tables, packed_values = _expand_grids(open(GRIDS_INC).read())
    for (name, width, count, _, _), table in zip(gen_iq_grids.GRIDS, tables):
        assert bytes(b for entry in grids[name] for b in entry) == table, name
    assert bytes(v & 0xFF for v in values) == packed_values
