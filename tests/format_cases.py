"""Random GGUF matrices of every format the reference model accepts, and the
reference's known-answer blocks (tests/unit/test_qwen38_quant.c:467-488,
736-900).

Random matrices are random bytes with every fp16 scale field overwritten by
a finite value of moderate size, so that dot products stay finite and
exercise every bit of the packed fields (signs, grid indices, high bits,
sub-block scales).
"""
import numpy as np

from oracle import (BF16, F16, F32, FORMATS, IQ1_M, IQ1_S, IQ2_S, IQ2_XS, IQ2_XXS, IQ3_S, IQ3_XXS, IQ4_NL,
                    IQ4_XS, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0)

# byte offsets of the fp16 scale fields inside one block
SCALE_FIELDS = {Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,), IQ2_XXS: (0,),
                IQ2_XS: (0,), IQ2_S: (0,), IQ3_XXS: (0,), IQ3_S: (0,), IQ4_XS: (0,), IQ4_NL: (0,), IQ1_S: (0,),
                Q8_0: (0,)}


def random_halves(rng, count, lo=1e-3, hi=4e-2):
    values = rng.uniform(lo, hi, size=count) * rng.choice([-1.0, 1.0], size=count, p=[0.1, 0.9])
    return values.astype(np.float16).view(np.uint16)


def random_matrix(qtype, rows, width, rng):
    """uint8 [rows * row_bytes] of `qtype`."""
    elements, nbytes = FORMATS[qtype]
    blocks = rows * (width // elements)
    if qtype == F32:
        return rng.standard_normal(rows * width).astype(np.float32).view(np.uint8).copy()
    if qtype == F16:
        return (rng.standard_normal(rows * width) * 0.05).astype(np.float16).view(np.uint8).copy()
    if qtype == BF16:
        bits = (rng.standard_normal(rows * width) * 0.05).astype(np.float32).view(np.uint32) >> 16
        return bits.astype(np.uint16).view(np.uint8).copy()
    data = rng.integers(0, 256, size=(blocks, nbytes), dtype=np.uint8)
    if qtype == IQ1_M:
        # the fp16 scale is spread over the high nibbles of bytes 48..55
        halves = random_halves(rng, blocks, 1e-2, 5e-2).astype(np.uint32)
        for k in range(4):
            word = data[:, 48 + 2 * k].astype(np.uint32) | data[:, 49 + 2 * k].astype(np.uint32) << 8
            word = (word & 0x0FFF) | (((halves >> (4 * k)) & 0xF) << 12)
            data[:, 48 + 2 * k] = word & 0xFF
            data[:, 49 + 2 * k] = word >> 8
        return data.reshape(-1)
    for offset in SCALE_FIELDS[qtype]:
        halves = random_halves(rng, blocks)
        data[:, offset] = halves & 0xFF
        data[:, offset + 1] = halves >> 8
    return data.reshape(-1)


def set_half(block, offset, value):
    block[offset] = value & 0xFF
    block[offset + 1] = value >> 8


def known_integer_blocks():
    """test_iq_known_block (:467-488): d = 1.0, every other byte zero, all
    activations 1.0 -> (qtype, block, expected GEMV value)."""
    expected = {IQ2_XXS: 256.0, IQ2_XS: 256.0, IQ3_XXS: 256.0, IQ3_S: 256.0, IQ4_XS: 1040384.0,
                IQ4_NL: -32512.0, IQ1_S: -224.0}
    out = []
    for qtype, value in expected.items():
        block = np.zeros(144, np.uint8)
        if qtype == IQ4_NL:
            for g in range(8):
                set_half(block, 18 * g, 0x3C00)
        else:
            set_half(block, 0, 0x3C00)
        out.append((qtype, block[:FORMATS[qtype][1] * (8 if qtype == IQ4_NL else 1)], value))
    return out


def known_float_blocks():
    """test_block calls of main (:780-847): (qtype, block, width, expected)
    for all-ones fp32 input; the K-quants also through the Q8_K GEMV."""
    q2 = np.zeros(84, np.uint8)
    q2[:16] = 0x01
    q2[16:80] = 0x55
    set_half(q2, 80, 0x3C00)
    q3 = np.zeros(110, np.uint8)
    q3[:32] = 0xFF
    q3[32:96] = 0x55
    q3[96:104] = 0x11
    q3[104:108] = 0xAA
    set_half(q3, 108, 0x3C00)
    q4 = np.zeros(144, np.uint8)
    set_half(q4, 0, 0x3C00)
    set_half(q4, 2, 0x3800)
    q4[4:8] = 1
    q4[8:12] = 2
    q4[16:] = 0x21
    q5 = np.zeros(176, np.uint8)
    set_half(q5, 0, 0x3C00)
    set_half(q5, 2, 0x3800)
    q5[4:8] = 1
    q5[8:12] = 2
    q5[48:] = 0x21
    q6 = np.zeros(210, np.uint8)
    q6[192:208] = 1
    set_half(q6, 208, 0x3C00)
    q8 = np.zeros(34, np.uint8)
    set_half(q8, 0, 0x3800)
    q8[2:] = 2
    return [(Q2_K, q2, 256, 256.0), (Q3_K, q3, 256, 256.0), (Q4_K, q4, 256, 64.0), (Q5_K, q5, 256, 64.0),
            (Q6_K, q6, 256, -8192.0), (Q8_0, q8, 32, 32.0)]
