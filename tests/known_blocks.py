"""Known-answer inputs of the reference's own kernel tests
(tests/unit/test_qwen38_quant.c of shyringo/qwen3.8-27b-in-c), rebuilt as
numpy arrays, plus the reference's LCG and random-block helpers."""
import numpy as np

Q4_K, Q6_K, IQ1_M = 12, 14, 29


def lcg(state):
    """x = x * 1664525 + 1013904223 (test_qwen38_quant.c:34-38)."""
    state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
    return state, state


def set_half(block, offset, value):
    block[offset] = value & 0xFF
    block[offset + 1] = (value >> 8) & 0xFF


def set_block_scales(block, qtype, scale, minimum):
    """set_random_block_scales (test_qwen38_quant.c:40-80) for our types."""
    if qtype == Q4_K:
        set_half(block, 0, scale)
        set_half(block, 2, minimum)
    elif qtype == Q6_K:
        set_half(block, 208, scale)
    elif qtype == IQ1_M:
        set_half(block, 48, (scale & 0x000F) << 12)
        set_half(block, 50, (scale & 0x00F0) << 8)
        set_half(block, 52, (scale & 0x0F00) << 4)
        set_half(block, 54, scale & 0xF000)


def q4k_known_block():
    """Q4_K block whose dot with all-ones is 64.0 (test_qwen38_quant.c:794-800)."""
    q4 = np.zeros(144, dtype=np.uint8)
    set_half(q4, 0, 0x3C00)
    set_half(q4, 2, 0x3800)
    q4[4:8] = 1
    q4[8:12] = 2
    q4[16:144] = 0x21
    return q4


def iq1m_known_block():
    """IQ1_M block whose dot with all-ones is -224.0 (test_qwen38_quant.c:467-489, 882-883)."""
    blk = np.zeros(56, dtype=np.uint8)
    set_block_scales(blk, IQ1_M, 0x3C00, 0)
    return blk


def q6k_known_block():
    """Q6_K block whose dot with all-ones is -8192.0 (test_qwen38_quant.c:838-841)."""
    q6 = np.zeros(210, dtype=np.uint8)
    q6[192:208] = 1
    set_half(q6, 208, 0x3C00)
    return q6


def random_iq_trials(qtype, nbytes, trials=200):
    """Blocks and activations of test_iq_kernel (test_qwen38_quant.c:337-372):
    random bytes, scale 0x34cd, activation ((r >> 20) - 2048) / (89 + i % 13)."""
    state = (0xF012CA65 + qtype) & 0xFFFFFFFF
    out = []
    for _ in range(trials):
        data = np.zeros(nbytes, dtype=np.uint8)
        for i in range(nbytes):
            state, r = lcg(state)
            data[i] = r >> 24
        set_block_scales(data, qtype, 0x34CD, 0)
        act = np.zeros(256, dtype=np.float32)
        for i in range(256):
            state, r = lcg(state)
            act[i] = np.float32((r >> 20) - 2048) / np.float32(89 + i % 13)
        out.append((data, act))
    return out


def batch_exact_case(qtype, block_bytes):
    """Inputs of test_integer_batch_exact (test_qwen38_quant.c:637-684):
    WIDTH 512, ROWS 3, up to 5 tokens."""
    width, rows, tokens = 512, 3, 5
    state = (0x91E10DA5 + qtype) & 0xFFFFFFFF
    weights = np.zeros(rows * 2 * block_bytes, dtype=np.uint8)
    for i in range(weights.size):
        state, r = lcg(state)
        weights[i] = r >> 24
    for row in range(rows):
        for block in range(2):
            view = weights[(row * 2 + block) * block_bytes:(row * 2 + block + 1) * block_bytes]
            set_block_scales(view, qtype, 0x2800 + row * 0x80 + block, 0x2400 + row * 0x40 + block)
    act = np.zeros(tokens * width, dtype=np.float32)
    for i in range(act.size):
        state, r = lcg(state)
        act[i] = np.float32((r >> 19) - 4096) / np.float32(101 + (i % 7))
    return weights, act, width, rows, tokens
