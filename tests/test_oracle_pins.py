"""Pins for the CPU oracle (oracle/q38_oracle.c), CPU only.

The oracle is checked against (1) the reference's own known-answer kernel
tests, (2) closed forms and brute force from the block formats, (3) the
committed golden vectors written by the compiled reference
(tests/golden/make_golden.py), and (4) when it was built here, the
compiled reference itself (oracle/_ref) on seeded random inputs.
"""
import hashlib
import os

import numpy as np
import pytest

import known_blocks as kb
from oracle import BLOCK_BYTES, IQ1_M, Q4_K, Q6_K, Q8K_DTYPE
from q38hip import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def close_to(actual, expected):
    """test_qwen38_quant.c:29-32"""
    return abs(actual - expected) <= 1e-5 * max(1.0, abs(expected))


# ---- (1) the reference's known answers ---------------------------------------

def test_f16_known_values(oracle):
    assert oracle.f16_to_f32(0x3C00) == 1.0
    assert oracle.f16_to_f32(0xC000) == -2.0
    assert oracle.f16_to_f32(0x0001) == 2.0 ** -24


def test_f16_exhaustive_matches_numpy(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    expected = bits.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32).view(np.uint32)
    nan = np.isnan(bits.view(np.float16))
    assert np.array_equal(got[~nan], expected[~nan])
    assert np.all(np.isnan(got[nan].view(np.float32)))


def test_q8k_signed_range(oracle):
    x = (np.arange(256, dtype=np.float32) - 128) / 128
    q = oracle.quantize(x)
    assert q["quants"][0, 0] == -127 and q["quants"][0, 128] == 0


def test_q4k_known_block(oracle):
    q = oracle.quantize(np.ones(256, dtype=np.float32))
    assert close_to(oracle.gemv(Q4_K, kb.q4k_known_block(), 1, q)[0], 64.0)


def test_q4k_known_batch_major(oracle):
    w = np.concatenate([kb.q4k_known_block(), kb.q4k_known_block()])
    x = np.concatenate([np.ones(256, np.float32), np.full(256, 2.0, np.float32)])
    out = oracle.gemm(Q4_K, w, 2, oracle.quantize(x), 2).reshape(-1)
    assert all(close_to(a, b) for a, b in zip(out, (64.0, 64.0, 128.0, 128.0)))


def test_iq1m_known_block(oracle):
    q = oracle.quantize(np.ones(256, dtype=np.float32))
    assert close_to(oracle.gemv(IQ1_M, kb.iq1m_known_block(), 1, q)[0], -224.0)


def test_q6k_known_block(oracle):
    q = oracle.quantize(np.ones(256, dtype=np.float32))
    assert close_to(oracle.gemv(Q6_K, kb.q6k_known_block(), 1, q)[0], -8192.0)


def _iq1m_scalar_reference(block, q):
    """Independent restatement in numpy of reference_iq1_m_q8_k
    (test_qwen38_quant.c:292-335), using the codebook from the oracle."""
    from oracle import Oracle
    grid_of = Oracle().grid_entry
    qs, qh, sc = block[:32], block[32:48], block[48:56]
    u = sc.view("<u2")
    bits = (int(u[0]) >> 12) | ((int(u[1]) >> 8) & 0xF0) | ((int(u[2]) >> 4) & 0xF00) | (int(u[3]) & 0xF000)
    d = np.float32(np.uint16(bits).view(np.float16)) * q["scale"][0]
    a = q["quants"][0].astype(np.int64)
    weighted = correction = 0
    for g in range(8):
        dot, cdot = [0, 0], [0, 0]
        for s in range(4):
            h = int(qh[2 * g + s // 2])
            gi = int(qs[4 * g + s]) | ((h << (8 - 4 * (s % 2))) & 0x700)
            delta = -1 if h & (0x80 if s % 2 else 0x08) else 1
            seg = a[32 * g + 8 * s: 32 * g + 8 * s + 8]
            dot[s // 2] += int(np.dot(seg, grid_of(gi).astype(np.int64)))
            cdot[s // 2] += int(seg.sum()) * delta
        packed = int(u[g // 2])
        s0 = 1 + 2 * ((packed >> (6 * (g % 2))) & 7)
        s1 = 1 + 2 * ((packed >> (6 * (g % 2) + 3)) & 7)
        weighted += s0 * dot[0] + s1 * dot[1]
        correction += s0 * cdot[0] + s1 * cdot[1]
    return weighted, correction, np.float32(d * (np.float32(weighted) + np.float32(0.125) * np.float32(correction)))


def test_iq1m_randomized_trials(oracle):
    """200 randomized blocks of test_iq_kernel (test_qwen38_quant.c:337-372, 905-907);
    the oracle must agree with the independent scalar form exactly (ints and fp32)."""
    for data, act in kb.random_iq_trials(IQ1_M, 56):
        q = oracle.quantize(act)
        ints = oracle.block_ints(IQ1_M, data, q)
        w, c, val = _iq1m_scalar_reference(data, q)
        assert (int(ints[0]), int(ints[1])) == (w, c)
        got = oracle.gemv(IQ1_M, data, 1, q)[0]
        assert np.float32(got).view(np.uint32) == val.view(np.uint32)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, IQ1_M])
def test_batch_exact_gemm_equals_gemv(oracle, qtype):
    """test_integer_batch_exact (test_qwen38_quant.c:637-684): GEMM rows are
    bit-identical to per-token GEMV for M = 1..5."""
    w, act, width, rows, tokens = kb.batch_exact_case(qtype, BLOCK_BYTES[qtype])
    q = oracle.quantize(act)
    nb = width // 256
    for m in range(1, tokens + 1):
        batch = oracle.gemm(qtype, w, rows, q[:m * nb], m)
        for t in range(m):
            single = oracle.gemv(qtype, w, rows, q[t * nb:(t + 1) * nb])
            assert batch[t].tobytes() == single.tobytes()


# ---- (2) closed forms and brute force ----------------------------------------

def _q8k_dequant_dot_int64(qtype, block, q):
    """Block value as exact integers from the format definition (no lane structure):
    Q4_K  sum_sub sc*sum(q*a) - m*sum(a)  -> (weighted, minimum) totals
    Q6_K  sum_sub sc*sum((q-32)*a)."""
    a = q["quants"][0].astype(np.int64)
    if qtype == Q4_K:
        sc_bytes = block[4:16].astype(np.int64)
        qs = block[16:144].astype(np.int64)
        weighted = minimum = 0
        for c in range(4):
            for half in range(2):
                i = 2 * c + half
                if i < 4:
                    sc, m = sc_bytes[i] & 63, sc_bytes[i + 4] & 63
                else:
                    sc = (sc_bytes[i + 4] & 15) | ((sc_bytes[i - 4] >> 6) << 4)
                    m = (sc_bytes[i + 4] >> 4) | ((sc_bytes[i] >> 6) << 4)
                nib = (qs[32 * c:32 * c + 32] >> (4 * half)) & 15
                seg = a[64 * c + 32 * half: 64 * c + 32 * half + 32]
                weighted += sc * int(np.dot(nib, seg))
                minimum += m * int(seg.sum())
        return weighted, minimum
    if qtype == Q6_K:
        ql, qh = block[:128].astype(np.int64), block[128:192].astype(np.int64)
        sc = block[192:208].view(np.int8).astype(np.int64)
        total = 0
        for e in range(256):
            h, r = divmod(e, 128)
            j, i = divmod(r, 32)
            low = ql[64 * h + 32 * (j & 1) + i]
            lo4 = (low & 15) if j < 2 else (low >> 4)
            hi2 = (qh[32 * h + i] >> (2 * j)) & 3
            total += sc[e // 16] * ((lo4 | hi2 << 4) - 32) * a[e]
        return total, 0
    raise ValueError


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_lane_sums_match_format_definition(oracle, qtype):
    rng = np.random.default_rng(11 + qtype)
    for _ in range(50):
        block = rng.integers(0, 256, BLOCK_BYTES[qtype], dtype=np.uint8)
        q = oracle.quantize(rng.normal(size=256).astype(np.float32))
        ints = oracle.block_ints(qtype, block, q)
        weighted, minimum = _q8k_dequant_dot_int64(qtype, block, q)
        assert int(ints[:8].sum()) == weighted
        if qtype == Q4_K:
            assert int(ints[8:12].sum()) == minimum


def test_q8k_quantize_edge_cases(oracle):
    zero = oracle.quantize(np.zeros(256, np.float32))
    assert zero["scale"][0] == 0 and not zero["quants"].any() and not zero["sums"].any()
    # the first element of largest magnitude sets the sign: -3 before +3
    x = np.zeros(256, np.float32)
    x[5], x[9] = -3.0, 3.0
    q = oracle.quantize(x)
    assert q["quants"][0, 5] == -127 and q["quants"][0, 9] == 127
    assert q["scale"][0] == np.float32(1.0) / (np.float32(-127.0) / np.float32(-3.0))
    # half-way cases round to even: max -127 -> inverse +1, so 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2], x[3], x[4] = -127.0, 0.5, 1.5, 2.5, -3.5
    q = oracle.quantize(x)
    assert list(q["quants"][0, :5]) == [-127, 0, 2, 2, -4]
    # group sums are the int sums of each 16
    q = oracle.quantize(np.random.default_rng(3).normal(size=1024).astype(np.float32))
    assert np.array_equal(q["quants"].reshape(-1, 16).sum(1), q["sums"].reshape(-1))


def test_argmax_first_index_and_nan(oracle):
    v = np.array([1.0, 3.0, 3.0, 2.0], np.float32)
    assert oracle.argmax(v) == 1
    v = np.array([np.nan, 5.0, 1.0], np.float32)
    assert oracle.argmax(v) == 0
    v = np.array([1.0, np.nan, 5.0, np.nan], np.float32)
    assert oracle.argmax(v) == 2
    v = np.array([-0.0, 0.0], np.float32)
    assert oracle.argmax(v) == 0


def test_accept_brute_force(oracle):
    """Acceptance against an independent scan over every match pattern of 4 rows."""
    rng = np.random.default_rng(5)
    count = 50
    for pattern in range(16):
        logits = rng.normal(size=(4, count)).astype(np.float32)
        targets = logits.argmax(1)
        drafts = np.array([targets[i] if pattern >> i & 1 else (targets[i] + 1) % count for i in range(4)],
                          np.uint32)
        consumed, matched, nxt, accepted = oracle.accept(logits, drafts)
        m = 0
        while m < 4 and pattern >> m & 1:
            m += 1
        assert matched == m
        assert consumed == (m + 1 if m < 4 else 4)
        assert nxt == (targets[m] if m < 4 else drafts[3])
        assert list(accepted) == [int(d) for d in drafts[:m]] + ([int(targets[m])] if m < 4 else [])


def test_iq1m_grid_table_invariants(oracle):
    import re
    inc = os.path.join(os.path.dirname(GOLDEN), "..", "qwen3.8-27b-in-c_amd", "csrc", "q38_iq1m_grid.inc")
    text = open(inc).read()
    digest = re.search(r'Q38_IQ1M_GRID_SHA256 "([0-9a-f]+)"', text).group(1)
    grid = np.array([oracle.grid_entry(i) for i in range(2048)], dtype=np.int8)
    assert set(np.unique(grid)) <= {-1, 0, 1}
    assert len({bytes(r) for r in grid.view(np.uint8)}) == 2048
    assert hashlib.sha256(grid.tobytes()).hexdigest() == digest
    ref_header = "/root/reference/third_party/ggml-common.h"
    if os.path.exists(ref_header):
        import importlib.util
        spec = importlib.util.spec_from_file_location(
            "gen", os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "gen_iq1m_grid.py"))
        gen = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(gen)
        assert np.array_equal(np.array(gen.read_reference_grid(ref_header), np.int8), grid)


# ---- (3) golden vectors written by the compiled reference ----------------------

def _golden_files():
    if not os.path.isdir(GOLDEN):
        return []
    # kernel fixtures of tests/golden/make_golden.py (the model, decode and
    # attention fixtures have scripts and tests of their own)
    return sorted(f for f in os.listdir(GOLDEN)
                  if f.endswith(".npz") and f.split("_")[0] in ("q4k", "q6k", "iq1m"))


@pytest.mark.parametrize("name", _golden_files())
def test_oracle_matches_golden(oracle, name):
    g = np.load(os.path.join(GOLDEN, name))
    qtype, rows, width, tokens = (int(v) for v in g["meta"])
    q = oracle.quantize(g["x"])
    assert q.tobytes() == g["q8k"].tobytes()
    out = oracle.gemm(qtype, g["w"], rows, q, tokens)
    assert out.view(np.uint32).tobytes() == g["y"].view(np.uint32).tobytes()


# ---- (4) the compiled reference, when present ----------------------------------

@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, IQ1_M])
@pytest.mark.parametrize("rows,width", [(96, 5120), (24, 17408)])
def test_oracle_matches_compiled_reference(oracle, reference, qtype, rows, width):
    w = synth.matrix(qtype, rows, width, seed=1000 + qtype + rows)
    x = synth.activations(width, seed=77, count=5).reshape(-1)
    qo, qr = oracle.quantize(x), reference.quantize(x)
    assert qo.tobytes() == qr.tobytes()
    nb = width // 256
    for m in (1, 2, 3, 4, 5):
        a = oracle.gemm(qtype, w, rows, qo[:m * nb], m)
        b = reference.gemm(qtype, w, rows, qr[:m * nb], m)
        assert a.view(np.uint32).tobytes() == b.view(np.uint32).tobytes()


def test_row_dequant_matches_compiled_reference(oracle, reference):
    w = synth.matrix(Q4_K, 4, 1024, seed=9)
    for row in range(4):
        a = oracle.row_f32(Q4_K, w, 1024, row)
        b = reference.row_f32(Q4_K, w, 1024, row, 4)
        assert a.view(np.uint32).tobytes() == b.view(np.uint32).tobytes()


# ---- attention core (orc_attention_decode) -----------------------------------

def _oracle_core(oracle):
    def core(q_and_gate, key, value, key_cache, value_cache, q_norm, k_norm, position):
        return oracle.attention_decode(q_and_gate, key, value, key_cache, value_cache, q_norm, k_norm, position)
    return core


def test_attention_oracle_position_zero_closed_form(oracle):
    """At position 0 the softmax has one term: e = 1, probability 1, so each
    output is fmaf(1, v, 0) * sigmoid(gate) = v * sigmoid(gate) exactly
    (qwen38_model.c:863-882), whatever q and k are."""
    import attention_cases as ac
    rows_in, qn, kn, kc, vc = ac.inputs(4, 0, 1)
    att = ac.run_rows(_oracle_core(oracle), rows_in, qn, kn, kc, vc, 0)[0]
    gate = rows_in[0, :ac.KEY].reshape(24, 512)[:, 256:]
    value = rows_in[0, ac.VALUE:].reshape(4, 256)
    sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-gate.astype(np.float64)).astype(np.float32)))
    want = (value[np.arange(24) // 6] * sig).reshape(-1)
    # numpy's exp is not the C library's expf: compare to 1 ulp of the sigmoid
    assert np.allclose(att, want, rtol=2e-7, atol=0)
    assert np.array_equal(vc[0], value.reshape(-1))


def test_attention_oracle_matches_golden(oracle):
    """The oracle equals the reference's own q38_full_core (compiled from its
    source, tests/golden/make_attention_golden.py) at positions 0, 1, 31,
    32, 33, 2047 and 4100, output and written K row bit for bit."""
    import attention_cases as ac
    g = np.load(os.path.join(GOLDEN, "attention_ref.npz"))
    for i, position in enumerate(g["positions"]):
        position = int(position)
        rows_in, qn, kn, kc, vc = ac.inputs(position + 1, position, 1)
        att = ac.run_rows(_oracle_core(oracle), rows_in, qn, kn, kc, vc, position)[0]
        assert np.array_equal(att[:64].view(np.uint32), g["first64"][i].view(np.uint32)), position
        assert ac.digest(att) == g["digests"][i], position
        assert ac.digest(kc[position]) == g["key_digests"][i], position


def test_attention_oracle_matches_compiled_reference_rows(oracle, reference):
    """Several consecutive rows (positions 28..35, across the 32-position
    batch boundary), outputs and both caches, against the compiled reference."""
    import attention_cases as ac
    rows_in, qn, kn, kc, vc = ac.inputs(48, 28, 8)
    kc2, vc2 = kc.copy(), vc.copy()
    got = ac.run_rows(_oracle_core(oracle), rows_in, qn, kn, kc, vc, 28)
    want = ac.run_rows(reference.full_core, rows_in, qn, kn, kc2, vc2, 28)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(kc.view(np.uint32), kc2.view(np.uint32))
    assert np.array_equal(vc.view(np.uint32), vc2.view(np.uint32))
