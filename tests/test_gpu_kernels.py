"""GPU parity of the HIP kernels against the CPU oracle (bit-exact).

Every test calls libq38hip through its C ABI (q38hip ctypes binding) and
compares with oracle/ on the same seeded inputs: integer/index results and
fp32 outputs must be identical bit for bit (the reference's AVX2 lane order).
"""
import os

import numpy as np
import pytest

import known_blocks as kb
from oracle import IQ1_M, Q4_K, Q6_K
from q38hip import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def hip(device):
    import q38hip
    q38hip.lib()
    return q38hip


def to_dev(array, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_quantize_matches_oracle(hip, oracle, device):
    rng = np.random.default_rng(1)
    x = rng.normal(size=(3, 17408)).astype(np.float32)
    x[0, :256] = 0.0                                   # zero block
    x[1, 256:512] = 0.0
    x[1, 300], x[1, 400] = -2.5, 2.5                   # |max| tie: first wins
    x[2, 512:768] = np.float32(-127.0)                 # half-way rounding block
    x[2, 513:517] = [0.5, 1.5, 2.5, -3.5]
    x[2, 768:1024] *= np.float32(1e-30)                # tiny values
    got = hip.quantize_q8_k(to_dev(x, device)).cpu().numpy()
    want = oracle.quantize(x.reshape(-1)).view(np.uint8)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("qtype", [Q4_K, IQ1_M, Q6_K])
@pytest.mark.parametrize("rows,width", [(17408, 5120), (5120, 17408)])
def test_gemv_full_shape_bit_exact(hip, oracle, device, qtype, rows, width):
    """cfg1/cfg2 shapes: 17408x5120 and 5120x17408, one activation row."""
    w = synth.matrix(qtype, rows, width, seed=7 * qtype + rows)
    x = synth.activations(width, seed=rows + 3)
    q = oracle.quantize(x.reshape(-1))
    want = oracle.gemv(qtype, w, rows, q)
    xq = hip.quantize_q8_k(to_dev(x, device))
    assert xq.cpu().numpy().tobytes() == q.view(np.uint8).tobytes()
    got = hip.gemm_q8_k(to_dev(w, device), qtype, width, rows, xq, 1).cpu().numpy()[0]
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("qtype", [Q4_K, IQ1_M, Q6_K])
@pytest.mark.parametrize("rows,width", [(1024, 5120), (96, 17408), (48, 5120), (77, 6144)])
def test_gemm_rows_bit_exact(hip, oracle, device, qtype, rows, width):
    """Verify-batch and prefill GEMM, M = 1..8 rows, against the per-token
    oracle GEMV."""
    w = synth.matrix(qtype, rows, width, seed=11 * qtype + rows)
    x = synth.activations(width, seed=width + rows, count=8)
    q = oracle.quantize(x.reshape(-1))
    wd = to_dev(w, device)
    xq = hip.quantize_q8_k(to_dev(x, device))
    nb = width // 256
    for m in range(1, 9):
        want = oracle.gemm(qtype, w, rows, q[:m * nb], m)
        got = hip.gemm_q8_k(wd, qtype, width, rows, xq[:m * nb * 292], m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), "M=%d" % m


@pytest.mark.parametrize("name", sorted(f for f in os.listdir(GOLDEN)
                                          if f.endswith(".npz") and f.split("_")[0] in ("q4k", "q6k", "iq1m")))
def test_gpu_matches_reference_golden(hip, device, name):
    g = np.load(os.path.join(GOLDEN, name))
    qtype, rows, width, tokens = (int(v) for v in g["meta"])
    xq = hip.quantize_q8_k(to_dev(g["x"].reshape(tokens, width), device))
    assert xq.cpu().numpy().tobytes() == g["q8k"].tobytes()
    got = hip.gemm_q8_k(to_dev(g["w"], device), qtype, width, rows, xq, tokens).cpu().numpy()
    assert np.array_equal(bits(got), bits(g["y"]))


def test_host_dropins_known_answers(hip):
    """The reference kernel ABI (host pointers) on the reference's known blocks."""
    ones = hip.host_quantize_q8_k(np.ones(256, np.float32))
    assert abs(hip.host_tensor_gemv_q8_k(Q4_K, kb.q4k_known_block(), 1, ones)[0] - 64.0) <= 64e-5
    assert abs(hip.host_tensor_gemv_q8_k(IQ1_M, kb.iq1m_known_block(), 1, ones)[0] + 224.0) <= 224e-5
    assert abs(hip.host_tensor_gemv_q8_k(Q6_K, kb.q6k_known_block(), 1, ones)[0] + 8192.0) <= 8192e-5
    w = np.concatenate([kb.q4k_known_block(), kb.q4k_known_block()])
    x = hip.host_quantize_q8_k(np.concatenate([np.ones(256, np.float32), np.full(256, 2.0, np.float32)]))
    out = hip.host_tensor_gemm_q8_k(Q4_K, w, 2, x, 2).reshape(-1)
    assert np.allclose(out, [64.0, 64.0, 128.0, 128.0], rtol=1e-5)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, IQ1_M])
def test_host_dropins_batch_exact(hip, oracle, qtype):
    """test_integer_batch_exact inputs: GEMM = GEMV bit-exact, and equal to the oracle."""
    from oracle import BLOCK_BYTES
    w, act, width, rows, tokens = kb.batch_exact_case(qtype, BLOCK_BYTES[qtype])
    q = hip.host_quantize_q8_k(act)
    assert q.tobytes() == oracle.quantize(act).tobytes()
    nb = width // 256
    for m in range(1, tokens + 1):
        batch = hip.host_tensor_gemm_q8_k(qtype, w, rows, q[:m * nb], m)
        assert np.array_equal(bits(batch), bits(oracle.gemm(qtype, w, rows, q[:m * nb], m)))
        for t in range(m):
            single = hip.host_tensor_gemv_q8_k(qtype, w, rows, q[t * nb:(t + 1) * nb])
            assert batch[t].tobytes() == single.tobytes()


def test_iq1m_randomized_trials_gpu(hip, oracle):
    for data, act in kb.random_iq_trials(IQ1_M, 56, trials=50):
        q = hip.host_quantize_q8_k(act)
        got = hip.host_tensor_gemv_q8_k(IQ1_M, data, 1, q)
        assert bits(got).tobytes() == bits(oracle.gemv(IQ1_M, data, 1, q)).tobytes()


def test_argmax_matches_oracle(hip, oracle, device):
    rng = np.random.default_rng(4)
    v = rng.normal(size=(5, 248320)).astype(np.float32)
    v[1, 1000] = v[1, 200000] = 50.0          # tie: lower index wins
    v[2, 0] = np.nan                           # NaN at 0 keeps index 0
    v[3, 17] = np.nan
    v[3, 99] = 60.0                            # NaN elsewhere never wins
    v[4, :] = -np.inf
    got = hip.argmax(to_dev(v, device)).cpu().numpy()
    want = [oracle.argmax(row) for row in v]
    assert list(got) == want


def test_accept_matches_oracle(hip, oracle, device):
    import torch
    rng = np.random.default_rng(8)
    count = 1000
    for pattern in range(16):
        logits = rng.normal(size=(4, count)).astype(np.float32)
        targets = logits.argmax(1).astype(np.int32)
        drafts = np.array([targets[i] if pattern >> i & 1 else (targets[i] + 3) % count for i in range(4)],
                          np.int32)
        for rows in (1, 2, 3, 4):
            res = hip.accept(to_dev(targets[:rows], device), to_dev(drafts[:rows], device)).cpu().numpy()
            consumed, matched, nxt, accepted = oracle.accept(logits[:rows], drafts[:rows].astype(np.uint32))
            assert (res[0], res[1], res[2]) == (consumed, matched, nxt)
            assert list(res[3:3 + consumed]) == list(accepted)
    torch.cuda.synchronize()


def tiled_numpy(w, rows, width):
    """Host restatement of the 16-row tiled layout: [tile][block][row % 16][144]."""
    nb = width // 256
    tiles = (rows + 15) // 16
    padded = np.zeros((tiles * 16, nb, 144), dtype=np.uint8)
    padded[:rows] = w.reshape(rows, nb, 144)
    return np.ascontiguousarray(padded.reshape(tiles, 16, nb, 144).transpose(0, 2, 1, 3)).reshape(-1)


@pytest.mark.parametrize("rows,width", [(1000, 5120), (48, 5120), (2064, 6144), (520, 10240), (1040, 17408),
                                        (4112, 5120), (4100, 6144), (5136, 17408), (3, 5120), (1003, 17408)])
def test_tiled_repack_and_gemm_bit_exact(hip, oracle, device, rows, width):
    """Tiled Q4_K copy (one token on the dot4/dot2 lanes, 2..8 tokens on the
    matrix cores) equals the oracle bit for bit; the repack equals the host
    restatement of the layout (zero-padded tail).  From 4096 rows on, 2..8
    tokens run the 32-row kernel (5..8 with a second token set): 4112 and
    5136 rows end on an unpaired 16-row tile, 4100 also on a padded one; 3
    and 1003 rows end inside the one-token kernel's 8-row groups."""
    w = synth.matrix(Q4_K, rows, width, seed=rows + width)
    wd = to_dev(w, device)
    tiled = hip.repack_q4k_tiles(wd, width, rows)
    assert tiled.cpu().numpy().tobytes() == tiled_numpy(w, rows, width).tobytes()
    x = synth.activations(width, seed=rows * 3 + 1, count=8)
    q = oracle.quantize(x.reshape(-1))
    xq = hip.quantize_q8_k(to_dev(x, device))
    nb = width // 256
    for m in range(1, 9):
        want = oracle.gemm(Q4_K, w, rows, q[:m * nb], m)
        got = hip.gemm_q8_k_tiled(tiled, width, rows, xq[:m * nb * 292], m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), "M=%d" % m


@pytest.mark.parametrize("rows,width", [(48, 5120), (1000, 5120), (520, 10240), (5136, 17408), (2064, 6144),
                                        (1003, 5120), (3, 6144)])
def test_tiled_iq1m_repack_and_gemm_bit_exact(hip, oracle, device, rows, width):
    """16-row tiled IQ1_M copy ([tile][block][row % 16][56 bytes], zero rows
    past the last): the repack equals the host restatement of the layout, and
    the matrix-core kernel over it equals the oracle bit for bit for 1..8
    tokens, with row counts that end inside a tile (1000, 520, 5136) and
    inside a 4-row quad (1003, 3: the one-token kernel's unit)."""
    w = synth.matrix(IQ1_M, rows, width, seed=rows + 2 * width)
    wd = to_dev(w, device)
    tiled = hip.repack_iq1m_tiles(wd, width, rows)
    nb = width // 256
    tiles = (rows + 15) // 16
    padded = np.zeros((tiles * 16, nb, 56), dtype=np.uint8)
    padded[:rows] = w.reshape(rows, nb, 56)
    want_layout = np.ascontiguousarray(padded.reshape(tiles, 16, nb, 56).transpose(0, 2, 1, 3)).reshape(-1)
    assert tiled.cpu().numpy().tobytes() == want_layout.tobytes()
    x = synth.activations(width, seed=rows * 5 + 3, count=8)
    q = oracle.quantize(x.reshape(-1))
    xq = hip.quantize_q8_k(to_dev(x, device))
    for m in range(1, 9):
        want = oracle.gemm(IQ1_M, w, rows, q[:m * nb], m)
        got = hip.gemm_q8_k_iq1m_tiled(tiled, width, rows, xq[:m * nb * 292], m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), "M=%d" % m


@pytest.mark.parametrize("m", [1, 2, 3])
def test_tiled_iq1m_full_shape_matches_row_major(hip, device, m):
    """34816x5120 (fused gate|up), 5120x17408 (down) and 16480x5120 (the
    DeltaNet input group) IQ1_M: the tiled copy's kernel (the v_dot4 one for
    1..3 tokens) equals the row-major matrix-core kernel bit for bit."""
    for rows, width in ((34816, 5120), (5120, 17408), (16480, 5120)):
        w = synth.matrix(IQ1_M, rows, width, seed=m + rows + 1)
        wd = to_dev(w, device)
        x = synth.activations(width, seed=m * 11 + width, count=m)
        xq = hip.quantize_q8_k(to_dev(x, device))
        want = hip.gemm_q8_k(wd, IQ1_M, width, rows, xq, m).cpu().numpy()
        got = hip.gemm_q8_k_iq1m_tiled(hip.repack_iq1m_tiles(wd, width, rows), width, rows, xq, m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), (rows, width)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
def test_tiled_gemm_full_shape_matches_row_major(hip, device, m):
    """34816x5120 (fused gate|up) and 5120x17408 (down): tiled = row-major kernels;
    24584x5120 ends on an unpaired 16-row tile at a size where the 32-row
    kernel's workgroups run in more than one wave over the chip; 33000 and
    36864 rows are a ragged last tile and the largest matrix of the 16-row
    streaming kernel (q38_mm16.hip, 2..4 tokens from 32768 rows on)."""
    shapes = ((34816, 5120), (5120, 17408), (24584, 5120))
    if m <= 4:
        shapes += ((33000, 5120), (36864, 5120))
    for rows, width in shapes:
        w = synth.matrix(Q4_K, rows, width, seed=m + rows)
        wd = to_dev(w, device)
        x = synth.activations(width, seed=m * 7 + width, count=m)
        xq = hip.quantize_q8_k(to_dev(x, device))
        want = hip.gemm_q8_k(wd, Q4_K, width, rows, xq, m).cpu().numpy()
        got = hip.gemm_q8_k_tiled(hip.repack_q4k_tiles(wd, width, rows), width, rows, xq, m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), (rows, width)


@pytest.mark.parametrize("qtype", [Q4_K, IQ1_M, Q6_K])
def test_gemm_any_batch_size(hip, oracle, device, qtype):
    """q38hip_gemm_q8_k and the host drop-in q38_tensor_gemm_q8_k take any
    batch size, as the reference's GEMM (qwen38_quant.c:2950-2956): 9, 12,
    13 and 17 tokens run as launches of up to 8 and equal the oracle's
    per-token GEMVs bit for bit."""
    rows, width = 520, 5120
    w = synth.matrix(qtype, rows, width, seed=qtype + 40)
    x = synth.activations(width, seed=qtype + 41, count=17)
    q = oracle.quantize(x.reshape(-1))
    nb = width // 256
    wd = to_dev(w, device)
    xq = hip.quantize_q8_k(to_dev(x, device))
    for m in (9, 12, 13, 17):
        want = oracle.gemm(qtype, w, rows, q[:m * nb], m)
        got = hip.gemm_q8_k(wd, qtype, width, rows, xq[:m * nb * 292], m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), "M=%d" % m
    host = hip.host_tensor_gemm_q8_k(qtype, w, rows, q[:12 * nb], 12)
    assert np.array_equal(bits(host), bits(oracle.gemm(qtype, w, rows, q[:12 * nb], 12)))


def test_tiled_gemm_any_batch_size(hip, oracle, device):
    """The tiled entry point splits 9, 10 and 17 tokens into launches of 2..8."""
    rows, width = 4112, 5120
    w = synth.matrix(Q4_K, rows, width, seed=77)
    x = synth.activations(width, seed=78, count=17)
    q = oracle.quantize(x.reshape(-1))
    nb = width // 256
    tiled = hip.repack_q4k_tiles(to_dev(w, device), width, rows)
    xq = hip.quantize_q8_k(to_dev(x, device))
    for m in (9, 10, 17):
        want = oracle.gemm(Q4_K, w, rows, q[:m * nb], m)
        got = hip.gemm_q8_k_tiled(tiled, width, rows, xq[:m * nb * 292], m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want)), "M=%d" % m


@pytest.mark.parametrize("rows,width", [(136, 5120), (64, 17408), (200, 6144), (72, 10240)])
def test_wide_gemm_prefill_batches_bit_exact(hip, oracle, device, rows, width):
    """Prefill batches (16 tokens and more) on the 64 x 64 matrix-core tiles:
    every token's row equals the oracle's one-token GEMV bit for bit, with
    ragged row counts (a padded last 16-row tile, a workgroup past the last
    tile) and token counts that end inside a 64-token tile."""
    w = synth.matrix(Q4_K, rows, width, seed=rows * 7 + width)
    x = synth.activations(width, seed=rows + width, count=100)
    q = oracle.quantize(x.reshape(-1))
    nb = width // 256
    tiled = hip.repack_q4k_tiles(to_dev(w, device), width, rows)
    xq = hip.quantize_q8_k(to_dev(x, device))
    want = oracle.gemm(Q4_K, w, rows, q, 100)
    for m in (16, 33, 64, 100):
        got = hip.gemm_q8_k_tiled(tiled, width, rows, xq[:m * nb * 292], m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want[:m])), "M=%d" % m


@pytest.mark.parametrize("rows,width", [(34816, 5120), (5120, 17408), (16480, 5120)])
def test_wide_gemm_full_shapes_match_decode_kernels(hip, device, rows, width):
    """Full prefill shapes (gate|up, down, DeltaNet input group) at 256 tokens
    against the 2..8-token kernels on the same activations."""
    m = 256
    w = synth.matrix(Q4_K, rows, width, seed=rows + 3)
    wd = to_dev(w, device)
    tiled = hip.repack_q4k_tiles(wd, width, rows)
    x = synth.activations(width, seed=width + 5, count=m)
    xq = hip.quantize_q8_k(to_dev(x, device))
    got = hip.gemm_q8_k_tiled(tiled, width, rows, xq, m).cpu().numpy()
    nb = width // 256
    for t0 in (0, 8, 120, 248):
        want = hip.gemm_q8_k_tiled(tiled, width, rows, xq[t0 * nb * 292:(t0 + 8) * nb * 292], 8).cpu().numpy()
        assert np.array_equal(bits(got[t0:t0 + 8]), bits(want)), (rows, width, t0)


@pytest.mark.parametrize("rows,width", [(300, 5120), (40, 17408), (520, 6144)])
def test_iq1m_wide_gemm_prefill_batches_bit_exact(hip, oracle, device, rows, width):
    """IQ1_M prefill batches (9 tokens and more: 256 x 64 matrix-core tiles,
    from 128 tokens on 256 x 128 tiles): every token's row equals the
    oracle's one-token GEMV bit for bit, with a row count that ends inside a
    wavefront's 32 rows and token counts that end inside a token tile."""
    w = synth.matrix(IQ1_M, rows, width, seed=rows * 5 + width)
    x = synth.activations(width, seed=rows + 2 * width, count=200)
    q = oracle.quantize(x.reshape(-1))
    nb = width // 256
    wd = to_dev(w, device)
    xq = hip.quantize_q8_k(to_dev(x, device))
    want = oracle.gemm(IQ1_M, w, rows, q, 200)
    for m in (9, 16, 33, 64, 100, 128, 200):
        got = hip.gemm_q8_k(wd, IQ1_M, width, rows, xq[:m * nb * 292], m).cpu().numpy()
        assert np.array_equal(bits(got), bits(want[:m])), "M=%d" % m


@pytest.mark.parametrize("rows,width,m", [(34744, 5120, 1100), (5120, 17408, 4096)])
def test_iq1m_wide_gemm_large_batches_bit_exact(hip, oracle, device, rows, width, m):
    """Prompt batches large enough for the 256-row workgroups (gate|up, a
    ragged last row group and token tile) and a full 4096-token down
    projection on the 128-row ones: token windows equal the 8-token kernel
    on the same activations, and the first window the oracle."""
    w = synth.matrix(IQ1_M, rows, width, seed=rows + 21)
    wd = to_dev(w, device)
    x = synth.activations(width, seed=width + 23, count=m)
    xq = hip.quantize_q8_k(to_dev(x, device))
    got = hip.gemm_q8_k(wd, IQ1_M, width, rows, xq, m).cpu().numpy()
    nb = width // 256
    for t0 in (0, 8, 640, m - 8):
        want = hip.gemm_q8_k(wd, IQ1_M, width, rows, xq[t0 * nb * 292:(t0 + 8) * nb * 292], 8).cpu().numpy()
        assert np.array_equal(bits(got[t0:t0 + 8]), bits(want)), (rows, width, t0)
    q = oracle.quantize(x[:8].reshape(-1))
    assert np.array_equal(bits(got[:8]), bits(oracle.gemm(IQ1_M, w, rows, q, 8)))


def test_iq1m_wide_gemm_tiny_scales_bit_exact(hip, oracle, device):
    """Tokens whose Q8_K scales are below 2^-99 (activations near 1e-30) or
    zero: a 128-token tile holding one runs the literal chain
    d * (E * 0.125f), the others the folded one; both equal the oracle bit
    for bit."""
    rows, width, m = 264, 5120, 256
    w = synth.matrix(IQ1_M, rows, width, seed=77)
    x = synth.activations(width, seed=78, count=m).reshape(m, width).copy()
    x[5] *= np.float32(1e-33)       # scales near 3e-35: the first tile's chain is the literal one
    x[140] = 0.0                    # zero scale: the second tile folds
    x[141] *= np.float32(1e-20)
    q = oracle.quantize(x.reshape(-1))
    xq = hip.quantize_q8_k(to_dev(x, device))
    assert np.array_equal(xq.cpu().numpy(), q.view(np.uint8)), "quantized activations differ"
    want = oracle.gemm(IQ1_M, w, rows, q, m)
    got = hip.gemm_q8_k(to_dev(w, device), IQ1_M, width, rows, xq, m).cpu().numpy()
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("rows,width", [(34816, 5120), (5120, 17408)])
def test_iq1m_wide_gemm_full_shapes_match_decode_kernel(hip, device, rows, width):
    m = 256
    w = synth.matrix(IQ1_M, rows, width, seed=rows + 11)
    wd = to_dev(w, device)
    x = synth.activations(width, seed=width + 13, count=m)
    xq = hip.quantize_q8_k(to_dev(x, device))
    got = hip.gemm_q8_k(wd, IQ1_M, width, rows, xq, m).cpu().numpy()
    nb = width // 256
    for t0 in (0, 8, 120, 248):
        want = hip.gemm_q8_k(wd, IQ1_M, width, rows, xq[t0 * nb * 292:(t0 + 8) * nb * 292], 8).cpu().numpy()
        assert np.array_equal(bits(got[t0:t0 + 8]), bits(want)), (rows, width, t0)
