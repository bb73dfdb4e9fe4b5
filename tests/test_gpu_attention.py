"""Full-attention decode core on the GPU (q38hip_attention_rows: the engine's
attention prep, score, softmax, value-mix and Q8_K kernels) against the
oracle's orc_attention_decode, which is pinned to the reference's own
q38_full_core (src/qwen38/qwen38_model.c:816-885; tests/test_oracle_pins.py).

Bar: bit-identical outputs, K/V cache rows and Q8_K blocks of the output.
Cases: the 2048-token cache of a verify block with M = 1..5 rows (the last
row at position 2047), a 5124-token cache with 5 rows at positions
4096-4100 and 5119-5123, contexts of 1..66 positions around the 32-position
chunks of the value stream, prefill batches of 9-130 rows (8-row score
tiles, a ragged last tile, batches starting at position 0, a context that
is not a multiple of four floats), a 16384-token cache,
and a context above 32768 positions, where the softmax weights stay in the
scores buffer instead of LDS.  Cache rows past the last row's position hold
NaN, so a kernel that read them would fail the comparison."""
import numpy as np
import pytest

import attention_cases as ac

pytestmark = pytest.mark.gpu

CASES = [
    # (context, position, rows)
    (64, 0, 1),
    (96, 28, 8),
    (2048, 2047, 1),
    (2048, 2046, 2),
    (2048, 2045, 3),
    (2048, 2044, 4),
    (2048, 2043, 5),
    (5124, 4096, 5),
    (5124, 5119, 5),
    (700, 600, 12),
    (160, 100, 9),
    (300, 0, 64),
    (1100, 37, 130),
    (203, 150, 11),
    (40, 0, 2),
    (80, 30, 4),
    (80, 62, 4),
    (16384, 16000, 2),
    (40000, 60, 3),
]


def _oracle_core(oracle):
    def core(q_and_gate, key, value, key_cache, value_cache, q_norm, k_norm, position):
        return oracle.attention_decode(q_and_gate, key, value, key_cache, value_cache, q_norm, k_norm, position)
    return core


@pytest.mark.parametrize("context,position,rows", CASES)
def test_attention_rows_bit_exact(device, oracle, context, position, rows):
    import torch
    import q38hip
    print("attention context=%d position=%d rows=%d" % (context, position, rows), flush=True)
    rows_in, qn, kn, kc, vc = ac.inputs(context, position, rows)
    kc[position + rows:] = np.nan
    vc[position + rows:] = np.nan
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    # the library keeps the value cache channel-major, padded to 32 positions
    pitch = q38hip.value_pitch(context)
    vc_t = np.full((1024, pitch), np.nan, dtype=np.float32)
    vc_t[:, :context] = vc.T
    dk, dv = d(kc), d(vc_t)
    got, got_q = q38hip.attention_rows(d(rows_in), d(qn), d(kn), dk, dv, position)
    torch.cuda.synchronize()
    want = ac.run_rows(_oracle_core(oracle), rows_in, qn, kn, kc, vc, position)
    got = got.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        "max abs diff %g" % np.abs(got - want).max()
    span = slice(position, position + rows)
    assert np.array_equal(dk.cpu().numpy()[span].view(np.uint32), kc[span].view(np.uint32))
    assert np.array_equal(np.ascontiguousarray(dv.cpu().numpy()[:, span].T).view(np.uint32), vc[span].view(np.uint32))
    assert got_q.cpu().numpy().tobytes() == oracle.quantize(want.reshape(-1)).tobytes()
