"""q38hip_argmax_noalloc (include/q38hip.h): the argmax entry point that
allocates nothing keeps its partial maxima in the library's fixed device
array.  Its results must equal q38hip_argmax's (and the oracle's first-maximum
rule, src/qwen38/qwen38_model.c:1228-1239) on two calls in a row, the second
with a smaller input, and it must refuse a call larger than that array."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _rows_with_edge_cases(rng, rows, count):
    v = rng.normal(size=(rows, count)).astype(np.float32)
    v[min(1, rows - 1), count // 7] = v[min(1, rows - 1), count - 5] = 50.0   # tie: lower index wins
    if rows > 2:
        v[2, 0] = np.nan                                                     # NaN at 0 keeps index 0
    if rows > 3:
        v[3, 17] = np.nan
        v[3, 99] = 60.0                                                      # NaN elsewhere never wins
    if rows > 4:
        v[4, :] = -np.inf
    return v


def test_noalloc_argmax_equals_argmax(device, oracle):
    import torch
    import q38hip
    rng = np.random.default_rng(21)
    # 248320-wide verify rows, then a smaller call that reuses the array
    for rows, count in ((6, 248320), (2, 1000)):
        v = _rows_with_edge_cases(rng, rows, count)
        d = torch.from_numpy(v).to(device)
        got = q38hip.argmax_noalloc(d)
        want = q38hip.argmax(d)
        torch.cuda.synchronize()
        got, want = got.cpu().numpy(), want.cpu().numpy()
        print("noalloc argmax rows=%d count=%d -> %s" % (rows, count, list(got)), flush=True)
        assert list(got) == list(want)
        assert list(got) == [oracle.argmax(row) for row in v]


def test_noalloc_argmax_largest_and_refused_sizes(device):
    import torch
    import q38hip
    rng = np.random.default_rng(22)
    # ceil(248320 / 4096) = 61 partials per row: 134 rows fill 8174 of 8192
    v = torch.from_numpy(rng.normal(size=(135, 248320)).astype(np.float32)).to(device)
    out = torch.zeros(135, dtype=torch.int32, device=device)
    got = q38hip.argmax_noalloc(v[:134], out=out[:134])
    want = q38hip.argmax(v[:134])
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want.cpu())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # 135 rows need 8235 partials: refused on the host, nothing launched
    ok = q38hip.lib().q38hip_argmax_noalloc(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(v.data_ptr()),
                                            248320, 135, stream)
    assert ok == 0
    assert "8192" in q38hip.last_error()
    torch.cuda.synchronize()
