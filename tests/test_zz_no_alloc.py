"""twd_select_noalloc, the selection entry point that allocates nothing (its scratch is a fixed
device array), against twd_select with a selector on identical inputs: penalised rows and ids
bit for bit, on two calls in a row, the second smaller, then the size limits."""
import ctypes

import numpy as np
import pytest

from helpers import twd

pytestmark = pytest.mark.gpu


def _rows(rng, rows, n):
    out = (rng.standard_normal((rows, n)) * rng.uniform(1, 6, (rows, 1))).astype(np.float32)
    out[0, 5:9] = out[0].max()  # ties at the top of one row
    return out


def _params(t, rng, rows, n, hist_len):
    out = []
    for m in range(rows):
        kind = m % 4
        u = t.uniform_from_seed(t.splitmix64(31 * m + n))
        if kind == 0:
            out.append(t.RowParams(0.0, 1.0, 0, 1.0, 0.0, 30.0, 0, 0))  # greedy
        elif kind == 1:
            out.append(t.RowParams(0.7, 0.9, 40, 1.1, u, 30.0, m * hist_len, hist_len))
        elif kind == 2:
            out.append(t.RowParams(1.0, 1.0, 0, 1.0, u, 30.0, 0, 0))  # top-256 shortlist
        else:
            out.append(t.RowParams(0.9, 0.95, int(rng.integers(20, 101)), 1.3, u, 30.0,
                                   m * hist_len, hist_len))
    return out


def _noalloc(t, lg, params, hist, tok, stream):
    arr = (t.RowParams * len(params))(*params)
    rows, n = lg.shape
    rc = t.twd.lib.twd_select_noalloc(lg.data_ptr(), n, rows, n, arr,
                                      None if hist is None else hist.data_ptr(), tok.data_ptr(),
                                      stream)
    if rc != 0:
        raise t.TwdError(rc, t.twd.last_error())
    return tok


@pytest.mark.parametrize("shape", [[(64, 262144), (5, 50000)], [(9, 200000), (1, 1000)]])
def test_noalloc_matches_selector(shape):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    sel = t.Selector(262144, 64)
    rng = np.random.default_rng(sum(r * n for r, n in shape))
    for rows, n in shape:  # two calls in a row, the second smaller
        hist_len = 512
        base = _rows(rng, rows, n)
        hist = torch.from_numpy(rng.integers(0, n, rows * hist_len).astype(np.int32)).to(dev)
        params = _params(t, rng, rows, n, hist_len)
        a = torch.from_numpy(base).to(dev)
        b = torch.from_numpy(base).to(dev)
        ta = torch.full((rows,), -7, dtype=torch.int32, device=dev)
        tb = torch.full((rows,), -7, dtype=torch.int32, device=dev)
        sel.select(a, params, hist, ta, stream=stream)
        _noalloc(t, b, params, hist, tb, stream)
        torch.cuda.synchronize()
        assert np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))
        assert ta.cpu().tolist() == tb.cpu().tolist(), (rows, n)
    sel.close()


def test_noalloc_greedy_one_pass():
    # every row greedy: the one-pass finish on the fixed scratch's row slots and counter, two
    # calls in a row (the second smaller), against the selector
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    sel = t.Selector(262144, 64)
    rng = np.random.default_rng(8)
    for rows, n in [(64, 262144), (3, 20000)]:
        base = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
        base[1 % rows, [n - 1, 4]] = base.max() + 1.0  # a tie across slices
        params = [t.RowParams(0.0, 1.0, 0, 1.0, 0.0, 30.0, 0, 0) for _ in range(rows)]
        a = torch.from_numpy(base).to(dev)
        ta = torch.full((rows,), -7, dtype=torch.int32, device=dev)
        tb = torch.full((rows,), -7, dtype=torch.int32, device=dev)
        sel.select(a, params, None, ta, stream=stream)
        _noalloc(t, a, params, None, tb, stream)
        torch.cuda.synchronize()
        want = [int(np.argmax(base[m])) for m in range(rows)]
        assert ta.cpu().tolist() == want and tb.cpu().tolist() == want, (rows, n)
    sel.close()


def test_noalloc_rejects_sizes_beyond_its_scratch():
    import torch
    t = twd()
    dev = torch.device("cuda:0")
    lg = torch.zeros(1, 262145, dtype=torch.float32, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    p = [t.RowParams(0.0, 1.0, 0, 1.0, 0.0, 0.0, 0, 0)]
    with pytest.raises(t.TwdError) as e:
        _noalloc(t, lg, p, None, tok, None)
    assert e.value.code == t.TWD_E_INVALID and "262144" in str(e.value)
    lg = torch.zeros(65, 16, dtype=torch.float32, device=dev)
    tok = torch.zeros(65, dtype=torch.int32, device=dev)
    with pytest.raises(t.TwdError) as e:
        _noalloc(t, lg, p * 65, None, tok, None)
    assert e.value.code == t.TWD_E_INVALID and "64" in str(e.value)
