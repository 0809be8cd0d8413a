"""The device builds of the two libm restatements against the host C library, bit for bit:
exp(double) of the sampled shortlist (csrc/exp_libm.h; std::exp(double) at sampling.cpp:145,157)
over the shortlist's argument families and random arguments, and the specials. (The draft
verify's expf has its own device check in test_gpu_verify_draft.py.)"""
import numpy as np
import pytest

from helpers import twd

pytestmark = pytest.mark.gpu


def test_device_exp_matches_host(oracle):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(11)
    l = (-60.0 * rng.random(1 << 21)).astype(np.float32)
    mx = (-60.0 * rng.random(1 << 21)).astype(np.float32)
    lo, hi = np.minimum(l, mx), np.maximum(l, mx)
    x0 = lo.astype(np.float64) - hi.astype(np.float64)            # exp(l - max)
    T = (0.05 + 1.95 * rng.random(1 << 21)).astype(np.float32)
    x1 = x0 / T.astype(np.float64)                                  # exp((l - max) / T)
    x2 = -745.2 * rng.random(1 << 21)                               # every nonzero result of x <= 0
    x3 = -1100.0 + 1900.0 * rng.random(1 << 20)                     # past both ends
    inv = 1.4426950408889634 * 128
    k = np.arange(-95000, 90000, 7, dtype=np.float64)
    half = ((k + 0.5) / inv).view(np.int64)
    x4 = np.concatenate([(half + d).view(np.float64) for d in (-2, -1, 0, 1, 2)])
    x5 = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 2.0**-54, -2.0**-54, 709.782712893384,
                   709.79, -708.4, -745.1332191019411, -745.14, 512.0, -512.0, 1024.0, -1024.0])
    for x in (x0, x1, x2, x3, x4, x5):
        got = t.twd.probe_exp(torch.from_numpy(x).to(dev)).cpu().numpy()
        want = oracle.exp(x)
        both_nan = np.isnan(got) & np.isnan(want)
        bad = (got.view(np.uint64) != want.view(np.uint64)) & ~both_nan
        assert not bad.any(), (int(bad.sum()), x[bad][:5], got[bad][:5], want[bad][:5])
