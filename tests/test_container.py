"""The .g4dense container header (include/g4dense/format.hpp:26-110): validation on the host
against the reference's own validate_header (src/format.cpp:6-65) -- its messages as golden
vectors, and the reference build itself when present -- and, on the GPU, the LM-head load of
src/runner.cpp:423-443 and :488-497 checked against the oracle."""
import ctypes
import os
import sys

import numpy as np
import pytest

from helpers import ROOT, allclose_report, bf16_rne, container_header, twd, write_container

sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
from make_golden import HEADER_BASE, HEADER_END  # noqa: E402


def inspect(path):
    t = twd()
    info = t.ContainerInfo()
    rc = t.lib.twd_container_inspect(os.fsencode(str(path)), ctypes.byref(info))
    return rc, t.lib.twd_last_error().decode(), info


def test_header_validation_matches_reference_messages(golden, tmp_path):
    t = twd()
    for c in golden["container_headers"]:
        size = c["file_size"] or HEADER_END
        path = tmp_path / f"{c['case']}.g4dense"
        path.write_bytes(container_header(**{**HEADER_BASE, **c["fields"]}) + b"\0" * (size - 4096))
        rc, msg, info = inspect(path)
        if c["error"] is None:
            assert rc == 0, (c["case"], msg)
            assert info.vocab_size == 1024 and info.d_model == 256 and info.file_size == size
            assert info.final_logit_softcapping == 30.0 and info.lm_head_offset == 4096
        else:
            assert rc == t.TWD_E_INVALID and msg == c["error"], (c["case"], msg)


def test_header_validation_fuzz_against_reference_build(reference, tmp_path):
    rng = np.random.default_rng(12)
    t = twd()
    path = tmp_path / "fuzz.g4dense"
    for trial in range(300):
        f = dict(HEADER_BASE)
        for key in rng.choice(["magic", "version", "num_layers", "d_model", "d_ff", "vocab_size",
                               "embed_offset", "lm_head_offset", "layers"], size=2):
            if key == "layers":
                n = 60
                f["layer_offsets"] = [int(x) * int(rng.choice([1, 4096])) for x in
                                      rng.integers(0, 300, n)]
                f["layer_sizes"] = [int(x) for x in rng.integers(0, 3, n) * 4096]
            elif key in ("magic", "version"):
                f[key] = int(rng.choice([f[key], f[key] + 1, 0]))
            elif key == "num_layers":
                f[key] = int(rng.integers(0, 64))
            else:
                f[key] = int(rng.choice([0, 4096, 4097, 8192]))
        size = int(rng.choice([HEADER_END, 4096 * 100, 4096 * 300]))
        hdr = container_header(**f)
        path.write_bytes(hdr + b"\0" * (size - 4096))
        want = reference.validate_header(hdr, size)
        rc, msg, _ = inspect(path)
        if want is None:
            assert rc == 0, (trial, msg)
        else:
            assert rc == t.TWD_E_INVALID and msg == want, (trial, msg, want)


def test_short_or_missing_file(tmp_path):
    t = twd()
    rc, msg, _ = inspect(tmp_path / "missing.g4dense")
    assert rc == t.TWD_E_INVALID and "cannot open" in msg
    p = tmp_path / "short.g4dense"
    p.write_bytes(b"G4DN" * 10)
    rc, msg, _ = inspect(p)
    assert rc == t.TWD_E_INVALID and "4096-byte header" in msg


@pytest.mark.gpu
def test_head_load_matches_oracle(oracle, tmp_path):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    dev = torch.device("cuda:0")
    V, d = 1000, 640
    W, S, B = oracle.gen_lm_head(31, V, d)
    rng = np.random.default_rng(4)
    norm = bf16_rne(rng.uniform(0.5, 1.5, d).astype(np.float32))
    path = str(tmp_path / "tiny.g4dense")
    write_container(path, W, S, B, norm, V, d, softcap=25.0)
    assert t.container_info(path)["final_logit_softcapping"] == 25.0
    head = t.LMHead.load(path)
    assert head.vocab == V and head.d_model == d and head.softcap == 25.0
    # the container's head: plain bf16 h
    h = bf16_rne(rng.standard_normal((3, d)).astype(np.float32))
    got = head.logits(torch.from_numpy(h.view(np.int16)).to(dev)).cpu().numpy()
    want = np.stack([oracle.lm_head(W, S, B, (h[m].astype(np.uint32) << 16).view(np.float32), d,
                                    softcap=25.0) for m in range(3)])
    ratio, err, _ = allclose_report(got, want, 1e-3, 1e-3)
    assert ratio <= 1.0, (ratio, err)
    # and its final norm weight, through the RMSNorm prologue
    x = rng.uniform(-2, 2, (2, d)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    got = head.logits_rmsnorm(xd, head.norm_weight()).cpu().numpy()
    want = np.stack([oracle.lm_head(W, S, B, oracle.rmsnorm(x[m], norm, 1e-6), d, softcap=25.0)
                     for m in range(2)])
    ratio, err, _ = allclose_report(got, want, 1e-3, 1e-3)
    assert ratio <= 1.0, (ratio, err)
    head.close()


@pytest.mark.gpu
def test_head_load_rejections(oracle, tmp_path):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    V, d = 64, 128
    W, S, B = oracle.gen_lm_head(2, V, d)
    norm = bf16_rne(np.ones(d, np.float32))
    path = str(tmp_path / "bad.g4dense")
    write_container(path, W, S, B, norm, V, d, quant_type=2)
    with pytest.raises(t.TwdError) as e:
        t.LMHead.load(path)
    assert e.value.code == t.TWD_E_UNSUPPORTED
    write_container(path, W, S, B, norm, V, d, lm_head_size=4096)
    with pytest.raises(t.TwdError) as e:
        t.LMHead.load(path)
    assert e.value.code == t.TWD_E_INVALID and "exceeds header lm_head_size 4096" in str(e.value)


def test_head_load_rejects_offsets_past_the_file(oracle, tmp_path):
    # an LM-head offset near 2^64 must not wrap around the bounds check; the load fails on the
    # host before any device allocation
    t = twd()
    V, d = 64, 128
    W, S, B = oracle.gen_lm_head(2, V, d)
    norm = bf16_rne(np.ones(d, np.float32))
    path = str(tmp_path / "far.g4dense")
    write_container(path, W, S, B, norm, V, d, lm_head_offset=(1 << 64) - 4096, lm_head_size=1 << 40)
    out = ctypes.c_void_p()
    rc = t.lib.twd_head_load(os.fsencode(path), None, ctypes.byref(out))
    assert rc == t.TWD_E_INVALID and not out.value
    assert "extends beyond the file" in t.lib.twd_last_error().decode()
