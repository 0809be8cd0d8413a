"""CPU checks of the C-ABI library: it loads, exports every declared entry point, and its host
side (seeding, validation, argument checks) agrees with the oracle. No GPU compute is run."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from helpers import ROOT, twd

HEADER = os.path.join(ROOT, "include", "twd_head.h")
LIB = os.path.join(ROOT, "turbo-winfare-dense_amd", "libtwd_head.so")


def declared_symbols():
    text = open(HEADER).read()
    return re.findall(r"TWD_API\s+[\w\s\*]+?\b(twd_\w+)\s*\(", text)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    syms = declared_symbols()
    assert len(syms) == 36, syms
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_cpp_dropin_symbols_exported():
    out = subprocess.run(["nm", "-DC", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    for sig in ["g4dense::sample_token(float const*, unsigned int, g4dense::SamplingParams const&, unsigned long)",
                "g4dense::apply_repetition_penalty(float*, unsigned int, std::vector<unsigned int, std::allocator<unsigned int> > const&, float, float)",
                "g4dense::seed_for(g4dense::SamplingParams const&, int)",
                "g4dense::splitmix64(unsigned long)",
                "g4dense::validate_sampling(g4dense::SamplingParams const&)",
                "g4dense::SpeculativeCoordinator::evaluate_verification("]:
        assert sig in out, sig


def test_host_seeding_matches_oracle(oracle):
    t = twd()
    for x in [0, 1, 2, 3, 12345, 2**63, 2**64 - 1]:
        assert t.splitmix64(x) == oracle.splitmix64(x)
    for seed in [0, 7, 12345]:
        for pos in [0, 1, 99, 4095, -1]:
            for has in (True, False):
                p = t.SamplingParams(has_seed=has, seed=seed)
                s = t.seed_for(p, pos)
                assert s == oracle.seed_for(has, seed, pos)
                assert t.uniform_from_seed(s) == oracle.uniform_from_seed(s)


def test_rejection_uniforms_match_oracle(oracle):
    # host-side draws of the rejection branch: the library's std::mt19937_64 +
    # uniform_real_distribution<float> against the oracle's restatement
    t = twd()
    for i in range(2000):
        seed = oracle.splitmix64(i * 7919)
        assert t.rejection_uniforms(seed) == oracle.rejection_uniforms(seed)


def test_verify_draft_argument_checks():
    t = twd()
    res = ctypes.c_void_p(16)
    rp = t.RowParams(0.8, 1.0, 0, 1.0, 0.0, 0.0, 0, 0)
    assert t.lib.twd_verify_draft(None, None, 10, 1, 10, None, 0, ctypes.byref(rp), 0, None, 0,
                                  res, None) == t.TWD_E_INVALID
    assert b"null selector" in t.lib.twd_last_error()


def test_host_validation_matches_golden(golden):
    t = twd()
    for tt, p, k, rp, want in golden["validate_sampling"]:
        ok = True
        try:
            t.validate_sampling(t.SamplingParams(float(tt), float(p), k, float(rp)))
        except t.G4DenseFormatError:
            ok = False
        assert ok == want


def test_argument_errors_without_gpu():
    t = twd()
    lib = t.twd.lib
    assert lib.twd_head_logits(None, None, 1, None, None) == t.twd.TWD_E_INVALID
    assert "null" in t.twd.last_error()
    assert lib.twd_head_greedy(None, None, 1, None, None, None) == t.twd.TWD_E_INVALID
    assert lib.twd_select(None, None, 1, 1, 1, None, None, None, None) == t.twd.TWD_E_INVALID
    out = ctypes.c_void_p()
    assert lib.twd_head_create(None, 0, 1, 128, 64, 30.0, ctypes.byref(out)) == t.twd.TWD_E_INVALID
    buf = np.zeros(16, np.uint8)
    assert lib.twd_head_create(buf.ctypes.data, 16, 16, 100, 64, 30.0,
                               ctypes.byref(out)) == t.twd.TWD_E_UNSUPPORTED
    assert lib.twd_head_create(buf.ctypes.data, 16, 16, 128, 32, 30.0,
                               ctypes.byref(out)) == t.twd.TWD_E_UNSUPPORTED
    assert lib.twd_head_create(buf.ctypes.data, 16, 16, 128, 64, 30.0,
                               ctypes.byref(out)) == t.twd.TWD_E_INVALID  # too few bytes
    assert lib.twd_head_create(buf.ctypes.data, 16, (1 << 30) + 1, 128, 64, 30.0,
                               ctypes.byref(out)) == t.twd.TWD_E_UNSUPPORTED
    assert "2^30" in t.twd.last_error()
    assert t.head_bytes(262144, 5376) == 792723456


def test_head_bytes_matches_reference_size():
    # docs/FORWARD_PASS.md:55 of the reference: 792,723,456 B for V=262144, d=5376
    t = twd()
    assert t.head_bytes(262144, 5376) == 262144 * (2688 + 168 + 168)


def test_generator_and_probe_argument_errors_without_gpu():
    t = twd()
    lib = t.twd.lib
    out = ctypes.c_void_p()
    gp = t.twd.GenerationParams(0.7, 0.9, 40, 1.1, 1, 5, 16)
    prompt = (ctypes.c_uint32 * 2)(1, 2)
    assert lib.twd_generator_create(None, ctypes.byref(gp), prompt, 2, None, 0,
                                    ctypes.byref(out)) == t.twd.TWD_E_INVALID
    assert "null head" in t.twd.last_error()
    tok, fin = ctypes.c_uint32(), ctypes.c_int()
    assert lib.twd_generator_step(None, None, None, ctypes.byref(tok),
                                  ctypes.byref(fin)) == t.twd.TWD_E_INVALID
    assert "null generator" in t.twd.last_error()
    us, nb = ctypes.c_float(), ctypes.c_uint64()
    assert lib.twd_probe_read_bandwidth(None, 1 << 20, 64, 1, None, ctypes.byref(us),
                                        ctypes.byref(nb)) == t.twd.TWD_E_INVALID
    buf = np.zeros(16, np.uint8)
    # waves must be a multiple of 8, and each stripe at least 1 KB
    assert lib.twd_probe_read_bandwidth(buf.ctypes.data, 1 << 20, 12, 1, None, ctypes.byref(us),
                                        ctypes.byref(nb)) == t.twd.TWD_E_INVALID
    assert lib.twd_probe_read_bandwidth(buf.ctypes.data, 4096, 8, 1, None, ctypes.byref(us),
                                        ctypes.byref(nb)) == t.twd.TWD_E_INVALID
    assert "stripes" in t.twd.last_error()
