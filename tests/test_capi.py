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
    assert len(syms) == 46, syms
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


OPTION_FIELDS = ["max_tokens", "temperature", "top_p", "top_k", "repetition_penalty", "has_seed",
                 "seed", "system_prompt", "stop_strings", "stop_count", "tier_id"]


def _layout_of(tmp_path, include_lines, name):
    """sizeof and every field offset of G4DenseGenerationOptions as a C compiler sees it."""
    src = tmp_path / f"{name}.c"
    body = "\n".join(f'    printf("%zu\\n", offsetof(G4DenseGenerationOptions, {f}));'
                     for f in OPTION_FIELDS)
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n" + include_lines +
                   "\nint main(void) {\n    printf(\"%zu\\n\", sizeof(G4DenseGenerationOptions));\n"
                   + body + "\n    return 0;\n}\n")
    exe = tmp_path / name
    subprocess.run(["gcc", "-std=c11", "-I" + os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True, capture_output=True)
    return [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                           check=True).stdout.split()]


def test_generation_options_layout(tmp_path):
    # twd_head.h declares the reference's G4DenseGenerationOptions (c_api.h:24-36) when the
    # reference header is absent; both must give the same layout, and the ctypes mirror too
    t = twd()
    ours = _layout_of(tmp_path, '#include "twd_head.h"', "ours")
    ct = t.twd.GenerationOptions
    assert ours == [ctypes.sizeof(ct)] + [getattr(ct, f).offset for f in OPTION_FIELDS]
    ref_h = "/root/reference/include/g4dense/c_api.h"
    if os.path.exists(ref_h):
        theirs = _layout_of(tmp_path, f'#include "{ref_h}"', "theirs")
        assert ours == theirs
        # the reference header first, then ours: one declaration, no conflict
        both = _layout_of(tmp_path, f'#include "{ref_h}"\n#include "twd_head.h"', "both")
        assert both == theirs


def test_options_default_mirror():
    # g4dense_options_default's values (c_api.cpp:40-53 of the reference)
    t = twd()
    o = t.twd.options_default()
    assert (o.max_tokens, o.top_k, o.has_seed, o.seed, o.stop_count, o.tier_id) == (512, 64, 0, 0, 0, 1)
    assert np.float32(o.temperature) == np.float32(0.2) and np.float32(o.top_p) == np.float32(0.95)
    assert o.repetition_penalty == 1.0 and not o.system_prompt and not o.stop_strings


def test_generator_ex_argument_errors_without_gpu():
    t = twd()
    lib = t.twd.lib
    out = ctypes.c_void_p()
    o = t.twd.options_default()
    prompt = (ctypes.c_uint32 * 2)(1, 2)
    assert lib.twd_generator_create_ex(None, ctypes.byref(o), prompt, 2, None, 0,
                                       t.twd.TokenCallback(), None,
                                       ctypes.byref(out)) == t.twd.TWD_E_INVALID
    assert "null head" in t.twd.last_error()
    fin = ctypes.c_int()
    assert lib.twd_generator_sync(None, ctypes.byref(fin)) == t.twd.TWD_E_INVALID
    assert lib.twd_generator_stop_reason(None) == t.twd.STOP_NONE
    lib.twd_generator_cancel(None)  # a no-op on a null generator
    assert lib.twd_head_finish_state(None) is None
