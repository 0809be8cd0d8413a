"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each block names the reference test or the independent check it rests on. Nothing here needs a
GPU; the reference-build comparisons are skipped when oracle/_ref was not built.
"""
import hashlib
import math
import os
import sys

import numpy as np
import pytest

V = 262144
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def full_sort_sample(logits, t, p, k, u):
    """The naive full-sort sampler of tests/test_sampling.cpp:36-84, written independently:
    numpy lexsort for the order, libm exp (math.exp) and left-to-right Python sums."""
    lg = np.asarray(logits, np.float32)
    if t <= 0.0:
        return int(np.argmax(lg))  # first maximum, i.e. ties to the lower index
    key = lg.astype(np.float64) + 0.0  # folds -0 into +0 so it ties with +0
    order = np.lexsort((np.arange(lg.size), -key))
    best = float(lg[order[0]])
    total = 0.0
    for v in lg.tolist():
        total += math.exp(v - best)
    cut = lg.size
    if p < 1.0:
        run = 0.0
        for i, j in enumerate(order.tolist()):
            run += math.exp(float(lg[j]) - best) / total
            if run >= float(np.float32(p)):
                cut = i + 1
                break
    if k > 0:
        cut = min(cut, k)
    cut = max(1, cut)
    td = float(np.float32(t))
    q = [math.exp((float(lg[j]) - best) / td) for j in order[:cut].tolist()]
    denom = 0.0
    for x in q:
        denom += x
    r = float(np.float32(u)) * denom
    acc = 0.0
    for i, x in enumerate(q):
        acc += x
        if acc >= r:
            return int(order[i])
    return int(order[cut - 1])


# ---- splitmix64 / seed_for / uniform -----------------------------------------------------------

def test_splitmix64_known_answers(oracle):
    # tests/test_sampling.cpp:118-121
    assert oracle.splitmix64(0) == 0xE220A8397B1DCDAF
    assert oracle.splitmix64(1) == 0x910A2DEC89025CC1
    assert oracle.splitmix64(2) == 0x975835DE1C9756CE
    assert oracle.splitmix64(3) == 0x1D0B14E4DB018FED


def test_seed_for_properties(oracle):
    # tests/test_sampling.cpp:123-136: nonzero, stable, decorrelated
    seen = set()
    for pos in range(10000):
        a = oracle.seed_for(True, 12345, pos)
        assert a != 0 and a == oracle.seed_for(True, 12345, pos)
        seen.add(a)
    assert len(seen) == 10000
    assert oracle.seed_for(True, 12345, 5) != oracle.seed_for(True, 99, 5)


def test_seed_for_golden(oracle, golden):
    for x, want in golden["splitmix64"]:
        assert oracle.splitmix64(int(x)) == int(want)
    for has_seed, seed, pos, want in golden["seed_for"]:
        assert oracle.seed_for(bool(has_seed), int(seed), pos) == int(want)


def test_uniform_is_24_bit_fraction(oracle):
    for s in range(1, 2000):
        u = oracle.uniform_from_seed(oracle.splitmix64(s))
        assert 0.0 <= u < 1.0 and float(u * 16777216.0).is_integer()


# ---- validate_sampling ---------------------------------------------------------------------------

def test_validate_matrix(oracle):
    # tests/test_sampling.cpp:92-112
    ok = oracle.validate_sampling
    assert ok(0.2, 0.95, 64, 1.0) and ok(0.0, 1.0, 0, 1.0)
    assert not ok(-0.1, 1.0, 0, 1.0)
    assert not ok(0.2, 0.0, 64, 1.0)
    assert not ok(0.2, 1.5, 64, 1.0)
    assert not ok(0.2, 0.95, 257, 1.0)
    assert not ok(0.2, 0.95, -1, 1.0)
    assert not ok(0.2, 0.95, 64, 0.0)
    assert not ok(0.7, 0.9, 0, 1.0)
    assert ok(0.7, 1.0, 0, 1.0)
    assert ok(0.0, 0.9, 0, 1.0)


def test_validate_golden_grid(oracle, golden):
    for t, p, k, rp, want in golden["validate_sampling"]:
        assert oracle.validate_sampling(float(t), float(p), k, float(rp)) == want, (t, p, k, rp)


# ---- repetition penalty -------------------------------------------------------------------------

def test_penalty_known_answers(oracle):
    # tests/test_sampling.cpp:198-228
    lg = np.array([10.0, -10.0, 0.0, 29.999], np.float32)
    v = oracle.apply_repetition_penalty(lg, [0, 1, 3, 99999], 2.0, 30.0)
    assert abs(v[0] - 5.0) < 1e-5 and abs(v[1] + 20.0) < 1e-5 and v[2] == 0.0
    assert 14.9 < v[3] < 15.1
    assert np.all(np.abs(v) <= 30.0)
    assert np.array_equal(oracle.apply_repetition_penalty(lg, [0, 1, 3], 1.0, 30.0), lg)
    assert np.array_equal(oracle.apply_repetition_penalty(lg, [], 2.0, 30.0), lg)
    g = np.array([9.0, 8.0], np.float32)
    assert oracle.argmax(g) == 0
    assert oracle.argmax(oracle.apply_repetition_penalty(g, [0], 2.0, 30.0)) == 1


def test_penalty_duplicates_compound(oracle):
    # Brute force: n occurrences apply the single-occurrence op n times, each with the clamp.
    lg = np.array([3.0, -3.0, 29.0, -29.0, 0.5], np.float32)
    for rp in (1.1, 0.5, 2.0):
        once = lg.copy()
        for n in range(1, 6):
            once = oracle.apply_repetition_penalty(once, [0, 1, 2, 3, 4], rp, 30.0)
            many = oracle.apply_repetition_penalty(lg, [0, 1, 2, 3, 4] * n, rp, 30.0)
            assert np.array_equal(once, many)
    # rp < 1 grows |v|; the clamp caps it at 0.9999 * softcap
    big = oracle.apply_repetition_penalty(np.array([29.0], np.float32), [0] * 3, 0.5, 30.0)
    assert big[0] == np.float32(30.0) * np.float32(0.9999)


def test_penalty_golden(oracle, golden):
    for case in golden["penalty"]:
        _, seed, mean, sd, vocab, _, cap = case["gen"]
        lg = oracle.softcap(oracle.gen_mt19937_normal(seed, mean, sd, vocab), cap)
        assert sha(lg) == case["in_sha256"]
        got = oracle.apply_repetition_penalty(lg, case["history"], case["penalty"],
                                              case["softcap"])
        assert sha(got) == case["out_sha256"]
        if case["out_f32_hex"]:
            assert [f"{x:08x}" for x in got.view(np.uint32)] == case["out_f32_hex"]


# ---- greedy / shortlist / sample_token -------------------------------------------------------------

def test_greedy_ties_low_index(oracle):
    # tests/test_sampling.cpp:141-148
    assert oracle.sample_token([1.0, 5.0, 3.0, 5.0, 2.0], 0.0, 1.0, 0, seed=1) == 1
    assert oracle.sample_token([7.0], 0.0, 1.0, 0, seed=1) == 0
    # -0 and +0 tie: the first one wins either way round
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32)) == 0
    assert oracle.argmax(np.array([0.0, -0.0], np.float32)) == 0


def test_truncation_order_top_p_then_top_k(oracle):
    # tests/test_sampling.cpp:161-172
    lg = [3.0, 2.5, 2.0, 1.5, -1.0, -2.0, -3.0, -4.0]
    seen = {oracle.sample_token(lg, 1.0, 0.9, 2, seed=oracle.seed_for(True, 7, i))
            for i in range(4000)}
    assert seen == {0, 1}


def test_seed_determinism(oracle):
    # tests/test_sampling.cpp:177-193
    lg = oracle.gen_mt19937_normal(4242, 0.0, 4.0, 4096)
    a = [oracle.sample_token(lg, 0.8, 0.95, 64, seed=oracle.seed_for(True, 20260721, i))
         for i in range(64)]
    b = [oracle.sample_token(lg, 0.8, 0.95, 64, seed=oracle.seed_for(True, 20260721, i))
         for i in range(64)]
    c = [oracle.sample_token(lg, 0.8, 0.95, 64, seed=oracle.seed_for(True, 20260722, i))
         for i in range(64)]
    assert a == b and a != c


def test_shortlist_matches_lexsort(oracle):
    lg = oracle.gen_mt19937_normal(20260723, 0.0, 6.0, V)
    # plant exact ties and signed zeros so the index tie-break is exercised
    lg[1000:1010] = lg[5]
    lg[7] = 0.0
    lg[8] = -0.0
    order = np.lexsort((np.arange(V), -(lg.astype(np.float64) + 0.0)))
    for want in (1, 8, 40, 64, 256, 1000):
        assert np.array_equal(oracle.shortlist(lg, want), order[:want].astype(np.uint32))
    small = np.array([0.0, -0.0, 1.0, 1.0, -1.0], np.float32)
    assert list(oracle.shortlist(small, 5)) == [2, 3, 0, 1, 4]


@pytest.mark.slow
def test_sample_token_equals_full_sort(oracle):
    # tests/test_sampling.cpp:238-265, re-derived: heap shortlist vs an independent full sort
    lg = oracle.gen_mt19937_normal(20260723, 0.0, 6.0, V)
    cfgs = [(0.2, 0.95, 64, 1), (1.0, 0.90, 8, 2), (0.7, 1.00, 256, 3), (0.5, 1.00, 0, 4),
            (1.5, 0.99, 1, 5)]
    for t, p, k, s in cfgs:
        for i in range(3):
            u = oracle.uniform_from_seed(oracle.seed_for(True, s, i))
            assert oracle.sample_token(lg, t, p, k, u=u) == full_sort_sample(lg, t, p, k, u)


def test_sample_token_golden_full_vocab(oracle, golden):
    g = golden["shortlist_vs_full_sort"]
    _, seed, mean, sd, n = g["gen"]
    lg = oracle.gen_mt19937_normal(seed, mean, sd, n)
    assert sha(lg) == g["logits_sha256"]
    checked = 0
    for cfg in g["configs"]:
        for sd_str, want in cfg["draws"]:
            got = oracle.sample_token(lg, cfg["t"], cfg["p"], cfg["k"], seed=int(sd_str))
            assert got == want
            checked += 1
    assert checked == 200


def test_u_seam_equals_seed_path(oracle, golden):
    # The u-injection seam is the seed path with next_uniform factored out.
    c1 = golden["config1"]
    _, seed, mean, sd, n, _, cap = c1["gen"]
    z = oracle.softcap(oracle.gen_mt19937_normal(seed, mean, sd, n), cap)
    assert sha(z) == c1["logits_sha256"]
    assert oracle.sample_token(z, 0.0, 1.0, 0, seed=1) == c1["greedy"]
    for sd_str, want in c1["sampled"]:
        u = oracle.uniform_from_seed(int(sd_str))
        assert oracle.sample_token(z, 0.8, 0.95, 64, u=u) == want
        assert oracle.sample_token(z, 0.8, 0.95, 64, seed=int(sd_str)) == want


def test_penalised_sampling_golden(oracle, golden):
    for case in golden["penalised_sampling"]:
        _, seed, mean, sd, n, _, cap = case["gen"]
        z = oracle.softcap(oracle.gen_mt19937_normal(seed, mean, sd, n), cap)
        hist = np.random.default_rng(case["history_gen"][1]).integers(
            0, n, size=case["history_gen"][2], dtype=np.uint32)
        assert sha(hist) == case["history_sha256"]
        pz = oracle.apply_repetition_penalty(z, hist, case["rp"], cap)
        assert sha(pz) == case["penalised_sha256"]
        for sd_str, want in case["draws"]:
            assert oracle.sample_token(pz, case["t"], case["p"], case["k"],
                                       seed=int(sd_str)) == want


def test_degenerate_and_empty(oracle):
    with pytest.raises(RuntimeError):
        oracle.sample_token(np.full(8, -np.inf, np.float32), 0.7, 1.0, 0, seed=1)
    with pytest.raises(RuntimeError):
        oracle.sample_token(np.zeros(0, np.float32), 0.7, 1.0, 0, seed=1)


# ---- speculative verify -------------------------------------------------------------------------------

def test_verify_known_cases(oracle):
    # tests/test_speculative.cpp:29-77
    rows = [np.zeros(1024, np.float32) for _ in range(5)]
    for r, j in zip(rows, (42, 100, 200, 300, 400)):
        r[j] = 10.0
    full = oracle.verify([42, 100, 200, 300], rows, base_seed=12345)
    assert full["num_accepted"] == 4 and full["bonus_token"] == 400
    assert full["tokens"] == [42, 100, 200, 300, 400]
    part = oracle.verify([42, 100, 999, 300], rows, base_seed=12345)
    assert part["num_accepted"] == 2 and part["tokens"] == [42, 100, 200]
    miss = oracle.verify([999, 100], rows, base_seed=12345)
    assert miss["num_accepted"] == 0 and miss["tokens"] == [42]
    none = oracle.verify([], rows)
    assert none["tokens"] == [] and none["total_drafted"] == 0


def test_verify_golden(oracle, golden):
    for case in golden["verify"]:
        _, seed0, mean, sd, vocab, _, cap, nrows = case["rows_gen"]
        rows = [oracle.softcap(oracle.gen_mt19937_normal(seed0 + j, mean, sd, vocab), cap)
                for j in range(nrows)]
        got = oracle.verify(case["drafts"], rows, case["t"], case["p"], case["k"],
                            int(case["base_seed"]))
        want = case["result"]
        for key in ("tokens", "num_accepted", "total_drafted", "bonus_token_sampled"):
            assert got[key] == want[key], key
        if want["bonus_token_sampled"]:
            assert got["bonus_token"] == want["bonus_token"]
        assert got["acceptance_rate"] == want["acceptance_rate"]


# ---- against the reference build directly ------------------------------------------------------------

def test_reference_build_random_rows(oracle, reference):
    rng = np.random.default_rng(123)
    for trial in range(30):
        n = int(rng.integers(1, 3000))
        lg = (rng.standard_normal(n) * rng.uniform(0.5, 8)).astype(np.float32)
        if trial % 3 == 0:
            lg[rng.integers(0, n, size=max(1, n // 10))] = lg[0]  # ties
        t = float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.7]))
        p = float(rng.choice([1.0, 0.5, 0.9, 0.99]))
        k = int(rng.choice([0, 1, 5, 40, 256, 300]))
        seed = int(rng.integers(0, 2**63))
        assert oracle.sample_token(lg, t, p, k, seed=seed) == reference.sample_token(lg, t, p, k,
                                                                                       seed)
        hist = rng.integers(0, n + 5, size=int(rng.integers(0, 400)), dtype=np.uint32)
        rp = float(rng.choice([1.0, 1.1, 0.8, 2.0]))
        cap = float(rng.choice([0.0, 30.0]))
        a = oracle.apply_repetition_penalty(lg, hist, rp, cap)
        b = reference.apply_repetition_penalty(lg, hist, rp, cap)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_reference_build_verify(oracle, reference):
    rng = np.random.default_rng(9)
    for _ in range(40):
        vocab = int(rng.integers(2, 600))
        rows = [rng.standard_normal(vocab).astype(np.float32) for _ in range(int(rng.integers(1, 7)))]
        drafts = [int(np.argmax(r)) if rng.random() < 0.6 else int(rng.integers(0, vocab))
                  for r in rows[: int(rng.integers(0, 7))]]
        drafts += [int(rng.integers(0, vocab)) for _ in range(int(rng.integers(0, 2)))]
        t = float(rng.choice([0.0, 0.8]))
        base = int(rng.integers(0, 2**63))
        got = oracle.verify(drafts, rows, t, 0.9 if t else 1.0, 20 if t else 0, base)
        want = reference.verify(drafts, rows, t, 0.9 if t else 1.0, 20 if t else 0, 1.0, base)
        assert got == want


# ---- verify with draft logits: the rejection branch (speculator.cpp:14-30, :71-122) --------

def test_mt19937_64_known_answer(oracle):
    # [rand.predef]: the 10000th consecutive invocation of a default-constructed mt19937_64
    # produces 9981545732273789042
    assert oracle.mt64_outputs(5489, 10000)[-1] == 9981545732273789042
    assert oracle.std_mt64_10000th() == 9981545732273789042


def test_rejection_uniforms_match_libstdcxx(oracle):
    seeds = [oracle.splitmix64(i) for i in range(10000)] + [0, 1, 5489, 2**63, 2**64 - 1]
    std = oracle.std_rejection_uniforms(seeds)
    mine = np.array([oracle.rejection_uniforms(s) for s in seeds], np.float32)
    assert np.array_equal(std.view(np.uint32), mine.view(np.uint32))
    assert float(std.min()) >= 0.0 and float(std.max()) < 1.0


def test_canonical_float_closed_forms(oracle):
    assert oracle.canonical_float(0) == 0.0
    assert oracle.canonical_float(1 << 40) == 2.0 ** -24
    assert oracle.canonical_float(3 << 62) == 0.75
    below_one = float(np.nextafter(np.float32(1), np.float32(0)))
    # every x whose float rounds to 2^64 is clamped below 1
    for x in (2**64 - 1, 2**64 - 2**39, 2**64 - 2**40 + 1):
        assert oracle.canonical_float(x) == below_one
    assert oracle.canonical_float(2**64 - 2**40 - 2**39) < below_one


def test_softmax_closed_forms(oracle):
    # equal logits: every p is 1/n; T scales the logits first; T <= 0 means T = 1
    p = oracle.softmax(np.zeros(8, np.float32), 0.7)
    assert np.all(p == np.float32(1.0 / 8.0))
    two = np.array([0.0, np.log(3.0)], np.float32)
    q = oracle.softmax(two, 0.0)
    assert abs(float(q[1]) / float(q[0]) - 3.0) < 1e-6
    # all logits below -1e9: every exp underflows, the sum is 0 and the division uses 1
    z = oracle.softmax(np.full(4, -3e9, np.float32), 1.0)
    assert np.all(z == 0.0)


def _draft_case(golden_case):
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    from make_golden import draft_case_drafts, draft_case_rows
    c = golden_case
    rows = draft_case_rows(c["rows_seed"], c["vocab"], c["nrows"])
    drs = draft_case_drafts(c["rows_seed"], c["vocab"], rows, c["alpha"], c["draft_sd"], c["mask"])
    for r, j in zip(drs, c.get("nan_at", [])):
        r[j] = np.nan
    return rows, drs


def test_verify_draft_golden(oracle, golden):
    kinds = {"accepted": 0, "residual": 0, "fallback": 0}
    for c in golden["verify_draft"]:
        rows, drs = _draft_case(c)
        got = oracle.verify_draft(c["drafts"], rows, drs, c["t"], c["p"], c["k"], c["rp"],
                                  int(c["base_seed"]))
        for d in got.pop("diag"):
            if d is not None:
                kinds["accepted" if d["accepted"] else
                      ("fallback" if d["corr"] == 0xFFFFFFFF else "residual")] += 1
        assert got == c["result"], c
    assert min(kinds.values()) >= 5, kinds


def test_verify_draft_identical_rows_always_accept(oracle):
    # p == q elementwise gives r = p/q = 1 exactly, and every draw is < 1
    rng = np.random.default_rng(5)
    for trial in range(20):
        vocab = int(rng.integers(2, 3000))
        rows = [rng.standard_normal(vocab).astype(np.float32) * 3 for _ in range(4)]
        drafts = [int(rng.integers(0, vocab)) for _ in range(3)]
        got = oracle.verify_draft(drafts, rows, [r.copy() for r in rows[:3]], 0.9, 1.0, 0, 1.0,
                                  int(rng.integers(0, 2**63)))
        assert got["num_accepted"] == 3 and got["tokens"][:3] == drafts
        assert all(d["r"] == 1.0 for d in got["diag"])


def test_reference_build_verify_draft(oracle, reference):
    rng = np.random.default_rng(31)
    kinds = set()
    for case in range(150):
        vocab = int(rng.integers(2, 5000))
        K = int(rng.integers(1, 6))
        rows = [(rng.standard_normal(vocab) * rng.uniform(0.5, 4)).astype(np.float32)
                for _ in range(K + int(rng.integers(0, 2)))]
        drs = []
        for i in range(K):
            if rng.random() < 0.15:
                drs.append(None)
                continue
            mix = float(rng.uniform(0, 1))
            d = (mix * rows[min(i, len(rows) - 1)] +
                 (1 - mix) * rng.standard_normal(vocab) * 2).astype(np.float32)
            if rng.random() < 0.1:
                d = rows[min(i, len(rows) - 1)].copy()
                d[int(rng.integers(0, vocab))] = np.nan  # unnormalised q: the fallback
            drs.append(d)
        drafts = [int(np.argmax(rows[i])) if i < len(rows) and rng.random() < 0.5
                  else int(rng.integers(0, vocab)) for i in range(K)]
        t = float(rng.choice([0.0, 0.5, 0.8, 1.0, 1.3]))
        rp = float(rng.choice([1.0, 1.1]))
        k = int(rng.choice([0, 40]))
        p = 1.0 if k == 0 else 0.9
        base = int(rng.integers(0, 2**63))
        got = oracle.verify_draft(drafts, rows, drs, t, p, k, rp, base)
        for d in got.pop("diag"):
            if d is not None:
                kinds.add("a" if d["accepted"] else ("f" if d["corr"] == 0xFFFFFFFF else "r"))
        assert got == reference.verify_draft(drafts, rows, drs, t, p, k, rp, base), case
    assert kinds == {"a", "r", "f"}


# ---- final RMSNorm (cpu_reference.cpp:141-150) ----------------------------------------------

def _bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_rmsnorm_closed_forms(oracle):
    d = 5376
    one = _bf16(np.ones(d, np.float32))
    # a constant row c: mean square c^2, so every output is c / sqrt(c^2 + eps)
    for c in (2.0, -0.5, 0.125):  # c * c sums exactly in fp32
        out = oracle.rmsnorm(np.full(d, c, np.float32), one, 1e-6)
        want = c / math.sqrt(c * c + 1e-6)
        assert np.allclose(out, want, rtol=2e-6, atol=0)
    # a zero row stays zero; the weight scales elementwise
    assert np.all(oracle.rmsnorm(np.zeros(d, np.float32), one, 1e-6) == 0.0)
    w = _bf16(np.linspace(-2, 2, d).astype(np.float32))
    out = oracle.rmsnorm(np.full(d, 3.0, np.float32), w, 0.0)
    assert np.allclose(out, (w.astype(np.uint32) << 16).view(np.float32), rtol=1e-6, atol=0)


def test_rmsnorm_against_float64(oracle):
    # the reference kernel test's data (test_gpu_kernels.cpp:145-160) and its tolerance
    rng = np.random.default_rng(6)
    d = 5376
    x = rng.uniform(-2, 2, d).astype(np.float32)
    w = _bf16(rng.uniform(-2, 2, d).astype(np.float32) * 0.5 + 1.0)
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * wf
    got = oracle.rmsnorm(x, w, 1e-6)
    assert np.all(np.abs(got - want) <= 1e-4 + 1e-3 * np.abs(want))
    assert np.max(np.abs(got - want) / np.abs(want)) < 1e-5


# ---- LM head ---------------------------------------------------------------------------------------------

def _dequant_f64(W, S, B, d, group=64):
    """Independent float64 dequantisation: w[r, c] = q * s + b with nibble c%8 of word c/8."""
    shifts = (np.arange(d) % 8) * 4
    q = (W[:, np.arange(d) // 8] >> shifts.astype(np.uint32)) & 0xF
    s = (S.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    b = (B.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    g = np.arange(d) // group
    return q.astype(np.float64) * s[:, g] + b[:, g]


def test_lm_head_against_float64(oracle):
    d, rows = 5376, 96
    W, S, B = oracle.gen_lm_head(3, rows, d)
    h = np.random.default_rng(0).standard_normal(d).astype(np.float32)
    ref = _dequant_f64(W, S, B, d) @ h.astype(np.float64)
    f64 = oracle.lm_head_f64(W, S, B, h, d)
    assert np.allclose(f64, ref, rtol=1e-12, atol=1e-12)
    f32 = oracle.lm_head(W, S, B, h, d)
    assert np.allclose(f32, ref, rtol=1e-3, atol=1e-3)
    capped = oracle.lm_head(W, S, B, h, d, softcap=30.0)
    assert np.allclose(capped, 30.0 * np.tanh(ref / 30.0), rtol=1e-3, atol=1e-3)


def test_lm_head_reference_test_shape(oracle):
    # tests/test_gpu_kernels.cpp:259-353: 256 x 5376 rows, random words and bf16 scales/biases
    rng = np.random.default_rng(42)
    rows, d = 256, 5376
    W = rng.integers(0, 2**32, size=(rows, d // 8), dtype=np.uint64).astype(np.uint32)
    s = (np.abs(rng.uniform(-2, 2, size=(rows, 84))) * 0.05 + 0.01).astype(np.float32)
    b = (rng.uniform(-2, 2, size=(rows, 84)) * 0.05).astype(np.float32)
    S = (s.view(np.uint32) >> 16).astype(np.uint16)
    B = (b.view(np.uint32) >> 16).astype(np.uint16)
    x = (rng.uniform(-2, 2, size=d) * 0.1).astype(np.float32)
    ref = _dequant_f64(W, S, B, d) @ x.astype(np.float64)
    got = oracle.lm_head(W, S, B, x, d)
    assert np.allclose(got, ref, rtol=1e-3, atol=1e-3)


def test_gen_lm_head_formula(oracle):
    d, rows, row0, seed = 256, 5, 11, 77
    W, S, B = oracle.gen_lm_head(seed, rows, d, row0=row0)
    M = 0xFFFFFFFFFFFFFFFF
    for r in range(rows):
        for w in range(d // 8):
            i = (row0 + r) * (d // 8) + w
            assert int(W[r, w]) == oracle.splitmix64((seed + 0x1000000000000000 + i) & M) >> 32
    s = (S.astype(np.uint32) << 16).view(np.float32)
    b = (B.astype(np.uint32) << 16).view(np.float32)
    assert np.all((s >= 1e-3 * 0.99) & (s <= 1e-2 * 1.01))
    assert np.array_equal(b, -8.0 * s)
    # the rows are a pure function of the global row index
    W2, S2, B2 = oracle.gen_lm_head(seed, rows + row0, d)
    assert np.array_equal(W2[row0:], W) and np.array_equal(S2[row0:], S)


def _absorbed_tail_row(n=262144):
    # two equal maxima first, then a tail whose terms exp(-36.05) ~ 2.19e-16 each lie under half
    # an ulp of the running total 2.0 (2^-52 ~ 2.22e-16): the reference's in-order total drops
    # every one of them and stays exactly 2.0, while any tree of partial sums keeps ~5.7e-11 of
    # them. With p = 1/2 the first prefix, 1/total, is then exactly p in the reference.
    row = np.full(n, np.float32(-36.05), np.float32)
    row[:2] = 0.0
    return row


def test_absorbed_tail_total(oracle, reference):
    row = _absorbed_tail_row()
    terms = np.exp(row.astype(np.float64) - 0.0)
    assert np.cumsum(terms)[-1] == 2.0                    # in index order: every tail term drops
    assert np.sum(terms) - 2.0 > 5e-11                    # pairwise: the tail's mass survives
    # cut = 1 at p = 1/2, so the token is the first maximum whatever the draw; a total with the
    # tail's mass would put the cut at 2 and draw index 1 for u > 1/2
    for u in (0.25, 0.75, 0.999):
        assert oracle.sample_token(row, 1.0, 0.5, 0, u=u) == 0
    seed = next(s for s in range(1, 1000) if oracle.uniform_from_seed(s) > 0.5)
    assert reference.sample_token(row, 1.0, 0.5, 0, seed) == 0


def test_row_total_rounding_bound():
    # The device keeps a top-p cut away from p by (V + 2048) * 2^-52 (relative) unless it forms the
    # reference's own total; that allowance rests on the in-order double sum of V non-negative
    # terms lying within (V - 1) * 2^-53 of any other order's sum (each term of which is within a
    # few dozen roundings of exact). Rows built to approach the bound (tails just under half an
    # ulp of the running total, which the in-order sum drops) and ordinary rows.
    rng = np.random.default_rng(5)
    n = 262144
    rows = []
    for tail in (-36.05, -36.5, -38.0, -40.0):
        r = np.full(n, np.float32(tail), np.float32)
        r[:2] = 0.0
        rows.append(r)
    rows.append(rng.standard_normal(n).astype(np.float32) * 3)
    rows.append(np.sort(rng.standard_normal(n).astype(np.float32) * 5)[::-1].copy())
    worst = 0.0
    for r in rows:
        terms = np.exp(r.astype(np.float64) - float(r.max()))
        seq = np.cumsum(terms)[-1]                                # the reference's order
        blocked = np.sum(np.sum(terms.reshape(-1, 64), axis=1))   # per-64 records, then a tree
        pairwise = np.sum(terms)
        for other in (blocked, pairwise):
            rel = abs(other - seq) / seq
            worst = max(worst, rel / ((n - 1) * 2.0 ** -53))
            assert rel <= (n + 2048) * 2.0 ** -53
    # the tail rows reach a large part of the bound: it is not a loose estimate
    assert worst > 0.25


def test_nan_temperature_samples(oracle, reference):
    # sampling.cpp:97 takes the greedy branch only for temperature <= 0: a NaN temperature
    # samples, every weight exp((l - max) / T) is NaN, no running sum reaches u * denom, and the
    # token is the cut's last survivor (sampling.cpp:168)
    rng = np.random.default_rng(8)
    for trial in range(12):
        n = int(rng.integers(50, 3000))
        lg = (rng.standard_normal(n) * 3).astype(np.float32)
        p = float(rng.choice([1.0, 0.9, 0.5]))
        k = int(rng.choice([0, 1, 5, 40, 300]))
        seed = int(rng.integers(0, 2**63))
        got = oracle.sample_token(lg, float("nan"), p, k, seed=seed)
        assert got == reference.sample_token(lg, float("nan"), p, k, seed)
        assert got != int(np.argmax(lg)) or k == 1 or p == 0.5
