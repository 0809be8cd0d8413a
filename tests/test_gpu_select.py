"""GPU parity of the selection kernel (repetition penalty, greedy, top-p -> top-k -> temperature
draw, verify) against the reference's golden ids and the CPU oracle. Token ids and penalised
logits are compared bit-exactly. For sampled draws the oracle's cut and draw margins are
recorded for the run's summary line; a decision within the summation's rounding of its
threshold is taken with the reference's own additions and row total, so none may differ."""
import hashlib
import os
import subprocess

import numpy as np
import pytest

from helpers import ROOT, twd

pytestmark = pytest.mark.gpu

V = 262144


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def env():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    return torch, torch.device("cuda:0"), t, t.Selector(V, 65)


def select_rows(env, rows_np, params, history=None):
    torch, dev, t, sel = env
    lg = torch.from_numpy(np.ascontiguousarray(rows_np, np.float32)).to(dev)
    hist = None if history is None else torch.from_numpy(
        np.ascontiguousarray(history, np.uint32).view(np.int32)).to(dev)
    tok = sel.select(lg, params, hist)
    return (tok.cpu().numpy().astype(np.int64) & 0xFFFFFFFF), lg.cpu().numpy()


def rp(t, T, p, k, u, rep=1.0, cap=0.0, off=0, n=0):
    return t.RowParams(T, p, k, rep, u, cap, off, n)


def test_golden_shortlist_full_vocab(env, oracle, golden):
    # tests/test_sampling.cpp:238-265: 5 configs x 40 seeds at V=262144, ids from the reference
    torch, dev, t, sel = env
    g = golden["shortlist_vs_full_sort"]
    lg = oracle.gen_mt19937_normal(*g["gen"][1:])
    assert sha(lg) == g["logits_sha256"]
    for cfg in g["configs"]:
        draws = cfg["draws"]
        for start in range(0, len(draws), 20):  # 20 rows per launch
            chunk = draws[start:start + 20]
            params = [rp(t, cfg["t"], cfg["p"], cfg["k"], t.uniform_from_seed(int(s)))
                      for s, _ in chunk]
            tok, _ = select_rows(env, np.tile(lg, (len(chunk), 1)), params)
            assert [int(x) for x in tok] == [w for _, w in chunk], cfg


def test_golden_config1(env, oracle, golden):
    torch, dev, t, sel = env
    c1 = golden["config1"]
    _, seed, mean, sd, n, _, cap = c1["gen"]
    z = oracle.softcap(oracle.gen_mt19937_normal(seed, mean, sd, n), cap)
    assert sha(z) == c1["logits_sha256"]
    tok, _ = select_rows(env, z[None], [rp(t, 0.0, 1.0, 0, 0.0)])
    assert int(tok[0]) == c1["greedy"]
    draws = c1["sampled"]
    for start in range(0, len(draws), 32):
        chunk = draws[start:start + 32]
        params = [rp(t, 0.8, 0.95, 64, t.uniform_from_seed(int(s))) for s, _ in chunk]
        tok, _ = select_rows(env, np.tile(z, (len(chunk), 1)), params)
        assert [int(x) for x in tok] == [w for _, w in chunk]
    # the fixed-uniform pass of BASELINE config 1 (u = 0.37): oracle through the u seam
    tok, _ = select_rows(env, z[None], [rp(t, 0.8, 0.95, 64, 0.37)])
    want, diag = oracle.sample_token(z, 0.8, 0.95, 64, u=0.37, diag=True)
    print("config1 u=0.37 margins", diag["cut_margin"], diag["draw_margin"])
    assert int(tok[0]) == want


def test_golden_penalised_sampling(env, oracle, golden):
    torch, dev, t, sel = env
    for case in golden["penalised_sampling"]:
        _, seed, mean, sd, n, _, cap = case["gen"]
        z = oracle.softcap(oracle.gen_mt19937_normal(seed, mean, sd, n), cap)
        hist = np.random.default_rng(case["history_gen"][1]).integers(
            0, n, size=case["history_gen"][2], dtype=np.uint32)
        draws = case["draws"]
        params = [rp(t, case["t"], case["p"], case["k"], t.uniform_from_seed(int(s)), case["rp"],
                     cap, 0, len(hist)) for s, _ in draws]
        tok, pen = select_rows(env, np.tile(z, (len(draws), 1)), params, hist)
        for r in range(len(draws)):
            assert sha(pen[r]) == case["penalised_sha256"], "penalised logits differ"
        assert [int(x) for x in tok] == [w for _, w in draws], case["gen"]


def test_penalty_bit_exact_random(env, oracle):
    torch, dev, t, sel = env
    rng = np.random.default_rng(5)
    rows, params, hist_all, off = [], [], [], 0
    for r in range(24):
        n = int(rng.choice([1, 7, 1000, 16384, 16385, 40000]))
        row = (rng.standard_normal(n) * rng.uniform(1, 20)).astype(np.float32)
        row = oracle.softcap(row, 30.0) if r % 2 else row
        hlen = int(rng.integers(0, 3000))
        h = rng.integers(0, n + 3, size=hlen, dtype=np.uint32)  # out-of-range ids included
        if hlen and r % 3 == 0:
            h[: hlen // 2] = h[0]  # heavy duplicates compound
        rows.append(row)
        rep = float(rng.choice([1.1, 0.7, 2.0, 1.0]))
        cap = float(rng.choice([30.0, 0.0]))
        params.append((rep, cap, off, hlen, n))
        hist_all.append(h)
        off += hlen
    hist = np.concatenate(hist_all) if off else np.zeros(1, np.uint32)
    for row, (rep, cap, o, hlen, n), h in zip(rows, params, hist_all):
        p = rp(t, 0.0, 1.0, 0, 0.0, rep, cap, o, hlen)
        tok, pen = select_rows(env, row[None], [p], hist)
        want = oracle.apply_repetition_penalty(row, h, rep, cap)
        assert np.array_equal(pen[0].view(np.uint32), want.view(np.uint32))
        assert int(tok[0]) == oracle.argmax(want)


def test_penalty_sampled_rows(env, oracle):
    # sampled rows take the penalty pass over a per-row hash of the history (<= 4096 ids) and
    # fall back to the slice kernels past that: duplicates (one id 4096 times), ids past the
    # vocabulary, lengths at and past the limit, penalties below and above 1, with and without
    # the softcap clamp; penalised rows bit-exact, tokens against the oracle
    torch, dev, t, sel = env
    rng = np.random.default_rng(77)
    hashed = [(1, 1.1, 30.0), (4096, 1.3, 30.0), (3000, 0.7, 0.0), (4096, 2.0, 30.0),
              (2048, 1.1, 30.0), (0, 1.5, 30.0), (4096, 1.05, 0.0)]
    fallback = [(10, 1.1, 30.0), (4096, 1.3, 30.0), (4097, 1.3, 30.0)]  # one row past the limit
    for n, cases in ((1000, hashed), (40000, hashed), (V, hashed), (V, fallback)):
        rows, params, hists, off = [], [], [], 0
        for c, (hlen, rep, cap) in enumerate(cases):
            row = (rng.standard_normal(n) * 4.0).astype(np.float32)
            row = oracle.softcap(row, 30.0) if c % 2 else row
            h = rng.integers(0, n + 5, size=hlen, dtype=np.uint32)  # out-of-range ids included
            if c == 1:
                h[:] = h[0] % n  # one id, 4096 occurrences
            elif hlen and c % 3 == 0:
                h[: hlen // 2] = h[0]
            rows.append(row)
            params.append(rp(t, 0.8, 0.95, 50, float(rng.uniform()), rep, cap, off, hlen))
            hists.append(h)
            off += hlen
        hist = np.concatenate([h for h in hists if len(h)])
        tok, pen = select_rows(env, np.stack(rows), params, hist)
        for m, (row, h, p) in enumerate(zip(rows, hists, params)):
            want_pen = oracle.apply_repetition_penalty(row, h, p.repetition_penalty, p.softcap)
            assert np.array_equal(pen[m].view(np.uint32), want_pen.view(np.uint32)), (n, m)
            want, dg = oracle.sample_token(want_pen, p.temperature, p.top_p, p.top_k, u=p.uniform,
                                           diag=True)
            assert int(tok[m]) == want, (n, m, dg["cut_margin"], dg["draw_margin"])


@pytest.mark.parametrize("n", [1, 5, 100, 16384, 16385, 50000, V])
def test_select_random_vs_oracle(env, oracle, n):
    torch, dev, t, sel = env
    rng = np.random.default_rng(n)
    configs = [(0.7, 0.9, 40), (0.8, 0.95, 64), (1.0, 1.0, 0), (0.5, 1.0, 256), (1.2, 0.98, 100),
               (0.3, 0.5, 1), (2.0, 0.999, 256), (0.0, 1.0, 0), (1.0, 0.9, 8), (0.9, 1.0, 3)]
    rows, params, want = [], [], []
    worst = np.inf
    for i, (T, p, k) in enumerate(configs * 2):
        row = (rng.standard_normal(n) * rng.uniform(0.5, 8)).astype(np.float32)
        if i % 4 == 1 and n > 10:
            row[rng.integers(0, n, size=max(2, n // 50))] = row.max()  # ties at the top
        if i % 4 == 2 and n > 10:
            row[:5] = 0.0
            row[5:10] = -0.0
        if i % 4 == 3:
            row = np.round(row)  # many exact ties everywhere
        u = t.uniform_from_seed(t.splitmix64(1000 * n + i))
        rows.append(row)
        params.append(rp(t, T, p, k, u))
        w, diag = oracle.sample_token(row, T, p, k, u=u, diag=True)
        want.append(w)
        worst = min(worst, diag["cut_margin"], diag["draw_margin"])
    tok, _ = select_rows(env, np.stack(rows), params)
    print(f"n={n} smallest oracle margin {worst:.3e}")
    assert [int(x) for x in tok] == want


def shaped_rows(rng, n):
    """Rows whose values stress the distance-from-max shortlist: every branch of the kernel's
    top-`want` (direct ranking of the boundary bin, radix inside an overfull bin, radix over an
    unbinnable block, all entries) must give the oracle's ids."""
    base = (rng.standard_normal(n) * 3).astype(np.float32)
    out = {"all_equal": np.full(n, 1.25, np.float32)}
    gap = base.copy()
    gap[rng.integers(0, n, 3)] = 100.0  # a few entries far above the rest
    out["huge_gap"] = gap
    out["plateaus"] = np.round(base * 2) / 2  # every bin boundary holds exact ties
    masked = np.full(n, -np.inf, np.float32)
    keep = rng.integers(0, n, max(1, n // 10))
    masked[keep] = base[keep]
    out["mostly_minus_inf"] = masked
    few = np.full(n, -np.inf, np.float32)
    few[rng.integers(0, n, 7)] = rng.standard_normal(7).astype(np.float32)
    out["seven_finite"] = few
    out["narrow"] = (1.0 + rng.standard_normal(n) * 1e-4).astype(np.float32)
    crowd = base.copy()
    crowd[rng.integers(0, n, min(n, 5000))] = base.max()  # an overfull bin at the very top
    out["crowded_top"] = crowd
    wide = (rng.standard_normal(n) * 400).astype(np.float32)  # span far beyond the binned range
    out["wide"] = wide
    return out


@pytest.mark.parametrize("n", [300, 16384, 50000, V])
def test_select_shaped_rows_vs_oracle(env, oracle, n):
    torch, dev, t, sel = env
    rng = np.random.default_rng(77 + n)
    configs = [(0.7, 1.0, 0), (0.8, 0.95, 64), (1.0, 0.9, 256), (0.5, 1.0, 1), (1.5, 0.999, 100)]
    rows, params, want, names = [], [], [], []
    for name, row in shaped_rows(rng, n).items():
        for j, (T, p, k) in enumerate(configs):
            u = t.uniform_from_seed(t.splitmix64(31 * n + 7 * j + len(rows)))
            rows.append(row)
            params.append(rp(t, T, p, k, u))
            want.append(oracle.sample_token(row, T, p, k, u=u))
            names.append((name, T, p, k))
    for start in range(0, len(rows), 64):
        tok, _ = select_rows(env, np.stack(rows[start:start + 64]), params[start:start + 64])
        for got, w, nm in zip(tok, want[start:start + 64], names[start:start + 64]):
            assert int(got) == w, nm


def test_rows_with_own_params_and_histories(env, oracle):
    # config 5 style: 64 rows, own T/k/p, own 2048-id history with rp 1.1, own uniform
    torch, dev, t, sel = env
    rng = np.random.default_rng(55)
    rows = oracle.softcap((rng.standard_normal((64, V)) * 2.5).astype(np.float32), 30.0)
    hists = [rng.integers(0, V, 2048, dtype=np.uint32) for _ in range(64)]
    params = []
    for m in range(64):
        params.append(rp(t, float(np.float32(rng.uniform(0.5, 1.2))), float(np.float32(rng.uniform(0.8, 0.98))),
                         int(rng.integers(20, 101)), t.uniform_from_seed(t.splitmix64(m)), 1.1,
                         30.0, 2048 * m, 2048))
    tok, pen = select_rows(env, rows, params, np.concatenate(hists))
    for m in range(64):
        want_pen = oracle.apply_repetition_penalty(rows[m], hists[m], 1.1, 30.0)
        assert np.array_equal(pen[m].view(np.uint32), want_pen.view(np.uint32))
        p = params[m]
        assert int(tok[m]) == oracle.sample_token(want_pen, p.temperature, p.top_p, p.top_k,
                                                  u=p.uniform)


@pytest.mark.parametrize("n", [8193, 16384, 50000, V])
def test_greedy_one_pass_vs_oracle(env, oracle, n):
    # every row greedy and more than one slice: the slice blocks finish the rows (returning
    # atomic max per row, an epoch-armed arrival count); called three times in a row so the
    # counter is met both unarmed and armed. The reference's strict '>' scan: ties go to the
    # lowest index across slices, -0 and +0 tie, NaN is skipped except at index 0, all -inf
    # gives 0; penalised greedy rows take the penalty first (sampling.cpp:74-104)
    torch, dev, t, sel = env
    rng = np.random.default_rng(4000 + n)
    rows, params, hist_parts = [], [], []
    base = (rng.standard_normal((8, n)) * 3).astype(np.float32)
    r0 = base[0]
    r1 = base[1].copy()
    top = r1.max() + 1.0
    r1[[n - 1, 8200 % n, 5]] = top                        # ties in several slices
    r2 = base[2].copy()
    r2[:] = -np.abs(r2)
    r2[n - 3] = 0.0
    r2[9000 % n] = -0.0                                   # -0 and +0 tie at the top
    r3 = base[3].copy()
    r3[0] = np.nan                                        # NaN at index 0 -> 0
    r4 = base[4].copy()
    r4[rng.integers(0, n, 20)] = np.nan                   # NaN elsewhere is skipped
    r5 = np.full(n, -np.inf, np.float32)                  # all -inf -> 0
    r6 = base[6]
    r7 = base[7]
    hist = rng.integers(0, n + 5, 700).astype(np.uint32)
    hist[:40] = np.argsort(-r6)[:40]                      # penalise the current leaders
    for i, row in enumerate([r0, r1, r2, r3, r4, r5, r6, r7]):
        rows.append(row)
        if i in (6, 7):
            params.append(rp(t, 0.0, 1.0, 0, 0.0, rep=1.3 if i == 6 else 0.7, cap=30.0, off=0, n=700))
        else:
            params.append(rp(t, 0.0, 1.0, 0, 0.0))
    want = []
    for i, row in enumerate(rows):
        x = row
        if i in (6, 7):
            x = oracle.apply_repetition_penalty(row, hist, 1.3 if i == 6 else 0.7, 30.0)
        want.append(oracle.argmax(x))
    for rep_ in range(3):
        tok, _ = select_rows(env, np.stack(rows), params, history=hist)
        assert [int(x) for x in tok] == want, (n, rep_)


def test_degenerate_rows(env):
    torch, dev, t, sel = env
    nan_row = np.zeros(5000, np.float32)
    nan_row[1234] = np.nan
    inf_row = np.full(5000, -np.inf, np.float32)
    nan0 = np.full(300, 2.0, np.float32)
    nan0[0] = np.nan
    nan_mid = np.arange(300, dtype=np.float32)
    nan_mid[299] = np.nan
    tok, _ = select_rows(env, nan_row[None], [rp(t, 0.7, 1.0, 0, 0.5)])
    assert int(tok[0]) == t.twd.TOKEN_DEGENERATE
    tok, _ = select_rows(env, inf_row[None], [rp(t, 0.7, 1.0, 0, 0.5)])
    assert int(tok[0]) == t.twd.TOKEN_DEGENERATE
    # greedy follows the reference's strict '>' scan: all -inf -> 0, NaN at 0 -> 0, NaN skipped
    tok, _ = select_rows(env, inf_row[None], [rp(t, 0.0, 1.0, 0, 0.0)])
    assert int(tok[0]) == 0
    tok, _ = select_rows(env, nan0[None], [rp(t, 0.0, 1.0, 0, 0.0)])
    assert int(tok[0]) == 0
    tok, _ = select_rows(env, nan_mid[None], [rp(t, 0.0, 1.0, 0, 0.0)])
    assert int(tok[0]) == 298


def test_verify_selector_golden(env, oracle, golden):
    torch, dev, t, sel = env
    for case in golden["verify"]:
        _, seed0, mean, sd, vocab, _, cap, nrows = case["rows_gen"]
        rows = np.stack([oracle.softcap(oracle.gen_mt19937_normal(seed0 + j, mean, sd, vocab), cap)
                         for j in range(nrows)])
        lg = torch.from_numpy(rows).to(dev)
        drafts = case["drafts"]
        d = torch.tensor(drafts if drafts else [0], dtype=torch.int32, device=dev)[: len(drafts)]
        p = rp(t, case["t"], case["p"], case["k"], 0.0)
        got = t.decode_verify(sel.verify(lg, p, int(case["base_seed"]), d if drafts else None))
        want = case["result"]
        for key in ("tokens", "num_accepted", "total_drafted", "bonus_token_sampled"):
            assert got[key] == want[key], (key, got, want)


def test_python_mirror_api(env, oracle):
    torch, dev, t, sel = env
    lg = torch.tensor([1.0, 5.0, 3.0, 5.0, 2.0], device=dev)
    assert t.sample_token(lg, 5, t.SamplingParams(), 1) == 1
    v = torch.tensor([10.0, -10.0, 0.0, 29.999], device=dev)
    t.apply_repetition_penalty(v, 4, [0, 1, 3, 99999], 2.0, 30.0)
    want = oracle.apply_repetition_penalty(np.array([10.0, -10.0, 0.0, 29.999], np.float32),
                                           [0, 1, 3, 99999], 2.0, 30.0)
    assert np.array_equal(v.cpu().numpy(), want)
    rows = torch.zeros(5, 1024, device=dev)
    for i, j in enumerate((42, 100, 200, 300, 400)):
        rows[i, j] = 10.0
    sc = t.SpeculativeCoordinator()
    r = sc.evaluate_verification([42, 100, 999, 300], rows, 1024, t.SamplingParams(), 12345)
    assert r["tokens"] == [42, 100, 200] and r["num_accepted"] == 2


def test_cpp_dropin_program():
    exe = os.path.join(ROOT, "tests", "cpp", "test_dropin")
    assert os.path.exists(exe), "build() compiles tests/cpp/test_dropin"
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(res.stdout, res.stderr)
    assert res.returncode == 0 and "ALL OK" in res.stdout


@pytest.mark.parametrize("n", [1000, V])
def test_plus_inf_rows(env, oracle, n):
    # A row holding +inf has exp(+inf - max) = exp(NaN) in sample_token's total
    # (sampling.cpp:112-115), so the total is NaN and the reference throws (:116-118): the device
    # reports the degenerate id. Greedy takes the first +inf (strict '>', :97-104). A +inf that
    # the penalty clamps to 0.9999 * cap (:79-87) is finite again and samples normally.
    torch, dev, t, sel = env
    rng = np.random.default_rng(77 + n)
    base = (rng.standard_normal(n) * 3).astype(np.float32)
    one = base.copy()
    one[n // 3] = np.inf
    two = base.copy()
    two[[n // 5, n - 2]] = np.inf
    both = base.copy()
    both[[3, n // 2]] = [np.inf, -np.inf]
    rows = [one, two, both, two, one]
    params = [rp(t, 0.8, 0.95, 64, 0.37), rp(t, 1.0, 1.0, 0, 0.5), rp(t, 0.7, 0.9, 40, 0.1),
              rp(t, 0.0, 1.0, 0, 0.0), rp(t, 0.0, 1.0, 0, 0.0)]
    tok, _ = select_rows(env, np.stack(rows), params)
    for i in range(3):
        with pytest.raises(RuntimeError):
            oracle.sample_token(rows[i], params[i].temperature, params[i].top_p, params[i].top_k,
                                u=params[i].uniform)
        assert int(tok[i]) == t.TOKEN_DEGENERATE, i
    assert int(tok[3]) == n // 5 == oracle.argmax(two)
    assert int(tok[4]) == n // 3 == oracle.argmax(one)
    # the penalty clamps the +inf of an id in the history, after which the row is finite
    hist = np.array([n // 3, 5, n // 3], np.uint32)
    p = [rp(t, 0.8, 0.95, 64, 0.37, rep=1.1, cap=30.0, off=0, n=3)]
    tok, pen = select_rows(env, one[None, :], p, history=hist)
    want_pen = oracle.apply_repetition_penalty(one, hist, 1.1, 30.0)
    assert np.isfinite(want_pen).all()
    assert np.array_equal(pen[0].view(np.uint32), want_pen.view(np.uint32))
    assert int(tok[0]) == oracle.sample_token(want_pen, 0.8, 0.95, 64, u=0.37)


@pytest.mark.ties
@pytest.mark.parametrize("case", ["cut_on_p", "draw_on_r", "cut_and_draw", "near_tie"])
def test_prefix_sums_that_land_on_their_threshold(env, oracle, case):
    # Steps 5-7 decide by prefix sums compared with p (the top-p cut) and with u * denom (the
    # draw). Rows built so that a prefix equals its threshold exactly (or lies within a few ulp
    # of it) leave no margin between the reference's running sums and any other order of
    # additions, so the device must decide them with the reference's additions.
    torch, dev, t, sel = env
    n = 4096
    rows, params = [], []
    for s in range(8):
        row = np.full(n, -np.inf, np.float32)
        if case == "cut_on_p":
            # two equal maxima hold the whole mass: e = (1/2, 1/2), p = 1/2 exactly
            row[[17 + s, 900 + s]] = 0.0
            params.append(rp(t, 0.9, 0.5, 0, 0.25 + 0.0625 * s))
        elif case == "draw_on_r":
            # q = (1, 1), denom 2, u = 1/2: u * denom equals the first running sum
            row[[5 + s, 2000 + s]] = 1.5
            params.append(rp(t, 1.0, 1.0, 2, 0.5))
        elif case == "cut_and_draw":
            # four equal maxima: running sums 1/4, 1/2, 3/4 of the mass; p = 3/4, u = 2/3
            row[[3 + s, 300 + s, 1000 + s, 3000 + s]] = -2.0
            params.append(rp(t, 1.0, 0.75, 0, 2.0 / 3.0))
        else:
            # many near-equal values whose running sum passes p within a few ulp
            rng = np.random.default_rng(100 + s)
            idx = rng.choice(n, 64, replace=False)
            row[idx] = np.float32(0.0) + rng.integers(0, 3, 64).astype(np.float32) * np.float32(2 ** -23)
            params.append(rp(t, 0.8, 0.5, 0, float(np.float32(0.5))))
        rows.append(row)
    rows = np.stack(rows)
    tok, _ = select_rows(env, rows, params)
    for i in range(len(rows)):
        p = params[i]
        assert int(tok[i]) == oracle.sample_token(rows[i], p.temperature, p.top_p, p.top_k, u=p.uniform), (case, i)


@pytest.mark.ties
def test_cut_within_the_totals_rounding(env, oracle):
    # The reference's row total adds the vocab exponentials in index order, and terms under half
    # an ulp of the running total are dropped: two equal maxima first and a tail of exp(-36.05)
    # ~ 2.19e-16 each leave it exactly 2.0, while any tree of partial sums keeps ~5.7e-11 of the
    # tail. At p = 1/2 the first prefix then equals p in the reference (cut 1, token 0 whatever
    # the draw) and lies 2.9e-11 below it with a tree total (cut 2, token 1 for u > 1/2). Such a
    # cut is decided with the reference's own total. Rows through the wave-record path, the
    # long path (top_k > 256) and the slice path (a penalty over more ids than the hash takes),
    # with rows whose cut has a wide margin beside them.
    torch, dev, t, sel = env
    row = np.full(V, np.float32(-36.05), np.float32)
    row[:2] = 0.0
    rng = np.random.default_rng(71)
    hist = rng.integers(2, V, 5000).astype(np.uint32)  # tail ids only: the maxima stay as they are
    # one launch per path: a penalty over more ids than the hash takes sends the whole launch
    # through the slice kernels
    launches = [
        [("records", rp(t, 1.0, 0.5, 0, 0.75), 0),
         ("records k40", rp(t, 1.0, 0.5, 40, 0.999), 0),
         ("records wide margin", rp(t, 1.0, 0.4, 0, 0.75), 0),
         ("long k300", rp(t, 1.0, 0.5, 300, 0.75), 0),
         ("long k300 wide margin", rp(t, 1.0, 0.6, 300, 0.75), 1)],
        [("slice", rp(t, 1.0, 0.5, 0, 0.75, rep=1.5, off=0, n=len(hist)), 0),
         ("slice wide margin", rp(t, 1.0, 0.6, 0, 0.75, rep=1.5, off=0, n=len(hist)), 1)],
    ]
    for cases in launches:
        rows = np.tile(row, (len(cases), 1))
        tok, pen = select_rows(env, rows, [c[1] for c in cases], history=hist)
        for i, (name, p, expect) in enumerate(cases):
            want = oracle.sample_token(pen[i], p.temperature, p.top_p, p.top_k, u=p.uniform)
            assert want == expect, name
            assert int(tok[i]) == want, name


def test_masked_vocabulary(env, oracle):
    # A vocabulary masked to one value (-inf, or a large negative number) with fewer allowed
    # tokens than the shortlist: the shortlist is filled by ties of the masked value. Where both
    # of a masked entry's terms underflow to 0 it can be neither cut nor drawn, and the row is
    # finished from the allowed tokens alone; at T = 50 the masked terms do not underflow and the
    # ties go through the radix select.
    torch, dev, t, sel = env
    rng = np.random.default_rng(21)
    cases = []
    for fill in (-np.inf, -1e4, -1e30):
        for allowed in (1, 10, 300):
            row = np.full(V, np.float32(fill), np.float32)
            idx = rng.choice(V, allowed, replace=False)
            row[idx] = (rng.standard_normal(allowed) * 2).astype(np.float32)
            for T, p, k in ((0.8, 0.9, 0), (0.8, 1.0, 0), (0.8, 0.9, 40), (1.3, 0.95, 256)):
                cases.append((row, rp(t, T, p, k, float(rng.uniform()))))
    row = np.full(V, np.float32(-1e4), np.float32)
    row[rng.choice(V, 10, replace=False)] = 1.0
    cases.append((row, rp(t, 50.0, 1.0, 0, 0.99)))  # masked q = exp(-200): drawable
    for start in range(0, len(cases), 16):
        chunk = cases[start:start + 16]
        tok, _ = select_rows(env, np.stack([c[0] for c in chunk]), [c[1] for c in chunk])
        for i, (row, p) in enumerate(chunk):
            want = oracle.sample_token(row, p.temperature, p.top_p, p.top_k, u=p.uniform)
            assert int(tok[i]) == want, (start + i, p.temperature, p.top_p, p.top_k)


def test_nan_temperature_samples(env, oracle):
    # sampling.cpp:97: only temperature <= 0 is greedy. A NaN temperature samples with NaN
    # weights, and the token is the cut's last survivor; short, long (top_k > 256) and masked
    # rows, through the wave-record path, and a masked row at an infinite temperature
    torch, dev, t, sel = env
    rng = np.random.default_rng(33)
    nan = float("nan")
    rows, params = [], []
    for p, k in ((1.0, 0), (0.9, 40), (0.95, 0), (1.0, 300), (0.9, 1000)):
        rows.append((rng.standard_normal(V) * 3).astype(np.float32))
        params.append(rp(t, nan, p, k, float(rng.uniform())))
    masked = np.full(V, -np.inf, np.float32)
    masked[rng.choice(V, 10, replace=False)] = rng.standard_normal(10).astype(np.float32)
    rows.append(masked)
    params.append(rp(t, nan, 1.0, 0, 0.5))
    # an infinite temperature: the -inf entries' weights are exp(-inf / inf) = NaN
    rows.append(masked)
    params.append(rp(t, float("inf"), 1.0, 0, 0.5))
    tok, _ = select_rows(env, np.stack(rows), params)
    for i, p in enumerate(params):
        want = oracle.sample_token(rows[i], p.temperature, p.top_p, p.top_k, u=p.uniform)
        assert int(tok[i]) == want, (i, p.top_p, p.top_k)
