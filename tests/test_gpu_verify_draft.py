"""GPU parity of speculative verify with draft logits (src/speculator.cpp:14-30, :34-153): the
rejection-sampling branch (fp32 softmaxes of target and draft rows, ratio test, residual draw
from (p - q)+) composed with sample-and-compare and the bonus row.

The device reproduces the reference's sequential fp32 sums exactly, so results are compared
bit-exactly: against the reference build's outputs in tests/golden/sampling_golden.json, and
against the oracle (oracle.c, pinned by tests/test_oracle.py) on random cases. The oracle's
ratio-test margin |u1 - r| is printed for every rejection-branch position: only an expf last-ulp
difference within that margin could flip a decision."""
import os
import sys

import numpy as np
import pytest

from helpers import ROOT, twd

pytestmark = pytest.mark.gpu

V = 262144


@pytest.fixture(scope="module")
def env():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    return torch, torch.device("cuda:0"), t, t.Selector(V, 65)


def run_device(env, rows, draft_rows, drafts, T, p, k, rp, base):
    torch, dev, t, sel = env
    lg = torch.from_numpy(np.ascontiguousarray(np.stack(rows), np.float32)).to(dev)
    drs = [None if d is None else torch.from_numpy(np.ascontiguousarray(d, np.float32)).to(dev)
           for d in draft_rows]
    d = torch.from_numpy(np.asarray(drafts, np.uint32).view(np.int32)).to(dev)
    params = t.RowParams(T, p, k, rp, 0.0, 0.0, 0, 0)
    res = sel.verify_draft(lg, drs, params, base, d)
    torch.cuda.synchronize()
    return t.decode_verify(res)


def same(got, want):
    keys = ("tokens", "num_accepted", "total_drafted", "bonus_token_sampled")
    return all(got[k] == want[k] for k in keys) and (
        not want["bonus_token_sampled"] or got["bonus_token"] == want["bonus_token"])


def golden_case(c):
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    from make_golden import draft_case_drafts, draft_case_rows
    rows = draft_case_rows(c["rows_seed"], c["vocab"], c["nrows"])
    drs = draft_case_drafts(c["rows_seed"], c["vocab"], rows, c["alpha"], c["draft_sd"], c["mask"])
    for r, j in zip(drs, c.get("nan_at", [])):
        r[j] = np.nan
    return rows, drs


def test_verify_draft_golden(env, golden):
    # 46 cases (6 at V=262144) with the reference build's own outputs: accepted positions,
    # residual draws and the NaN-driven fallback to sample_token
    for i, c in enumerate(golden["verify_draft"]):
        rows, drs = golden_case(c)
        got = run_device(env, rows, drs, c["drafts"], c["t"], c["p"], c["k"], c["rp"],
                         int(c["base_seed"]))
        print(f"case {i} V={c['vocab']} -> {got['tokens']} accepted {got['num_accepted']}")
        assert same(got, c["result"]), (i, got, c["result"])


def _random_case(rng, vocab):
    K = int(rng.integers(1, 6))
    rows = [(rng.standard_normal(vocab) * rng.uniform(1.0, 5.0)).astype(np.float32)
            for _ in range(K + int(rng.integers(0, 2)))]
    drs = []
    for i in range(K):
        if rng.random() < 0.15:
            drs.append(None)
            continue
        mix = float(rng.choice([0.3, 0.8, 0.95]))
        base = rows[min(i, len(rows) - 1)]
        drs.append((mix * base + (1 - mix) * rng.standard_normal(vocab) * 3).astype(np.float32))
    drafts = [int(np.argmax(rows[i])) if i < len(rows) and rng.random() < 0.5
              else int(rng.integers(0, vocab)) for i in range(K)]
    T = float(rng.choice([0.5, 0.8, 1.0, 1.3]))
    k = int(rng.choice([0, 40]))
    return rows, drs, drafts, T, (1.0 if k == 0 else 0.9), k, int(rng.integers(0, 2**63))


def test_verify_draft_after_finish_counter_left_stale(env, oracle):
    # a plain host copy writes the residual launch's arrival counter (what a call that stopped
    # part-way would leave, and arbitrary values); the next calls must still finish their
    # accept chain in the right block, with the oracle's outcome
    import ctypes
    torch, dev, t, sel = env
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    rng = np.random.default_rng(404)
    cases = []
    for _ in range(3):  # every position with a draft row, so that each call has the residual launch
        rows, drs, dr, T, p, k, base = _random_case(rng, 5000)
        drs = [d if d is not None else (0.5 * rows[min(i, len(rows) - 1)]).astype(np.float32)
               for i, d in enumerate(drs)]
        cases.append((rows, drs, dr, T, p, k, base))
    wants = [oracle.verify_draft(dr, rows, drs, T, p, k, 1.0, base)
             for rows, drs, dr, T, p, k, base in cases]
    for w in wants:
        w.pop("diag")
    for (rows, drs, dr, T, p, k, base), w in zip(cases, wants):  # arms the counter
        assert same(run_device(env, rows, drs, dr, T, p, k, 1.0, base), w)
    state = t.twd.lib.twd_selector_verify_state(sel.handle)
    assert state
    cur = ctypes.c_uint64()
    assert hip.hipMemcpy(ctypes.byref(cur), state, 8, 2) == 0
    nxt = cur.value & 0xFFFFFFFF
    assert cur.value >> 32 == 0 and nxt > 0  # armed for the next call's epoch
    # a call of the previous epoch that stopped after two blocks, another epoch's count, all ones,
    # and zero
    for garbage in ((2 << 32) | (nxt - 1), (5 << 32) | (nxt + 77), 0xFFFFFFFFFFFFFFFF, 0):
        torch.cuda.synchronize()
        g = ctypes.c_uint64(garbage)
        assert hip.hipMemcpy(state, ctypes.byref(g), 8, 1) == 0
        for (rows, drs, dr, T, p, k, base), w in zip(cases, wants):  # that call and the next ones
            got = run_device(env, rows, drs, dr, T, p, k, 1.0, base)
            assert same(got, w), (hex(garbage), got, w)
    assert hip.hipMemcpy(ctypes.byref(cur), state, 8, 2) == 0
    assert cur.value >> 32 == 0 and cur.value & 0xFFFFFFFF != 0  # armed again


# 1000: the serial head alone (no segment); 2049: one one-term segment; 3000 and 50000: a last
# segment and a last exp block cut short; V: the config-4 rows
@pytest.mark.parametrize("vocab", [1000, 2049, 3000, 50000, V])
def test_verify_draft_random_vs_oracle(env, oracle, vocab):
    rng = np.random.default_rng(vocab)
    n_rej = n_sums = 0
    for case in range(12 if vocab == V else 30):
        rows, drs, drafts, T, p, k, base = _random_case(rng, vocab)
        want = oracle.verify_draft(drafts, rows, drs, T, p, k, 1.0, base)
        want_diag = want.pop("diag")
        for i, d in enumerate(want_diag):
            if d is not None:
                print(f"case {case} pos {i}: r={d['r']:.7g} u1={d['u1']:.7g} "
                      f"margin={abs(d['u1'] - d['r']):.3g} accepted={d['accepted']}")
                n_rej += 0 if d["accepted"] else 1
        got = run_device(env, rows, drs, drafts, T, p, k, 1.0, base)
        assert same(got, want), (case, got, want)
        # the compute_softmax sums, bit for bit, at every position that ran the ratio test
        sums = env[3].draft_sums()
        for i, d in enumerate(want_diag):
            if d is not None:
                sp, sq = sums[i]
                assert np.float32(sp) == np.float32(d["sum_p"]) and np.float32(sq) == np.float32(d["sum_q"]), \
                    (case, i, sp, d["sum_p"], sq, d["sum_q"])
                n_sums += 1
    assert n_rej > 0 and n_sums > 0


def test_verify_draft_edges(env, oracle):
    rng = np.random.default_rng(3)
    vocab = 5000
    t_rows = [(rng.standard_normal(vocab) * 3).astype(np.float32) for _ in range(4)]
    d_rows = [(rng.standard_normal(vocab) * 3).astype(np.float32) for _ in range(3)]
    cases = []
    # a draft id past the vocabulary: q_val = 0, so r = 1 and the position is accepted
    cases.append((t_rows, d_rows, [vocab + 7, 1, 2], 0.8, 1.0))
    # NaN in a target row: its softmax sum is NaN, p stays unnormalised
    tr = [r.copy() for r in t_rows]
    tr[0][17] = np.nan
    cases.append((tr, d_rows, [int(np.argmax(t_rows[0])), 3, 4], 0.8, 1.0))
    # a draft row of -inf except one entry: q is one-hot
    dr = [r.copy() for r in d_rows]
    dr[1][:] = -np.inf
    dr[1][123] = 0.0
    cases.append((t_rows, dr, [int(np.argmax(t_rows[0])), 123, 9], 1.0, 1.0))
    # temperature 0 with a penalty: not greedy, compute_softmax runs at T = 1
    cases.append((t_rows, d_rows, [5, 6, 7], 0.0, 1.1))
    # greedy params: the draft rows are ignored
    cases.append((t_rows, d_rows, [int(np.argmax(t_rows[0])), 6, 7], 0.0, 1.0))
    # fewer target rows than drafts: k = rows, no bonus row
    cases.append((t_rows[:2], d_rows, [11, 12, 13], 0.9, 1.0))
    for i, (tr, dr, drafts, T, rp) in enumerate(cases):
        base = 1000 + i
        want = oracle.verify_draft(drafts, tr, dr, T, 1.0, 0, rp, base)
        want.pop("diag")
        got = run_device(env, tr, dr, drafts, T, 1.0, 0, rp, base)
        assert same(got, want), (i, got, want)


def test_python_coordinator_with_draft_logits(env, oracle):
    torch, dev, t, sel = env
    rng = np.random.default_rng(8)
    vocab = 2048
    rows = [(rng.standard_normal(vocab) * 2).astype(np.float32) for _ in range(4)]
    drs = [(0.5 * rows[i] + rng.standard_normal(vocab)).astype(np.float32) for i in range(3)]
    drafts = [int(np.argmax(rows[i])) for i in range(3)]
    sc = t.SpeculativeCoordinator()
    sp = t.SamplingParams(0.9, 1.0, 0, 1.0)
    lg = torch.from_numpy(np.stack(rows)).to(dev)
    got = sc.evaluate_verification(drafts, lg, vocab, sp, 77,
                                   [torch.from_numpy(d).to(dev) for d in drs])
    want = oracle.verify_draft(drafts, rows, drs, 0.9, 1.0, 0, 1.0, 77)
    want.pop("diag")
    assert same(got, want), (got, want)


# ---- the exact sequential-sum engine on its own --------------------------------------------

def _seq_sum(env, x, thr=None):
    import ctypes
    torch, dev, t, sel = env
    n = len(x)
    buf = torch.zeros((n + 15) // 16 * 16, dtype=torch.float32, device=dev)
    buf[:n] = torch.from_numpy(np.ascontiguousarray(x, np.float32))
    out = torch.zeros(1, dtype=torch.float32, device=dev)
    stop = torch.full((1,), -1, dtype=torch.int32, device=dev)
    rc = t.lib.twd_sequential_sum(ctypes.c_void_p(buf.data_ptr()), ctypes.c_uint32(n),
                                  ctypes.c_float(0.0 if thr is None else thr),
                                  ctypes.c_void_p(out.data_ptr()),
                                  None if thr is None else ctypes.c_void_p(stop.data_ptr()), None)
    assert rc == 0, t.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()[0], int(stop.cpu().numpy()[0])


def _seq_cases():
    rng = np.random.default_rng(41)
    cases = []
    for n in (1, 5, 2048, 2049, 4097, 70001, V):  # around the serial start and the window sizes
        for sd in (1.0, 4.0):
            z = (rng.standard_normal(n) * sd).astype(np.float32)
            cases.append((f"softmax n={n} sd={sd}", np.exp(z - z.max()).astype(np.float32)))
    cases.append(("uniform", rng.random(100000).astype(np.float32)))
    # S in [0.5, 1) after the first term, terms k * 2^-25: every odd k is an exact half-way case
    ties = (rng.integers(0, 8, 50000) * 2.0 ** -25).astype(np.float32)
    ties[0] = 0.75
    cases.append(("ties", ties))
    # crossing into [1, 2) and beyond, with ties on both sides
    cross = (rng.integers(0, 64, 60000) * 2.0 ** -24).astype(np.float32)
    cross[0] = 0.999
    cases.append(("ties across binades", cross))
    # half the terms zero, and terms below half an ulp that never move the sum
    z = rng.random(30000).astype(np.float32)
    z[rng.random(30000) < 0.5] = 0.0
    cases.append(("zeros", z))
    tiny = np.full(20000, 1e-9, np.float32)
    tiny[0] = 1.0
    cases.append(("below half an ulp", tiny))
    # past the serial head the sum runs in 1024-term segments: lengths at segment edges, a sum
    # that doubles inside many segments, one whose binade changes exactly at segment starts
    # (each segment adds 2^k after a sum of 2^k), and long zero stretches between big terms
    for n in (3071, 3072, 3073, 2048 + 1024 * 7, 2048 + 1024 * 7 + 1):
        cases.append((f"segment edge n={n}", rng.random(n).astype(np.float32)))
    cases.append(("growing terms", (np.arange(200000) * 1e-3).astype(np.float32)))
    edge = np.zeros(2048 + 1024 * 12, np.float32)
    edge[0] = 1.0
    edge[1:2048] = 0.0
    for k in range(12):  # segment k adds the running sum again: the sum doubles per segment
        edge[2048 + 1024 * k] = np.float32(2.0 ** k)
    cases.append(("binade change at segment starts", edge))
    sparse = np.zeros(150000, np.float32)
    sparse[rng.integers(0, 150000, 40)] = rng.random(40).astype(np.float32) * 100
    cases.append(("sparse big terms", sparse))
    return cases


def test_sequential_sum_is_the_in_order_fp32_sum(env):
    # np.add.accumulate over float32 adds in index order, rounding each step to fp32: the loop
    # of speculator.cpp:22-26 and :104-116
    for name, x in _seq_cases():
        acc = np.add.accumulate(x, dtype=np.float32)
        got, _ = _seq_sum(env, x)
        assert np.float32(got).view(np.uint32) == acc[-1].view(np.uint32), (name, got, acc[-1])
        for frac in (0.0, 0.37, 0.999, 1.0):
            thr = np.float32(acc[-1] * np.float32(frac))
            want = int(np.argmax(acc >= thr)) if (acc >= thr).any() else len(x)
            s, stop = _seq_sum(env, x, float(thr))
            assert stop == want, (name, frac, stop, want)
            # the sum returned with a stop is the prefix through the stop index
            assert np.float32(s).view(np.uint32) == acc[min(want, len(x) - 1)].view(np.uint32), (name, frac)


def test_device_expf_matches_host(env, oracle):
    # the device build of the verify's expf against the host C library's expf (the
    # reference's std::exp(float)): every 16th float of [-104, 0], then random arguments
    torch, dev, t, _ = env
    top = int(np.float32(104.0).view(np.uint32))
    neg = (np.arange(0, top + 1, 16, dtype=np.uint64).astype(np.uint32) | np.uint32(0x80000000)).view(np.float32)
    rng = np.random.default_rng(5)
    more = rng.uniform(-120, 95, 1 << 20).astype(np.float32)
    special = np.array([np.inf, -np.inf, np.nan, 88.72, -103.97, 0.0, -0.0], np.float32)
    for x in (neg, more, special):
        got = t.probe_expf(torch.from_numpy(x).to(dev)).cpu().numpy()
        want = oracle.expf(x)
        both_nan = np.isnan(got) & np.isnan(want)
        bad = (got.view(np.uint32) != want.view(np.uint32)) & ~both_nan
        assert not bad.any(), (int(bad.sum()), x[bad][:5], got[bad][:5], want[bad][:5])


@pytest.mark.parametrize("k", [40, 600])
def test_verify_draft_bonus_and_fallback_tokens(env, oracle, k):
    # the target rows' sampled tokens (rows without draft logits, the bonus row, the fallback)
    # come from the selection run inside the draft chain's launches (k = 40) or from the
    # selector's own launches on the side stream (k = 600, a shortlist longer than 256); both
    # against the oracle, with every draft accepted so that the bonus row is drawn
    rng = np.random.default_rng(1000 + k)
    for case in range(6):
        K = 4
        rows = [(rng.standard_normal(V) * rng.uniform(1.0, 4.0)).astype(np.float32) for _ in range(K + 1)]
        drs = [rows[i].copy() if i != 2 or case % 2 else None for i in range(K)]  # p == q: r = 1
        want_tok = [oracle.sample_token(rows[i], 0.9, 0.95, k, seed=oracle.splitmix64(77 + i)) for i in range(K + 1)]
        drafts = [want_tok[i] for i in range(K)]
        got = run_device(env, rows, drs, drafts, 0.9, 0.95, k, 1.0, 77)
        want = oracle.verify_draft(drafts, rows, drs, 0.9, 0.95, k, 1.0, 77)
        want.pop("diag")
        assert same(got, want), (case, got, want)
        assert got["num_accepted"] == K and got["bonus_token"] == want_tok[K], (case, got)
