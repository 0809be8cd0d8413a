"""GPU parity of sample_token with shortlists longer than 256 entries (top_k > 256).

The reference takes any top_k: want = min(top_k, V) entries by nth_element + sort, the top-p
running sum over all of them, cut = min(cut, top_k), then the temperature draw over the cut
(src/sampling.cpp:120-168). Nothing on its path calls validate_sampling, so the CLI, the server
and g4dense_engine_generate_ex pass such values through (src/main.cpp:125-126,
src/c_api.cpp:137). Checked here at V = 262144:
  * twd_select for top_k in {257, 1000, 4096, 262144, 300000}, with top-p on and off, on
    N(0, 4^2) rows, softcapped rows and rows of heavy exact ties (the sort's index order);
  * penalised rows on both penalty paths (hashed histories, and histories past 4,096 ids);
  * long rows mixed with short, greedy and degenerate rows in one call;
  * twd_verify with such parameters;
  * the fused head sample pass (M <= 4) and the generator with G4DenseGenerationOptions
    (top_k = 500) on a V = 262144 head;
  * twd_select_noalloc's refusal (its fixed scratch holds no sort buffers).
Ids are compared bit for bit with the oracle on the same logits and, where the reference build
is present, with the reference's own sample_token.
"""
import numpy as np
import pytest

from helpers import hidden_bf16, twd, wsb_bytes

pytestmark = pytest.mark.gpu

V = 262144
CAP = 30.0
KS = [257, 1000, 4096, 262144, 300000]


@pytest.fixture(scope="module")
def env():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    sel = t.Selector(V, 65)
    yield torch, torch.device("cuda:0"), t, sel
    sel.close()


def ref_or_none():
    import oracle as O
    return O.Reference() if O.Reference.available() else None


def rows_of(kind, seed, n=V):
    import oracle as O
    rng = np.random.default_rng(seed)
    z = (rng.standard_normal(n) * 4.0).astype(np.float32)
    if kind == "softcap":
        return O.softcap((z * 3.0).astype(np.float32), CAP)
    if kind == "ties":  # about 200 distinct values: long runs of exact ties inside the shortlist
        return (np.round(z * 4.0) / 4.0).astype(np.float32)
    return z


def select(env, rows, params, history=None):
    torch, dev, t, sel = env
    lg = torch.from_numpy(np.ascontiguousarray(rows, np.float32)).to(dev)
    hist = None if history is None else torch.from_numpy(
        np.ascontiguousarray(history, np.uint32).view(np.int32)).to(dev)
    tok = sel.select(lg, params, hist)
    return (tok.cpu().numpy().astype(np.int64) & 0xFFFFFFFF), lg.cpu().numpy()


@pytest.mark.parametrize("k", KS)
@pytest.mark.parametrize("p", [0.9, 1.0])
def test_long_topk_vs_oracle_and_reference(env, oracle, k, p):
    torch, dev, t, sel = env
    ref = ref_or_none()
    kinds = ["normal", "softcap", "ties"]
    rows = np.stack([rows_of(kind, 1000 * k + i + int(p * 10)) for i, kind in enumerate(kinds)])
    seeds = [int(np.random.default_rng(k + i).integers(0, 2**63)) for i in range(len(kinds))]
    Ts = [0.8, 1.3, 0.6]
    params = [t.RowParams(Ts[i], p, k, 1.0, t.uniform_from_seed(s), 0.0, 0, 0) for i, s in enumerate(seeds)]
    tok, _ = select(env, rows, params)
    for i in range(len(kinds)):
        want, dg = oracle.sample_token(rows[i], Ts[i], p, k, u=params[i].uniform, diag=True)
        assert int(tok[i]) == want, (kinds[i], k, p, int(tok[i]), want, dg["cut"], dg["want"])
        if ref is not None:
            assert ref.sample_token(rows[i], Ts[i], p, k, seeds[i]) == want, (kinds[i], k, p)


def test_long_topk_many_draws_one_row(env, oracle):
    # one row, 40 draws (uniforms spread over [0, 1)) at k = 4096, p = 1: the draw position
    # walks the whole sorted shortlist
    torch, dev, t, sel = env
    row = rows_of("normal", 77)
    us = [(i + 0.5) / 40 for i in range(40)]
    params = [t.RowParams(2.0, 1.0, 4096, 1.0, u, 0.0, 0, 0) for u in us]
    tok, _ = select(env, np.tile(row, (40, 1)), params)
    want = [oracle.sample_token(row, 2.0, 1.0, 4096, u=u) for u in us]
    assert [int(x) for x in tok] == want
    assert len(set(want)) > 30  # the draws land at different shortlist positions


@pytest.mark.parametrize("hlen", [3000, 5000])
def test_long_topk_penalised(env, oracle, hlen):
    # 3000 ids: the hashed penalty pass; 5000 ids: the slice kernels' penalty (more than 4096)
    torch, dev, t, sel = env
    rng = np.random.default_rng(hlen)
    rows = np.stack([rows_of("softcap", hlen + i) for i in range(2)])
    hist = rng.integers(0, V + 5, size=2 * hlen, dtype=np.uint32)  # ids past V are skipped
    hist[:50] = hist[0]  # duplicates compound
    params = [t.RowParams(0.7, 0.95, 1000, 1.1, 0.3, CAP, 0, hlen),
              t.RowParams(1.1, 1.0, 20000, 0.8, 0.9, CAP, hlen, hlen)]
    tok, pen = select(env, rows, params, hist)
    for i, prm in enumerate(params):
        h = hist[prm.history_offset:prm.history_offset + prm.history_len]
        want_pen = oracle.apply_repetition_penalty(rows[i], h, prm.repetition_penalty, CAP)
        assert np.array_equal(pen[i].view(np.uint32), want_pen.view(np.uint32))
        want = oracle.sample_token(want_pen, prm.temperature, prm.top_p, prm.top_k, u=prm.uniform)
        assert int(tok[i]) == want, (hlen, i)


def test_long_rows_mixed_with_short_ones(env, oracle):
    torch, dev, t, sel = env
    base = rows_of("normal", 5)
    nan_row = base.copy()
    nan_row[1234] = np.nan
    rows = np.stack([base, base, base, base, nan_row, rows_of("ties", 6), base])
    params = [t.RowParams(0.7, 0.9, 40, 1.0, 0.25, 0.0, 0, 0),       # short
              t.RowParams(0.7, 0.9, 1000, 1.0, 0.25, 0.0, 0, 0),     # long
              t.RowParams(0.0, 1.0, 0, 1.0, 0.0, 0.0, 0, 0),         # greedy
              t.RowParams(0.9, 1.0, 300000, 1.0, 0.999, 0.0, 0, 0),  # long, the whole row
              t.RowParams(0.9, 0.9, 5000, 1.0, 0.5, 0.0, 0, 0),      # long, degenerate (NaN)
              t.RowParams(1.0, 0.97, 257, 1.0, 0.61, 0.0, 0, 0),     # long, ties
              t.RowParams(1.0, 1.0, 0, 1.0, 0.61, 0.0, 0, 0)]        # short: top 256 at k = 0
    tok, _ = select(env, rows, params)
    for i, prm in enumerate(params):
        if i == 4:
            assert int(tok[i]) == t.TOKEN_DEGENERATE
            continue
        want = oracle.sample_token(rows[i], prm.temperature, prm.top_p, prm.top_k, u=prm.uniform)
        assert int(tok[i]) == want, i


def test_long_topk_verify(env, oracle):
    # evaluate_verification without draft logits (speculator.cpp:123-134) at k = 2000: each row
    # is sample_token'd with splitmix64(base + i) and compared with the draft
    torch, dev, t, sel = env
    rows = np.stack([rows_of("normal", 300 + i) for i in range(4)])
    base = 4242
    want_rows = [oracle.sample_token(rows[i], 0.9, 0.95, 2000, seed=oracle.splitmix64(base + i))
                 for i in range(4)]
    drafts = [want_rows[0], want_rows[1], (want_rows[2] + 1) % V]
    lg = torch.from_numpy(rows).to(dev)
    prm = t.RowParams(0.9, 0.95, 2000, 1.0, 0.0, 0.0, 0, 0)
    res = t.decode_verify(sel.verify(lg, prm, base, torch.tensor(drafts, dtype=torch.int32, device=dev)))
    want = oracle.verify(drafts, list(rows), 0.9, 0.95, 2000, base)
    assert res["tokens"] == want["tokens"] and res["num_accepted"] == want["num_accepted"] == 2


@pytest.fixture(scope="module")
def wide_head(oracle):
    # a V = 262144 head of depth 128: the full vocabulary at a small size
    import torch
    t = twd()
    dev = torch.device("cuda:0")
    d = 128
    W, S, B = oracle.gen_lm_head(4100, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    yield torch, dev, t, head, d
    head.close()


def test_long_topk_fused_head_sample(wide_head, oracle):
    # twd_head_sample with M <= 4 (the fused sample pass: penalty and records in the head's
    # epilogue), long rows among its rows
    torch, dev, t, head, d = wide_head
    hs = hidden_bf16(71, 4, d)
    h = torch.from_numpy(hs.view(np.int16)).to(dev)
    raw = head.logits(h).cpu().numpy()
    rng = np.random.default_rng(72)
    hist = rng.integers(0, V, size=4 * 600, dtype=np.uint32)
    params = [t.RowParams(0.8, 0.95, 500, 1.1, 0.4, CAP, 0, 600),
              t.RowParams(0.7, 0.9, 40, 1.1, 0.7, CAP, 600, 600),
              t.RowParams(1.2, 1.0, 262144, 1.0, 0.05, CAP, 0, 0),
              t.RowParams(0.9, 0.99, 3000, 1.3, 0.95, CAP, 1800, 600)]
    tok, pen = head.sample(h, params, history=torch.from_numpy(hist.view(np.int32)).to(dev))
    tok = tok.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    pen = pen.cpu().numpy()
    for m, prm in enumerate(params):
        hh = hist[prm.history_offset:prm.history_offset + prm.history_len]
        want_pen = oracle.apply_repetition_penalty(raw[m], hh, prm.repetition_penalty, CAP) \
            if prm.repetition_penalty != 1.0 else raw[m]
        assert np.array_equal(pen[m].view(np.uint32), want_pen.view(np.uint32)), m
        want = oracle.sample_token(want_pen, prm.temperature, prm.top_p, prm.top_k, u=prm.uniform)
        assert int(tok[m]) == want, m


def test_generator_ex_top_k_500(wide_head, oracle):
    # g4dense_engine_generate_ex passes top_k unchecked (c_api.cpp:137): a generation with
    # top_k = 500, seeded, with the repetition penalty, against the reference's decode loop on the
    # GPU's own logits (runner.cpp:2314-2336)
    torch, dev, t, head, d = wide_head
    rng = np.random.default_rng(9)
    prompt = [int(x) for x in rng.integers(0, V, 40)]
    hs = hidden_bf16(91, 6, d)
    o = t.twd.options_default()
    o.max_tokens, o.temperature, o.top_p, o.top_k = 6, 0.9, 0.97, 500
    o.repetition_penalty, o.has_seed, o.seed = 1.15, 1, 2024
    history = list(prompt)
    want = []
    for i in range(6):
        raw = head.logits(torch.from_numpy(hs[i:i + 1].view(np.int16)).to(dev)).cpu().numpy()[0]
        lg = oracle.apply_repetition_penalty(raw, history, 1.15, CAP)
        tok = oracle.sample_token(lg, 0.9, 0.97, 500, seed=oracle.seed_for(True, 2024, len(history) - 1))
        history.append(tok)
        want.append(tok)
    gen = t.Generator.from_options(head, o, prompt)
    got = [gen.step(torch.from_numpy(hs[i:i + 1].view(np.int16)).to(dev)) for i in range(6)]
    assert [g[0] for g in got] == want
    assert gen.stop_reason() == t.twd.STOP_MAX_TOKENS
    gen.close()


def test_noalloc_refuses_long_shortlists(env):
    torch, dev, t, sel = env
    import ctypes
    row = torch.from_numpy(rows_of("normal", 3)[None]).to(dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    prm = (t.RowParams * 1)(t.RowParams(0.8, 1.0, 1000, 1.0, 0.5, 0.0, 0, 0))
    rc = t.twd.lib.twd_select_noalloc(ctypes.c_void_p(row.data_ptr()), V, 1, V, prm, None,
                                      ctypes.c_void_p(tok.data_ptr()), None)
    assert rc == t.twd.TWD_E_INVALID and "top_k > 256" in t.twd.last_error()
