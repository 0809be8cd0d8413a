"""head.sample with 17..64 rows (BASELINE config 5's path): the 32x32 MFMA head writes the
logits, then the selector's passes run over them -- the hashed penalty (histories up to 4,096 ids
per row) or the slice kernels' penalty (longer ones), the per-64-entry selection records and the
one-block-per-row merge, with the long path for top_k > 256.

Each case checks, per row, the penalised logits and the token bit for bit against the oracle's
apply_repetition_penalty + sample_token (sampling.cpp:74-169) on the GPU's own raw logits, and
against twd_select over a copy of the same raw logits (the entry point for caller-owned logits):
same logits, same tokens. The cases: config 5's shape at both m-tile counts with greedy and
unpenalised rows mixed in, history ids on head-block edges and past the vocabulary, one id
60,000 times in one row, top_k > 256 and a NaN row, small and odd vocabularies, empty
histories, and histories past the hashed penalty's 4,096 ids."""
import numpy as np
import pytest

from helpers import hidden_bf16, twd, wsb_bytes

pytestmark = pytest.mark.gpu

D = 5376
CAP = 30.0
V_FULL = 262144
SEED_FULL = 20260801


@pytest.fixture(scope="module")
def env():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch, torch.device("cuda:0"), twd()


@pytest.fixture(scope="module")
def full_head(env):
    torch, dev, t = env
    wsb = torch.empty(t.head_bytes(V_FULL, D), dtype=torch.uint8, device=dev)
    t.generate_head(wsb, V_FULL, D, SEED_FULL)
    head = t.LMHead(wsb, V_FULL, D, CAP)
    yield head
    head.close()


def dev_i32(torch, dev, a):
    a = np.ascontiguousarray(a, np.uint32)
    if a.size == 0:
        a = np.zeros(1, np.uint32)
    return torch.from_numpy(a.view(np.int32)).to(dev)


def check(env, oracle, head, hb, params, hist, tag, oracle_rows=None):
    """head.sample against twd_select on the same raw logits and against the oracle."""
    torch, dev, t = env
    h = torch.from_numpy(np.ascontiguousarray(hb).view(np.int16)).to(dev)
    M = len(params)
    print(f"[{tag}] M={M} V={head.vocab}", flush=True)
    raw_dev = head.logits(h)
    raw = raw_dev.cpu().numpy()
    hist_dev = dev_i32(torch, dev, hist)
    tok, lg = head.sample(h, params, history=hist_dev)
    tok = tok.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    lg = lg.cpu().numpy()
    # the selector over a copy of the same raw logits
    sel = t.Selector(head.vocab, M)
    lg_u = raw_dev.clone()
    tok_u = sel.select(lg_u, params, history=hist_dev).cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    lg_u = lg_u.cpu().numpy()
    sel.close()
    assert np.array_equal(lg.view(np.uint32), lg_u.view(np.uint32)), f"{tag}: penalised logits differ"
    assert np.array_equal(tok, tok_u), f"{tag}: head.sample {tok} != select {tok_u}"
    rows = range(M) if oracle_rows is None else oracle_rows
    for m in rows:
        p = params[m]
        hm = hist[p.history_offset: p.history_offset + p.history_len]
        pen = oracle.apply_repetition_penalty(raw[m], hm, p.repetition_penalty, p.softcap) \
            if p.repetition_penalty != 1.0 else raw[m]
        assert np.array_equal(lg[m].view(np.uint32), pen.view(np.uint32)), f"{tag} row {m}: penalty"
        try:
            want = oracle.sample_token(pen, p.temperature, p.top_p, p.top_k, u=p.uniform)
        except RuntimeError:
            assert tok[m] == t.TOKEN_DEGENERATE, f"{tag} row {m}: expected degenerate"
            continue
        assert tok[m] == want, f"{tag} row {m}: GPU {tok[m]} != oracle {want}"
    return tok


def random_rows(t, rng, M, V, hist_len, greedy_every=0, plain_every=0, k_hi=101):
    hists, params, off = [], [], 0
    for m in range(M):
        n = int(hist_len(m)) if callable(hist_len) else hist_len
        hists.append(rng.integers(0, V, n).astype(np.uint32))
        T = 0.0 if greedy_every and m % greedy_every == 3 else float(rng.uniform(0.5, 1.2))
        rp = 1.0 if plain_every and m % plain_every == 1 else 1.1
        params.append(t.RowParams(T, float(rng.uniform(0.8, 0.98)), int(rng.integers(20, k_hi)), rp,
                                  t.uniform_from_seed(t.splitmix64(1000 * M + m)), CAP, off, n))
        off += n
    return params, np.concatenate(hists)


@pytest.mark.parametrize("M", [17, 32, 33, 64])
def test_wide_sample_full_geometry(env, oracle, full_head, M):
    # config 5's shape (2048-id histories, rp 1.1, per-row T/k/p) at both m-tile counts, with
    # greedy rows and rows without a penalty mixed in; the oracle on every row
    torch, dev, t = env
    rng = np.random.default_rng(900 + M)
    params, hist = random_rows(t, rng, M, V_FULL, 2048, greedy_every=9, plain_every=7)
    # ids on head-block edges (256 rows each), a run of duplicates, ids past the vocabulary
    hist[:10] = [255, 256, 511, 512, V_FULL - 256, V_FULL - 1, V_FULL, 2**32 - 1, 255, 0]
    hist[2048 + 100: 2048 + 400] = hist[2048 + 50]
    check(env, oracle, full_head, hidden_bf16(910 + M, M, D), params, hist, f"full M={M}")


def test_wide_sample_heavy_duplicates(env, oracle, full_head):
    # one id 60,000 times in one row (the penalty compounds 60,000 times), a row whose history
    # falls in 256 consecutive vocabulary rows, and penalties below and above 1
    torch, dev, t = env
    M = 20
    rng = np.random.default_rng(931)
    lens = [60000, 4000] + [500] * (M - 2)
    params, hist = random_rows(t, rng, M, V_FULL, lambda m: lens[m])
    hist[:60000] = 123457
    hist[60000:64000] = 256 * 77 + rng.integers(0, 256, 4000)
    params[2] = t.RowParams(0.8, 0.9, 50, 0.7, 0.31, CAP, params[2].history_offset, 500)
    params[3] = t.RowParams(0.0, 1.0, 0, 1.6, 0.0, CAP, params[3].history_offset, 500)
    check(env, oracle, full_head, hidden_bf16(932, M, D), params, hist, "duplicates")


def test_wide_sample_long_shortlists_and_nan(env, oracle, full_head):
    # rows with top_k > 256 (the long path after the records) and a NaN row (degenerate)
    torch, dev, t = env
    M = 24
    rng = np.random.default_rng(941)
    params, hist = random_rows(t, rng, M, V_FULL, 1000)
    for m, k in ((1, 300), (5, 1000), (9, 262144)):
        p = params[m]
        params[m] = t.RowParams(p.temperature, 0.95, k, 1.1, p.uniform, CAP, p.history_offset, p.history_len)
    hb = hidden_bf16(942, M, D)
    hb[7, 11] = 0x7FC0
    tok = check(env, oracle, full_head, hb, params, hist, "long + nan")
    assert tok[7] == t.TOKEN_DEGENERATE


@pytest.mark.parametrize("V", [1000, 4099, 70000])
def test_wide_sample_small_vocabularies(env, oracle, V):
    # few head blocks and a partial last tile pair (V % 32 != 0; 4099 % 4 != 0: unaligned rows)
    torch, dev, t = env
    d = 384
    W, S, B = oracle.gen_lm_head(950 + V % 97, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    rng = np.random.default_rng(V)
    M = 40
    params, hist = random_rows(t, rng, M, V + 20, lambda m: rng.integers(0, 600), greedy_every=6,
                               plain_every=5)
    check(env, oracle, head, hidden_bf16(951, M, d), params, hist, f"V={V}")
    head.close()


def test_wide_sample_no_penalty_and_empty_histories(env, oracle, full_head):
    # no penalised row with ids at all: rp 1 rows, and penalised rows with empty histories
    torch, dev, t = env
    M = 18
    rng = np.random.default_rng(961)
    params = [t.RowParams(float(rng.uniform(0.5, 1.2)), 0.9, 40, 1.0 if m % 2 else 1.3,
                          float(rng.uniform()), CAP, 0, 0) for m in range(M)]
    check(env, oracle, full_head, hidden_bf16(962, M, D), params, np.zeros(0, np.uint32), "no penalty")


def test_wide_long_histories(env, oracle):
    # penalised histories past the hashed penalty's 4,096 ids per row (the slice kernels apply
    # the penalty): one row of 70,000 ids, then 17 rows of 16,000
    torch, dev, t = env
    V, d = 5000, 256
    W, S, B = oracle.gen_lm_head(971, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    rng = np.random.default_rng(972)
    M = 17
    params, hist = random_rows(t, rng, M, V, lambda m: 70000 if m == 0 else 1000)
    check(env, oracle, head, hidden_bf16(973, M, d), params, hist, "long row", oracle_rows=[0, 1, 16])
    params, hist = random_rows(t, rng, M, V, 16000)  # 272,000 ids > 262,144
    check(env, oracle, head, hidden_bf16(974, M, d), params, hist, "many ids", oracle_rows=[0, 8, 16])
    head.close()
