"""The fused sample pass of the LM head (rows <= 8): softcap and repetition penalty in the head's
epilogue, per-wave selection statistics, then one merge launch that reads only the blocks able
to hold a top-`want` entry; and head.sample past 8 rows (logits pass, then the selection over the
logits in memory). Every token is compared bit-exactly with the oracle's
apply_repetition_penalty + sample_token (sampling.cpp:74-169) on the GPU's own raw logits, and
the penalised rows bit for bit. The cases reach every branch of the merge: survivors ranked by
counting (few), by the binned top-`want` (up to 2048), by a radix select over the candidate blocks
in memory (heavy ties), every block a candidate (small vocabularies), and degenerate rows."""
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
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(dev)


def run_and_check(env, oracle, head, hb, params, hist, tag):
    """head.sample on bf16 rows hb against the oracle on head.logits of the same rows."""
    torch, dev, t = env
    h = torch.from_numpy(np.ascontiguousarray(hb).view(np.int16)).to(dev)
    raw = head.logits(h).cpu().numpy()
    hist_dev = dev_i32(torch, dev, hist if len(hist) else np.zeros(1, np.uint32))
    tok, lg = head.sample(h, params, history=hist_dev)
    tok = tok.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    lg = lg.cpu().numpy()
    for m, p in enumerate(params):
        hm = hist[p.history_offset: p.history_offset + p.history_len]
        pen = oracle.apply_repetition_penalty(raw[m], hm, p.repetition_penalty, p.softcap) \
            if p.repetition_penalty != 1.0 else raw[m]
        assert np.array_equal(lg[m].view(np.uint32), pen.view(np.uint32)), f"{tag} row {m}: penalty"
        try:
            want, dg = oracle.sample_token(pen, p.temperature, p.top_p, p.top_k, u=p.uniform, diag=True)
        except RuntimeError:
            assert tok[m] == t.TOKEN_DEGENERATE, f"{tag} row {m}: expected degenerate"
            continue
        print(f"{tag} row {m}: token {want} cut {dg['cut']}/{dg['want']} "
              f"margins {dg['cut_margin']:.3e} {dg['draw_margin']:.3e}")
        assert tok[m] == want, (f"{tag} row {m}: GPU {tok[m]} != oracle {want}; margins "
                                f"{dg['cut_margin']:.3e} {dg['draw_margin']:.3e}")
    return tok


PARAM_SETS = [  # (T, p, k, rp): top-256 shortlists, tiny and full k, greedy with a penalty
    [(0.7, 0.9, 40, 1.1)],
    [(1.0, 1.0, 0, 1.0), (0.0, 1.0, 0, 1.3)],
    [(0.8, 0.95, 256, 1.2), (1.5, 0.5, 1, 1.0), (0.3, 0.99, 7, 0.8)],
    [(0.9, 0.97, 100, 1.1), (2.0, 1.0, 0, 1.05), (0.0, 1.0, 0, 1.0), (0.6, 0.8, 64, 1.4)],
    # 5..8 rows: rows two apart in the MFMA's rows, two per lane in the epilogue
    [(0.7, 0.9, 40, 1.1), (0.0, 1.0, 0, 1.2), (1.2, 0.95, 100, 0.9), (0.5, 0.8, 20, 1.0),
     (0.9, 0.97, 256, 1.1)],
    [(0.7, 0.9, 40, 1.1)] * 6,
    [(0.8, 0.9, 300, 1.1), (1.0, 1.0, 0, 1.0), (0.6, 0.85, 50, 1.3), (0.0, 1.0, 0, 1.0),
     (1.1, 0.99, 3, 1.05), (0.7, 0.5, 1000, 1.1), (0.4, 0.9, 64, 0.8)],
    [(0.5 + 0.1 * m, 0.8 + 0.02 * m, 20 + 10 * m, 1.1) for m in range(8)],
]


@pytest.mark.parametrize("ps", range(len(PARAM_SETS)))
def test_fused_full_geometry(env, oracle, full_head, ps):
    torch, dev, t = env
    prm = PARAM_SETS[ps]
    M = len(prm)
    rng = np.random.default_rng(700 + ps)
    hist_len = 4096 // M
    hist = rng.integers(0, V_FULL, M * hist_len).astype(np.uint32)
    # ids on the head blocks' edges (512 rows each), duplicates, ids past the vocabulary
    hist[:8] = [511, 512, 1023, 1024, V_FULL - 1, V_FULL, 2**32 - 1, 511]
    hist[hist_len: hist_len + 20] = 77
    params = [t.RowParams(T, p, k, rp, t.uniform_from_seed(t.splitmix64(50 * ps + m)), CAP,
                          m * hist_len, hist_len) for m, (T, p, k, rp) in enumerate(prm)]
    run_and_check(env, oracle, full_head, hidden_bf16(710 + ps, M, D), params, hist, f"set {ps}")


def _tied_head(torch, dev, t, V, d, top_rows):
    """A head whose rows give exactly 0 for an all-ones hidden row (q = 8 everywhere, b = -8 s:
    every group's products and the bias cancel exactly), except `top_rows`: q = 15, b = 0, the
    same weights in each, so that their logits tie exactly at the top."""
    W = np.full((V, d // 8), 0x88888888, np.uint32)
    S = np.full((V, d // 64), 0x3C23, np.uint16)  # bf16 ~0.00996
    B = (((S.astype(np.uint32) << 16).view(np.float32) * -8).view(np.uint32) >> 16).astype(np.uint16)
    W[top_rows] = 0xFFFFFFFF
    B[top_rows] = 0
    return t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)


def test_fused_all_logits_equal(env, oracle, full_head):
    # a zero hidden row makes every logit exactly 0: the shortlist is the lowest indices; the
    # candidate blocks' survivors overflow the LDS list (the radix path), and top_k = 0 takes
    # 256 of the 512 blocks
    torch, dev, t = env
    params = [t.RowParams(0.8, 0.9, 40, 1.0, 0.61, CAP, 0, 0), t.RowParams(1.0, 1.0, 0, 1.0, 0.37, CAP, 0, 0),
              t.RowParams(0.7, 0.5, 3, 1.2, 0.99, CAP, 0, 6), t.RowParams(0.0, 1.0, 0, 1.0, 0.0, CAP, 0, 0)]
    hist = np.array([0, 1, 2, 600, 0, 70000], np.uint32)
    hb = np.zeros((4, D), np.uint16)
    tok = run_and_check(env, oracle, full_head, hb, params, hist, "all equal")
    assert tok[3] == 0  # greedy: the lowest index


def test_fused_ties_at_the_top(env, oracle):
    # 3000 rows share the top logit exactly, spread over the blocks; the other rows are 0
    torch, dev, t = env
    V, d = 131072, 512
    rng = np.random.default_rng(9)
    top = np.sort(rng.choice(V, 3000, replace=False))
    head = _tied_head(torch, dev, t, V, d, top)
    params = [t.RowParams(0.8, 0.95, 64, 1.0, 0.42, CAP, 0, 0), t.RowParams(1.2, 1.0, 0, 1.1, 0.9, CAP, 0, 500),
              t.RowParams(0.5, 0.7, 200, 1.0, 0.05, CAP, 0, 0)]
    hist = top[:500].astype(np.uint32)  # penalise the first 500 tied rows of row 1
    hb = np.full((3, d), 0x3F80, np.uint16)  # bf16 1.0
    raw = head.logits(torch.from_numpy(hb[:1].view(np.int16)).to(dev)).cpu().numpy()[0]
    assert len(np.unique(raw[top])) == 1 and np.all(raw[np.setdiff1d(np.arange(V), top)] == 0)
    assert raw[top[0]] > 1.0
    run_and_check(env, oracle, head, hb, params, hist, "top ties")
    head.close()


@pytest.mark.parametrize("V", [300, 1000, 5000])
@pytest.mark.parametrize("M", [2, 6])
def test_fused_small_vocabularies(env, oracle, V, M):
    # few head blocks: every block is a candidate (counting for 300, binned top for 1000, radix
    # for 5000 survivors); 2 rows (four apart) and 6 (two apart, 16-wave blocks)
    torch, dev, t = env
    d = 256
    W, S, B = oracle.gen_lm_head(730 + V, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    rng = np.random.default_rng(V)
    hist = rng.integers(0, V + 10, 300).astype(np.uint32)
    params = [t.RowParams(0.7, 0.9, 40, 1.1, 0.3, CAP, 0, 300), t.RowParams(1.0, 1.0, 0, 1.0, 0.8, CAP, 0, 0)]
    params += [t.RowParams(0.6 + 0.1 * m, 0.9, 30 + m, 1.2 if m % 2 else 1.0, 0.1 + 0.2 * m, CAP, 50 * m, 100)
               for m in range(M - 2)]
    run_and_check(env, oracle, head, hidden_bf16(731 + M, M, d), params, hist, f"V={V} M={M}")
    head.close()


@pytest.mark.parametrize("M", [2, 7])
def test_fused_degenerate_row(env, oracle, full_head, M):
    # a NaN hidden row gives NaN logits: that row is degenerate, the others sample normally
    torch, dev, t = env
    hb = hidden_bf16(740 + M, M, D)
    hb[1, 100] = 0x7FC0
    params = [t.RowParams(0.7, 0.9, 40, 1.0, 0.5, CAP, 0, 0)] * M
    tok = run_and_check(env, oracle, full_head, hb, params, np.zeros(0, np.uint32), f"nan row M={M}")
    assert tok[1] == t.TOKEN_DEGENERATE
    assert all(tok[m] != t.TOKEN_DEGENERATE for m in range(M) if m != 1)


@pytest.mark.parametrize("M", [9, 20, 40, 64])
def test_sample_rows_past_the_fused_pass(env, oracle, M):
    # head.sample with more than 4 rows: the logits pass (the staged 16x16 kernel at 9 rows, the
    # 32x32 kernel with one m tile at 20 and two at 40 and 64), then the penalty and the
    # wave-record selection over the logits in memory; per-row parameters and histories
    torch, dev, t = env
    V, d = 3000, 640
    W, S, B = oracle.gen_lm_head(750 + M, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    rng = np.random.default_rng(M)
    hists, params, off = [], [], 0
    for m in range(M):
        n = int(rng.integers(0, 400))
        hists.append(rng.integers(0, V + 10, n).astype(np.uint32))
        T = 0.0 if m % 7 == 3 else float(rng.uniform(0.5, 1.2))
        params.append(t.RowParams(T, float(rng.uniform(0.8, 0.98)), int(rng.integers(20, 101)),
                                  1.0 if m % 5 == 1 else 1.1, float(rng.uniform()), CAP, off, n))
        off += n
    hist = np.concatenate(hists)
    run_and_check(env, oracle, head, hidden_bf16(760 + M, M, d), params, hist, f"M={M}")
    head.close()


@pytest.mark.parametrize("M", [2, 6])
def test_fused_penalty_past_the_softcap(env, oracle, M):
    # The fused pass sums each record against a fixed bound of the row's values when it has one
    # (the softcap, or the penalty's clamp); a penalty without a clamp, or below 1, can take
    # values far past the softcap (v / rp^n grows, v * rp^n falls), where that bound would
    # overflow or underflow exp: such rows are summed against each wave's max. Histories repeat
    # a few ids hundreds of times, so their penalised values reach ~1e6 in magnitude.
    torch, dev, t = env
    V, d = 1000, 256
    W, S, B = oracle.gen_lm_head(770 + M, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    rng = np.random.default_rng(77 + M)
    hist = np.concatenate([np.repeat(rng.integers(0, V, 4).astype(np.uint32), 150),
                           rng.integers(0, V, 400).astype(np.uint32)])
    n = len(hist)
    cases = [
        (0.7, 0.9, 40, 0.95, 0.0),   # rp < 1, no clamp: values grow by 0.95^-150 ~ 2,200x
        (1.0, 0.95, 100, 1.1, 0.0),  # rp > 1, no clamp: negative values fall by 1.1^150 ~ 1.6e6x
        (0.8, 0.9, 64, 0.9, 500.0),  # a clamp at 499.95: past the bound the fixed form allows
        (0.7, 0.9, 40, 1.2, CAP),    # a clamp at the softcap: the fixed reference applies
        (1.2, 1.0, 0, 0.8, 10.0),    # a clamp below the softcap: the softcap bounds the row
        (0.0, 1.0, 0, 0.9, 0.0),     # greedy, grown values
    ]
    params = [t.RowParams(T, p, k, rp, float(rng.uniform()), cap, 0, n)
              for T, p, k, rp, cap in (cases[m % len(cases)] for m in range(M))]
    run_and_check(env, oracle, head, hidden_bf16(780 + M, M, d), params, hist, f"past the cap M={M}")
    head.close()
