"""The composed sampled chains at the BASELINE geometry (V=262144, d=5376): the LM head, then the
repetition penalty in place, then sample_token, as runner.cpp:2314-2328 runs them per step.

Configs 3 (M=1, T=0.7 k=40 p=0.9, rp 1.1 over a 4096-id history that grows by each sampled id)
and 5 (M=64, per-row T/k/p, rp 1.1 over a 2048-id history per row). Every token is compared
bit-exactly with the oracle's apply_repetition_penalty + sample_token run on the GPU's own raw
logits (the same kernel, called for logits alone on the same h), and the penalised rows are
compared bit for bit. The oracle's cut margin |run - p| and draw margin |acc - r| are logged per
row; a mismatch fails with them. Raw logits are checked at sampled rows against the scalar CPU
LM head within the reference's 1e-3 tolerance (tests/test_gpu_kernels.cpp:345)."""
import numpy as np
import pytest

from helpers import allclose_report, bf16_to_f32, hidden_bf16, twd

pytestmark = pytest.mark.gpu

V = 262144
D = 5376
CAP = 30.0
SEED_FULL = 20260801


@pytest.fixture(scope="module")
def env():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    dev = torch.device("cuda:0")
    wsb = torch.empty(t.head_bytes(V, D), dtype=torch.uint8, device=dev)
    t.generate_head(wsb, V, D, SEED_FULL)
    head = t.LMHead(wsb, V, D, CAP)
    yield torch, dev, t, head
    head.close()


def to_dev(torch, dev, a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a).view(dtype)).to(dev)


def check_logit_rows(oracle, raw, hb, rows):
    """Raw (softcapped) logits of hidden row hb at the vocabulary rows `rows` against the
    oracle's scalar LM head (cpu_reference.cpp:643-665) on the same synthetic weights."""
    W, S, B = zip(*[oracle.gen_lm_head(SEED_FULL, 1, D, row0=int(r)) for r in rows])
    want = oracle.lm_head(np.concatenate(W), np.concatenate(S), np.concatenate(B),
                          bf16_to_f32(hb), D, softcap=CAP)
    ratio, err, _ = allclose_report(raw[rows], want, 1e-3, 1e-3)
    assert ratio <= 1.0, (ratio, err)


def expect_row(oracle, raw, history, T, p, k, rp, u, got_pen, got_tok, tag):
    """The reference's step on the GPU's raw logits; asserts the penalised row and the token.
    Returns the oracle's smallest margin."""
    pen = oracle.apply_repetition_penalty(raw, history, rp, CAP) if rp != 1.0 else raw
    assert np.array_equal(got_pen.view(np.uint32), pen.view(np.uint32)), f"{tag}: penalised row"
    want, dg = oracle.sample_token(pen, T, p, k, u=u, diag=True)
    margin = min(dg["cut_margin"], dg["draw_margin"])
    print(f"{tag}: token {want} cut {dg['cut']}/{dg['want']} cut-margin {dg['cut_margin']:.3e} "
          f"draw-margin {dg['draw_margin']:.3e}")
    assert got_tok == want, (f"{tag}: GPU {got_tok} != oracle {want}; cut margin "
                             f"{dg['cut_margin']:.3e}, draw margin {dg['draw_margin']:.3e}")
    return want, margin


def test_config3_chain_16_steps(env, oracle):
    # BASELINE config 3 through the decode-loop generator: a 4096-id prompt history, each
    # sampled id appended (runner.cpp:2328), seed_for(position) draws, fresh h per step
    torch, dev, t, head = env
    rng = np.random.default_rng(3003)
    prompt = [int(x) for x in rng.integers(0, V, 4096)]
    sp = t.SamplingParams(0.7, 0.9, 40, 1.1, True, 777)
    steps = 16
    gen = t.Generator(head, sp, prompt, steps)
    history = list(prompt)
    hs = hidden_bf16(3100, steps, D)
    worst = np.inf
    for i in range(steps):
        h = to_dev(torch, dev, hs[i:i + 1], np.int16)
        raw = head.logits(h).cpu().numpy()[0]  # the kernel of the sampled pass, logits alone
        if i % 4 == 0:
            check_logit_rows(oracle, raw, hs[i], np.unique(np.concatenate(
                [rng.integers(0, V, 96), [0, V - 1, int(np.argmax(raw))]])))
        tok, fin = gen.step(h)
        pos = len(history) - 1
        u = t.uniform_from_seed(t.seed_for(sp, pos))
        pen = oracle.apply_repetition_penalty(raw, history, 1.1, CAP)
        want, dg = oracle.sample_token(pen, 0.7, 0.9, 40, u=u, diag=True)
        worst = min(worst, dg["cut_margin"], dg["draw_margin"])
        print(f"step {i}: token {want} cut {dg['cut']} cut-margin {dg['cut_margin']:.3e} "
              f"draw-margin {dg['draw_margin']:.3e}")
        assert tok == want, (f"step {i}: GPU {tok} != oracle {want}; cut margin "
                             f"{dg['cut_margin']:.3e}, draw margin {dg['draw_margin']:.3e}")
        history.append(want)
        assert fin == (i == steps - 1)
    assert gen.tokens() == history
    gen.close()
    print(f"config 3: {steps} steps bit-exact, smallest margin {worst:.3e}")


def test_config3_head_sample_direct(env, oracle):
    # the same chain through twd_head_sample itself, the entry point bench.py times: the
    # caller's device history, its penalised logits returned in place
    torch, dev, t, head = env
    rng = np.random.default_rng(3004)
    hist = rng.integers(0, V, 4096 + 8).astype(np.uint32)
    hist[100:140] = hist[7]  # one id 41 times: the penalty compounds 41 times
    hist_dev = to_dev(torch, dev, hist, np.int32)
    hs = hidden_bf16(3200, 8, D)
    for i in range(8):
        h = to_dev(torch, dev, hs[i:i + 1], np.int16)
        raw = head.logits(h).cpu().numpy()[0]
        u = t.uniform_from_seed(t.splitmix64(9000 + i))
        prm = [t.RowParams(0.7, 0.9, 40, 1.1, u, CAP, i, 4096)]
        tok, lg = head.sample(h, prm, history=hist_dev)
        expect_row(oracle, raw, hist[i:i + 4096], 0.7, 0.9, 40, 1.1, u, lg.cpu().numpy()[0],
                   int(tok.cpu().item()) & 0xFFFFFFFF, f"direct step {i}")


@pytest.mark.parametrize("trial", [0, 1])
def test_config5_chain_m64(env, oracle, trial):
    # 64 rows on the MFMA path, each with its own T/k/p, rp 1.1 over its own
    # 2048-id history and its own uniform, through twd_head_sample
    torch, dev, t, head = env
    M = 64
    rng = np.random.default_rng(5005 + trial)
    hb = hidden_bf16(5100 + trial, M, D)
    h = to_dev(torch, dev, hb, np.int16)
    hist = rng.integers(0, V, M * 2048).astype(np.uint32)
    hist[5 * 2048: 5 * 2048 + 30] = hist[5 * 2048 + 40]  # duplicates inside one row's history
    hist_dev = to_dev(torch, dev, hist, np.int32)
    Ts = rng.uniform(0.5, 1.2, M).astype(np.float32)
    ks = rng.integers(20, 101, M)
    ps = rng.uniform(0.8, 0.98, M).astype(np.float32)
    us = [t.uniform_from_seed(t.splitmix64(100 * trial + m)) for m in range(M)]
    prm = [t.RowParams(float(Ts[m]), float(ps[m]), int(ks[m]), 1.1, us[m], CAP, 2048 * m, 2048)
           for m in range(M)]
    raw = head.logits(h).cpu().numpy()
    tok, lg = head.sample(h, prm, history=hist_dev)
    tok = tok.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    lg = lg.cpu().numpy()
    sample = np.unique(np.concatenate([rng.integers(0, V, 96), [0, V - 1]]))
    for m in (0, 17, 63):
        check_logit_rows(oracle, raw[m], hb[m], sample)
    worst = np.inf
    for m in range(M):
        _, margin = expect_row(oracle, raw[m], hist[2048 * m: 2048 * (m + 1)], float(Ts[m]),
                               float(ps[m]), int(ks[m]), 1.1, us[m], lg[m], int(tok[m]),
                               f"trial {trial} row {m}")
        worst = min(worst, margin)
    print(f"config 5 trial {trial}: 64 rows bit-exact, smallest margin {worst:.3e}")
