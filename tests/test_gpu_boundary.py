"""GPU checks of the drop-in boundary around the head: the reference's own generation options
and token callback (c_api.h:24-40, c_api.cpp:121-162), the cancel flag and stop rules of
ForwardRunner::generate (runner.cpp:2312-2336), evaluate_verification beyond 64 drafts
(speculator.cpp:34-153 has no bound), and the head's shared grid-finish state: a counter left
non-zero from outside, and calls that alternate between streams. Tokens are compared with the
oracle's reference loop on the GPU's own logits."""
import ctypes

import numpy as np
import pytest

from helpers import hidden_bf16, twd, wsb_bytes

pytestmark = pytest.mark.gpu

CAP = 30.0


@pytest.fixture(scope="module")
def small(oracle):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    dev = torch.device("cuda:0")
    V, d = 3000, 512
    W, S, B = oracle.gen_lm_head(900, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    yield torch, dev, t, head, V, d
    head.close()


def dev_h(torch, dev, hb):
    return torch.from_numpy(np.ascontiguousarray(hb).view(np.int16)).to(dev)


def oracle_loop(oracle, head, torch, dev, hs, prompt, T, p, k, rp, has_seed, seed, n):
    """The reference's decode loop on the GPU's raw logits for n steps: the expected ids."""
    history = list(prompt)
    out = []
    for i in range(n):
        raw = head.logits(dev_h(torch, dev, hs[i:i + 1])).cpu().numpy()[0]
        pos = len(history) - 1
        lg = oracle.apply_repetition_penalty(raw, history, rp, CAP) if rp != 1.0 else raw
        tok = oracle.sample_token(lg, T, p, k, seed=oracle.seed_for(has_seed, seed, pos))
        history.append(tok)
        out.append(tok)
    return out


def test_generator_ex_options_default_and_callback(small, oracle):
    # the struct g4dense_options_default fills (T 0.2, p 0.95, k 64, rp 1, unseeded, 512
    # tokens), and a callback that asks to stop after its fifth id
    torch, dev, t, head, V, d = small
    rng = np.random.default_rng(1)
    prompt = [int(x) for x in rng.integers(0, V, 30)]
    hs = hidden_bf16(21, 8, d)
    want = oracle_loop(oracle, head, torch, dev, hs, prompt, 0.2, 0.95, 64, 1.0, False, 0, 8)
    seen = []

    def on_token(index, tok, delta):
        seen.append((index, tok, delta))
        return index < 4

    gen = t.Generator.from_options(head, t.twd.options_default(), prompt, on_token=on_token)
    toks = []
    for i in range(8):
        tok, fin = gen.step(dev_h(torch, dev, hs[i:i + 1]))
        toks.append(tok)
        if fin:
            break
    assert toks == want[:5]
    assert seen == [(i, want[i], b"") for i in range(5)]
    assert gen.stop_reason() == t.twd.STOP_CALLBACK
    assert gen.tokens() == prompt + want[:5]
    with pytest.raises(t.TwdError) as e:
        gen.step(dev_h(torch, dev, hs[5:6]))
    assert e.value.code == t.twd.TWD_E_INVALID and "finished" in str(e.value)
    gen.close()


def test_generator_ex_options_fields(small, oracle):
    # the sampling fields as c_api.cpp:132-140 copies them (seeded, penalty, top-k), with
    # max_tokens ending the generation, and NULL options meaning GenerationOptions' defaults
    torch, dev, t, head, V, d = small
    rng = np.random.default_rng(2)
    prompt = [int(x) for x in rng.integers(0, V, 25)]
    hs = hidden_bf16(22, 6, d)
    o = t.twd.options_default()
    o.max_tokens, o.temperature, o.top_p, o.top_k = 6, 0.9, 0.9, 40
    o.repetition_penalty, o.has_seed, o.seed, o.tier_id = 1.2, 1, 99, 3
    want = oracle_loop(oracle, head, torch, dev, hs, prompt, 0.9, 0.9, 40, 1.2, True, 99, 6)
    gen = t.Generator.from_options(head, o, prompt)
    got = [gen.step(dev_h(torch, dev, hs[i:i + 1])) for i in range(6)]
    assert [g[0] for g in got] == want and [g[1] for g in got] == [False] * 5 + [True]
    assert gen.stop_reason() == t.twd.STOP_MAX_TOKENS
    gen.close()
    # no options: greedy (SamplingParams{}), 512 tokens
    gen = t.Generator.from_options(head, None, prompt)
    got = [gen.step(dev_h(torch, dev, hs[i:i + 1])) for i in range(3)]
    greedy = oracle_loop(oracle, head, torch, dev, hs, prompt, 0.0, 1.0, 0, 1.0, False, 0, 3)
    assert [g[0] for g in got] == greedy and not any(g[1] for g in got)
    assert gen.stop_reason() == t.twd.STOP_NONE
    gen.close()
    # max_tokens <= 0 emits nothing
    o.max_tokens = 0
    gen = t.Generator.from_options(head, o, prompt)
    assert gen.stop_reason() == t.twd.STOP_MAX_TOKENS
    gen.close()


def test_generator_cancel(small, oracle):
    # runner.cpp:2315: a set cancel flag ends the loop before anything is sampled
    torch, dev, t, head, V, d = small
    prompt = [5, 6, 7]
    hs = hidden_bf16(23, 4, d)
    gen = t.Generator.from_options(head, t.twd.options_default(), prompt)
    first = [gen.step(dev_h(torch, dev, hs[i:i + 1]))[0] for i in range(2)]
    gen.cancel()
    tok, fin = gen.step(dev_h(torch, dev, hs[2:3]))
    assert fin and gen.stop_reason() == t.twd.STOP_CANCELLED
    assert gen.tokens() == prompt + first  # the cancelled step added nothing
    gen.close()


def test_generator_sync_applies_stop_rules(small, oracle):
    # steps enqueued without readback run past a stop id; sync cuts the history after it
    torch, dev, t, head, V, d = small
    rng = np.random.default_rng(4)
    prompt = [int(x) for x in rng.integers(0, V, 20)]
    hs = hidden_bf16(24, 8, d)
    sp = t.SamplingParams(0.8, 0.95, 50, 1.1, True, 7)
    want = oracle_loop(oracle, head, torch, dev, hs, prompt, 0.8, 0.95, 50, 1.1, True, 7, 8)
    stop = want[3]
    first_stop = want.index(stop)  # the first occurrence ends the generation
    gen = t.Generator(head, sp, prompt, 8, stop_ids=[stop])
    for i in range(8):
        gen.step_async(dev_h(torch, dev, hs[i:i + 1]))
    assert gen.sync()
    assert gen.stop_reason() == t.twd.STOP_TOKEN
    assert gen.tokens() == prompt + want[:first_stop + 1]
    gen.close()


def test_generator_sync_reports_degenerate(small, oracle):
    # a NaN hidden state gives NaN logits: sample_token throws (sampling.cpp:116-118); without
    # readback the draw is found by sync, which ends the history before it
    torch, dev, t, head, V, d = small
    prompt = [1, 2, 3]
    hs = hidden_bf16(25, 3, d)
    hs[1, 10] = 0x7FC0  # bf16 NaN
    sp = t.SamplingParams(0.8, 1.0, 0, 1.0, True, 3)
    want0 = oracle_loop(oracle, head, torch, dev, hs, prompt, 0.8, 1.0, 0, 1.0, True, 3, 1)
    gen = t.Generator(head, sp, prompt, 3)
    for i in range(3):
        gen.step_async(dev_h(torch, dev, hs[i:i + 1]))
    with pytest.raises(t.TwdError) as e:
        gen.sync()
    assert e.value.code == t.twd.TWD_E_DEGENERATE
    assert gen.stop_reason() == t.twd.STOP_DEGENERATE
    assert gen.tokens() == prompt + want0
    gen.close()


# ---- evaluate_verification with more than 64 drafts -----------------------------------------

@pytest.mark.parametrize("case", ["greedy_all", "greedy_miss_80", "sampled", "draft_rows"])
def test_verify_100_drafts(small, oracle, case):
    torch, dev, t, head, V, d = small
    rng = np.random.default_rng(100)
    K, n = 100, 2048
    rows = (rng.standard_normal((K + 1, n)) * 2).astype(np.float32)
    T, p, k = (0.0, 1.0, 0) if case.startswith("greedy") else (0.8, 0.9, 40)
    base = 4242
    target = [oracle.sample_token(rows[i], T, p, k, seed=oracle.splitmix64(base + i))
              for i in range(K + 1)]
    drafts = list(target[:K])
    if case == "greedy_miss_80":
        drafts[80] = (drafts[80] + 1) % n
    if case == "sampled":
        drafts[90] = (drafts[90] + 7) % n
    sp = t.SamplingParams(T, p, k, 1.0, True, 1)
    lg = torch.from_numpy(rows).to(dev)
    dl = ()
    if case == "draft_rows":
        dr = [None] * K
        draft_np = {i: (rows[i] + rng.standard_normal(n).astype(np.float32)) for i in (3, 70, 75)}
        for i, r in draft_np.items():
            dr[i] = torch.from_numpy(r).to(dev)
        dl = dr
        want = oracle.verify_draft(drafts, list(rows), [draft_np.get(i) for i in range(K)], t=T,
                                   p=p, k=k, base_seed=base)
    else:
        want = oracle.verify(drafts, list(rows), t=T, p=p, k=k, base_seed=base)
    got = t.SpeculativeCoordinator().evaluate_verification(drafts, lg, n, sp, base, dl)
    for key in ("tokens", "num_accepted", "total_drafted", "bonus_token_sampled"):
        assert got[key] == want[key], (key, got[key], want[key])
    if case == "greedy_all":
        assert got["num_accepted"] == K and got["bonus_token_sampled"]
    if case == "greedy_miss_80":
        assert got["num_accepted"] == 80


def test_verify_100_drafts_against_reference_build(small, oracle, reference):
    # the reference's own evaluate_verification (oracle/_ref) on the same rows
    torch, dev, t, head, V, d = small
    rng = np.random.default_rng(101)
    K, n = 100, 1024
    rows = (rng.standard_normal((K + 1, n)) * 2).astype(np.float32)
    drafts = [int(np.argmax(rows[i])) for i in range(K)]
    drafts[70] = (drafts[70] + 1) % n
    want = reference.verify(drafts, list(rows), t=0.0, base_seed=9)
    got = t.SpeculativeCoordinator().evaluate_verification(
        drafts, torch.from_numpy(rows).to(dev), n, t.SamplingParams(), 9)
    assert got["tokens"] == want["tokens"] and got["num_accepted"] == want["num_accepted"] == 70


# ---- the head's grid-finish state --------------------------------------------------------------

def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    return hip


@pytest.mark.parametrize("M", [1, 5, 40])
def test_greedy_after_counter_left_nonzero(small, oracle, M):
    # a plain host copy writes the arrival counter (what a launch that stopped part-way would
    # leave, and arbitrary values); the next greedy call must still finish in the right block
    torch, dev, t, head, V, d = small
    hip = _hip()
    state = t.twd.lib.twd_head_finish_state(head.handle)
    assert state
    ctr_addr = state + 64 * 8
    hs = hidden_bf16(30 + M, M, d)
    h = dev_h(torch, dev, hs)
    want = [oracle.argmax(r) for r in head.logits(h).cpu().numpy()]
    assert head.greedy(h).cpu().numpy().astype(np.int64).tolist() == want
    torch.cuda.synchronize()
    cur = ctypes.c_uint64()
    assert hip.hipMemcpy(ctypes.byref(cur), ctr_addr, 8, 2) == 0
    nxt = cur.value & 0xFFFFFFFF
    assert cur.value >> 32 == 0 and nxt > 0  # armed for the next launch's epoch
    # a launch of the previous epoch that stopped after 7 blocks, another epoch's count,
    # all ones, and zero
    for garbage in ((7 << 32) | (nxt - 1), (3 << 32) | (nxt + 1000), 0xFFFFFFFFFFFFFFFF, 0):
        torch.cuda.synchronize()
        g = ctypes.c_uint64(garbage)
        assert hip.hipMemcpy(ctr_addr, ctypes.byref(g), 8, 1) == 0
        tok = head.greedy(h).cpu().numpy().astype(np.int64).tolist()
        assert tok == want, hex(garbage)
        tok = head.greedy(h).cpu().numpy().astype(np.int64).tolist()  # and the launch after it
        assert tok == want, hex(garbage)
    torch.cuda.synchronize()
    assert hip.hipMemcpy(ctypes.byref(cur), ctr_addr, 8, 2) == 0
    assert cur.value >> 32 == 0 and cur.value & 0xFFFFFFFF != 0  # armed again


def test_calls_alternating_between_streams(small, oracle):
    # greedy calls on two streams, enqueued back to back without host waits: the head orders
    # them, so each finishes with its own rows' tokens (M=40 also shares the staged h)
    torch, dev, t, head, V, d = small
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cases = []
    for i, M in enumerate([1, 40, 5, 40, 1, 8, 40, 2]):
        hs = hidden_bf16(200 + i, M, d)
        h = dev_h(torch, dev, hs)
        want = [oracle.argmax(r) for r in head.logits(h).cpu().numpy()]
        cases.append((h, want))
    torch.cuda.synchronize()
    outs = []
    for rep in range(3):
        for i, (h, want) in enumerate(cases):
            s = streams[(i + rep) % 2]
            with torch.cuda.stream(s):
                tok = torch.empty(h.shape[0], dtype=torch.int32, device=dev)
                head.greedy(h, tokens=tok, stream=s.cuda_stream)
            outs.append((tok, want))
    torch.cuda.synchronize()
    for tok, want in outs:
        assert tok.cpu().numpy().astype(np.int64).tolist() == want
