"""Calls captured into a HIP graph and replayed.

A captured launch keeps the arguments it was captured with, its arrival-counter epoch among
them, so every replay repeats one epoch. Checked here:
  * head.greedy (the head kernels' grid finish) captured with torch.cuda.CUDAGraph, replayed six
    times with a new hidden state copied in before each replay and eager greedy calls between
    the replays, every replay's tokens against the eager result and the oracle's argmax;
  * two graphs of the same head (two captured epochs) replayed alternately, then eager calls;
  * twd_select_noalloc over all-greedy rows (the one-pass slice finish on its fixed scratch),
    captured and replayed the same way, eager twd_select_noalloc calls in between;
  * a captured call on a stream other than the object's previous one (it waits for nothing).
"""
import ctypes

import numpy as np
import pytest

from helpers import hidden_bf16, twd, wsb_bytes

pytestmark = pytest.mark.gpu

CAP = 30.0


@pytest.fixture(scope="module")
def env(oracle):
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    t = twd()
    dev = torch.device("cuda:0")
    V, d = 50000, 256  # about 100 blocks in the greedy grid
    W, S, B = oracle.gen_lm_head(5150, V, d)
    head = t.LMHead(torch.from_numpy(wsb_bytes(W, S, B)).to(dev), V, d, CAP)
    yield torch, dev, t, head, V, d
    head.close()


def h_dev(torch, dev, hb):
    return torch.from_numpy(np.ascontiguousarray(hb).view(np.int16)).to(dev)


def eager_greedy(env, oracle, hb):
    torch, dev, t, head, V, d = env
    h = h_dev(torch, dev, hb)
    tok = head.greedy(h).cpu().numpy().astype(np.int64).tolist()
    want = [oracle.argmax(r) for r in head.logits(h).cpu().numpy()]
    assert tok == want
    return tok


@pytest.mark.parametrize("M", [1, 5, 24])
def test_head_greedy_graph_replays(env, oracle, M):
    torch, dev, t, head, V, d = env
    s = torch.cuda.Stream()
    h_in = h_dev(torch, dev, hidden_bf16(800 + M, M, d))
    tok_out = torch.zeros(M, dtype=torch.int32, device=dev)
    with torch.cuda.stream(s):
        head.greedy(h_in, tokens=tok_out, stream=s.cuda_stream)  # eager warm-up on the stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        head.greedy(h_in, tokens=tok_out, stream=s.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(6):
        hb = hidden_bf16(900 + 10 * M + rep, M, d)
        want = eager_greedy(env, oracle, hb)  # eager work between the replays
        torch.cuda.synchronize()
        h_in.copy_(h_dev(torch, dev, hb))
        tok_out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert tok_out.cpu().numpy().astype(np.int64).tolist() == want, (M, rep)
    eager_greedy(env, oracle, hidden_bf16(999, M, d))
    del g


def test_two_graphs_of_one_head_alternate(env, oracle):
    torch, dev, t, head, V, d = env
    s = torch.cuda.Stream()
    ins = [h_dev(torch, dev, hidden_bf16(1000 + i, M, d)) for i, M in enumerate((2, 7))]
    outs = [torch.zeros(x.shape[0], dtype=torch.int32, device=dev) for x in ins]
    graphs = []
    for h_in, tok_out in zip(ins, outs):
        with torch.cuda.stream(s):
            head.greedy(h_in, tokens=tok_out, stream=s.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            head.greedy(h_in, tokens=tok_out, stream=s.cuda_stream)
        graphs.append(g)
    torch.cuda.synchronize()
    for rep in range(8):
        i = rep % 2
        hb = hidden_bf16(1100 + rep, ins[i].shape[0], d)
        want = eager_greedy(env, oracle, hb) if rep % 3 == 0 else None
        ins[i].copy_(h_dev(torch, dev, hb))
        torch.cuda.synchronize()
        graphs[i].replay()
        torch.cuda.synchronize()
        got = outs[i].cpu().numpy().astype(np.int64).tolist()
        if want is None:
            want = [oracle.argmax(r) for r in head.logits(ins[i]).cpu().numpy()]
        assert got == want, rep
    for k in range(3):
        eager_greedy(env, oracle, hidden_bf16(1200 + k, 3, d))
    del graphs


def _noalloc(t, lg, params, tok, stream):
    arr = (t.RowParams * len(params))(*params)
    rows, n = lg.shape
    rc = t.twd.lib.twd_select_noalloc(ctypes.c_void_p(lg.data_ptr()), n, rows, n, arr, None,
                                      ctypes.c_void_p(tok.data_ptr()), stream)
    if rc != 0:
        raise t.TwdError(rc, t.twd.last_error())


def test_select_noalloc_greedy_graph_replays(env, oracle):
    # all rows greedy over 262144 entries: 32 slice blocks per row finish the rows themselves
    torch, dev, t, head, V, d = env
    n, rows = 262144, 3
    rng = np.random.default_rng(17)
    params = [t.RowParams(0.0, 1.0, 0, 1.0, 0.0, 0.0, 0, 0)] * rows
    s = torch.cuda.Stream()
    lg_in = torch.from_numpy(rng.standard_normal((rows, n)).astype(np.float32)).to(dev)
    tok_out = torch.zeros(rows, dtype=torch.int32, device=dev)
    with torch.cuda.stream(s):
        _noalloc(t, lg_in, params, tok_out, s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _noalloc(t, lg_in, params, tok_out, s.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(6):
        x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
        x[rep % rows, 100 + rep] = x[rep % rows].max() + 1.0
        x[(rep + 1) % rows, [7, 900]] = x[(rep + 1) % rows].max() + 2.0  # a tie: lowest index
        want = [oracle.argmax(r) for r in x]
        # eager work between the replays: the same entry point on other rows
        other = torch.from_numpy((rng.standard_normal((2, n)) * 2).astype(np.float32)).to(dev)
        tok_e = torch.zeros(2, dtype=torch.int32, device=dev)
        _noalloc(t, other, params[:2], tok_e, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert tok_e.cpu().numpy().tolist() == [oracle.argmax(r) for r in other.cpu().numpy()]
        lg_in.copy_(torch.from_numpy(x))
        tok_out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert tok_out.cpu().numpy().astype(np.int64).tolist() == want, rep
    del g


def test_capture_on_another_stream(env, oracle):
    # the head's last eager call ran on the default stream; a capture on a new stream is
    # accepted and waits for nothing
    torch, dev, t, head, V, d = env
    eager_greedy(env, oracle, hidden_bf16(1300, 4, d))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    h_in = h_dev(torch, dev, hidden_bf16(1301, 4, d))
    tok_out = torch.zeros(4, dtype=torch.int32, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        head.greedy(h_in, tokens=tok_out, stream=s.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        hb = hidden_bf16(1310 + rep, 4, d)
        h_in.copy_(h_dev(torch, dev, hb))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert tok_out.cpu().numpy().astype(np.int64).tolist() == eager_greedy(env, oracle, hb), rep
    del g
