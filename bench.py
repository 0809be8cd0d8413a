"""LM-head + token-selection throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-power]
                    [--configs 1,2,3,4,5]

Headline (`value`): BASELINE config 2 -- the INT4 g64 LM head at M=1 (V=262144, d=5376, bf16 h)
with the softcap and greedy argmax fused, rows/s with every input already resident in HBM.
One step = one launch over one hidden row. The other BASELINE configs are timed the same way and
reported under "configs". `roofline` is the dominant kernel (the head pass of config 2): its
algorithmic bytes per launch divided by its mean launch duration, measured with HIP events on
the stream the kernel runs on. `cpu_baseline` times the reference's CPU path (restated in oracle/:
the scalar LM head of src/cpu_reference.cpp:643-665, then the config's selection or verify) on a
bounded sample of each config, one thread; its `value` is config 2's.
Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import hashlib
import importlib
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
V, D, G, CAP = 262144, 5376, 64, 30.0
HEAD_BYTES = V * (D // 2 + 4 * D // 64)  # 792,723,456
PEAK_HBM = 8.0e12
PEAK_BF16 = 2.5e15
SEED = 20260801


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def algorithmic_bytes(rows: int, hist_per_row: int = 0) -> int:
    """Weights once per pass + bf16 h per row + history ids + one id out per row."""
    return HEAD_BYTES + rows * D * 2 + rows * 4 * hist_per_row + rows * 4


def bf16_rne(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def hidden_pool(torch, dev, n, rows, seed):
    h = bf16_rne(np.random.default_rng(seed).standard_normal((n, rows, D)).astype(np.float32))
    return torch.from_numpy(h.view(np.int16)).to(dev)


def time_loop(torch, steps, warmup, step_fn, min_warm_s=0.1):
    """Runs `warmup` untimed steps (more, in chunks, until at least `min_warm_s` of warmup has
    passed: after the host-side set-up between configs the first few milliseconds of launches
    run measurably slower), then `steps` timed ones bracketed by synchronize + HIP events on the
    current stream (the stream every launch below uses). Returns seconds on the GPU clock
    between the two events."""
    t0 = time.perf_counter()
    i = 0
    while True:
        for _ in range(max(warmup, 1)):
            step_fn(i)
            i += 1
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= min_warm_s:
            break
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for k in range(steps):
        step_fn(i + k)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3


def launch_percentiles(torch, n, step_fn):
    """Each of n launches between its own pair of HIP events (after the timed region, so the
    GPU is warm): the p10 / p50 / p90 of single-launch durations in microseconds."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i, (a, b) in enumerate(evs):
        a.record()
        step_fn(i)
        b.record()
    torch.cuda.synchronize()
    us = np.array([a.elapsed_time(b) * 1e3 for a, b in evs])
    return {f"launch_us_p{q}": float(np.percentile(us, q)) for q in (10, 50, 90)}


def under_profiler() -> bool:
    """True when a profiler's library is preloaded into this process (rocprofv3 sets these):
    its child processes would initialise the GPU too, so no amd-smi child is started then."""
    env = " ".join(os.environ.get(k, "") for k in ("LD_PRELOAD", "ROCP_TOOL_LIBRARIES", "HSA_TOOLS_LIB"))
    return "rocprof" in env


def power_during(torch, seconds, step_fn):
    """Runs step_fn back to back for `seconds` (after the timed regions, outside every one of
    them) while `amd-smi metric -p -c`, started as a child process, samples the socket power
    and the eight XCDs' graphics clocks. Returns the medians over the samples taken once the
    loop has run for half a second, or None where amd-smi is not available."""
    import shutil
    import subprocess
    import threading
    exe = shutil.which("amd-smi")
    if not exe or under_profiler():
        return None
    samples, stop = [], threading.Event()

    def sampler():
        time.sleep(0.5)
        while not stop.is_set():
            try:
                out = subprocess.run([exe, "metric", "-p", "-c", "--csv"], capture_output=True,
                                     text=True, timeout=10).stdout
                lines = [ln for ln in out.splitlines() if ln.strip()]
                rec = dict(zip(lines[0].split(","), lines[1].split(",")))
                clks = [float(rec[f"gfx_{x}_clk"]) for x in range(8) if f"gfx_{x}_clk" in rec]
                samples.append((float(rec["socket_power"]), sum(clks) / len(clks)))
            except (OSError, ValueError, KeyError, IndexError, ZeroDivisionError,
                    subprocess.SubprocessError):
                pass
            time.sleep(0.2)

    th = threading.Thread(target=sampler)
    th.start()
    t0, i = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            step_fn(i)
            i += 1
        torch.cuda.synchronize()
    stop.set()
    th.join()
    if not samples:
        return None
    w, mhz = np.median(np.array(samples), axis=0)
    return {"socket_w": float(w), "gfx_mhz": float(mhz), "samples": len(samples),
            "loop_s": seconds, "source": "amd-smi metric -p -c (socket power, mean of the XCD clocks)"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _head_arrays(host):
    wpr, gpr = D // 8, D // G
    W = host[: V * wpr * 4].view(np.uint32).reshape(V, wpr)
    S = host[V * wpr * 4: V * wpr * 4 + V * gpr * 2].view(np.uint16).reshape(V, gpr)
    B = host[V * wpr * 4 + V * gpr * 2:].view(np.uint16).reshape(V, gpr)
    return W, S, B


def _rows_f32(rows_bf16):
    return (np.asarray(rows_bf16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def cpu_baseline(host, work: dict, rows2: int):
    """The reference's CPU path, restated in oracle/ (built -O3, one thread), on the same
    weights, hidden rows, histories and parameters the GPU legs use: the scalar LM head
    (cpu_reference.cpp:643-665) with softcap for every row, then per config what the engine
    does with the row -- greedy argmax (config 2), apply_repetition_penalty + sample_token
    (sampling.cpp:74-169; configs 3 and 5), evaluate_verification's greedy branch
    (speculator.cpp:34-69; config 4) -- and config 1's selection alone on its 1 MB row. Each
    config runs on a bounded sample; its rows/s is rows / (the sample's wall time)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    W, S, B = _head_arrays(host)
    where = f"one thread of {cpu_model()}, nproc={os.cpu_count()}"
    per = {}

    def head_row(hb):
        return O.lm_head(W, S, B, _rows_f32(hb), D, softcap=CAP)

    # config 2: head + softcap + greedy over `rows2` rows
    t0 = time.perf_counter()
    for m in range(rows2):
        O.argmax(head_row(work[2][m]))
    dt = time.perf_counter() - t0
    per["2"] = {"rows_per_s": rows2 / dt, "sample": f"{rows2} rows in {dt:.1f} s"}
    value = rows2 / dt

    # config 1: selection alone on the 1 MB row (softcapped N(0, 4^2)), greedy and T=.8 k=64
    # p=.95 u=.37
    z = work.get(1)
    reps = 20
    if z is None:
        reps = 0
    t0 = time.perf_counter()
    for _ in range(reps):
        O.argmax(z)
    tg = (time.perf_counter() - t0) / max(reps, 1)
    t0 = time.perf_counter()
    for _ in range(reps):
        O.sample_token(z, 0.8, 0.95, 64, u=0.37)
    ts = (time.perf_counter() - t0) / max(reps, 1)
    if reps:
        per["1"] = {"greedy_us_per_row": tg * 1e6, "sampled_us_per_row": ts * 1e6,
                    "sample": f"{reps} passes each over the {V}-entry row"}
    if 3 not in work or 4 not in work or 5 not in work:
        return {"value": value, "unit": "rows/s", "cores": 1, "kind": "port",
                "sample": f"config 2: {rows2} full rows; oracle built -O3; {where}", "configs": per}

    # config 3: head + penalty over a 4096-id history + sample_token (T .7, k 40, p .9) per step
    hs3, hist3, us3 = work[3]
    n3 = 2
    t0 = time.perf_counter()
    sel_s = 0.0
    for i in range(n3):
        lg = head_row(hs3[i])
        t1 = time.perf_counter()
        pen = O.apply_repetition_penalty(lg, hist3[i: i + 4096], 1.1, CAP)
        O.sample_token(pen, 0.7, 0.9, 40, u=us3[i])
        sel_s += time.perf_counter() - t1
    dt = time.perf_counter() - t0
    per["3"] = {"rows_per_s": n3 / dt, "selection_us_per_row": sel_s / n3 * 1e6,
                "sample": f"{n3} steps in {dt:.1f} s (head + penalty + sample_token each)"}

    # config 4: five rows through the head, then the greedy verify of four drafts
    hs4, drafts4 = work[4]
    t0 = time.perf_counter()
    rows = [head_row(hs4[m]) for m in range(5)]
    t1 = time.perf_counter()
    O.verify([int(x) for x in drafts4], rows, base_seed=0)
    tv = time.perf_counter() - t1
    dt = time.perf_counter() - t0
    per["4"] = {"rows_per_s": 5 / dt, "verify_us": tv * 1e6,
                "sample": f"one 5-row verify in {dt:.1f} s"}

    # config 5: per row, head + its own penalty and parameters + sample_token
    hs5, hist5, prm5 = work[5]
    n5 = 2
    t0 = time.perf_counter()
    sel_s = 0.0
    for m in range(n5):
        lg = head_row(hs5[m])
        T, p, k, u = prm5[m]
        t1 = time.perf_counter()
        pen = O.apply_repetition_penalty(lg, hist5[2048 * m: 2048 * (m + 1)], 1.1, CAP)
        O.sample_token(pen, T, p, k, u=u)
        sel_s += time.perf_counter() - t1
    dt = time.perf_counter() - t0
    per["5"] = {"rows_per_s": n5 / dt, "selection_us_per_row": sel_s / n5 * 1e6,
                "sample": f"rows 0..{n5 - 1} of the 64 in {dt:.1f} s"}
    return {"value": value, "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"config 2: {rows2} full rows (all {V} vocabulary rows, fp32 scalar dot as "
                      f"cpu_reference.cpp:643-665, softcap, argmax); oracle built -O3; {where}",
            "configs": per}


def cpp_verify_timing():
    """Runs tests/cpp/verify_timing (built by __graft_entry__.build) as a child process on the
    config-4 shape; its JSON line, or None when the program is not built."""
    import subprocess
    exe = os.path.join(ROOT, "tests", "cpp", "verify_timing")
    if not os.path.exists(exe):
        return None
    try:
        out = subprocess.run([exe, "400"], capture_output=True, text=True, timeout=120, check=True).stdout
        return json.loads(out.strip().splitlines()[-1])
    except (subprocess.SubprocessError, ValueError, IndexError, OSError):
        return None


def measured_traffic():
    """HBM bytes per launch of the config-2 kernel from the committed PMC summary
    (FETCH_SIZE and WRITE_SIZE passes, calibrated on a 1 GiB copy), or None."""
    path = os.path.join(ROOT, "profiles", "head_m1_greedy_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1]), "profiles/head_m1_greedy_traffic.md"
    except OSError:
        pass
    return None, None


def rows_sweep(torch, dev, twd, rounds: int = 3, n: int = 200):
    """The head's time by rows, and the fused sample pass against the two-pass form, each the
    median over `rounds` interleaved rounds of `n` back-to-back calls on one stream."""
    log("rows sweep: head by M, fused sample pass against logits + selector")
    wsb = torch.empty(HEAD_BYTES, dtype=torch.uint8, device=dev)
    twd.generate_head(wsb, V, D, SEED)
    head = twd.LMHead(wsb, V, D, CAP)
    sel = twd.Selector(V, 64)
    stream = torch.cuda.current_stream().cuda_stream
    hp = hidden_pool(torch, dev, 8, 64, 7)
    lg = torch.empty(64, V, dtype=torch.float32, device=dev)
    tk = torch.empty(64, dtype=torch.int32, device=dev)
    rng = np.random.default_rng(77)
    hist = torch.from_numpy(rng.integers(0, V, 8 * 2048, dtype=np.int64).astype(np.int32)).to(dev)
    # config 3's chain parameters (T = 0.7, k = 40, p = 0.9, rp 1.1) on every row, over 2,048
    # history ids per row: eight such rows stay within the fused pass's 16,384 ids
    prm = [twd.RowParams(0.7, 0.9, 40, 1.1, float(rng.uniform()), CAP, 2048 * m, 2048)
           for m in range(8)]
    cases = {}
    for m in (1, 2, 3, 4, 5, 8, 16, 32, 48, 64):
        cases[f"logits_M{m}"] = (lambda mm: lambda i: head.logits(hp[i % 8, :mm], out=lg[:mm],
                                                                  stream=stream))(m)
        cases[f"greedy_M{m}"] = (lambda mm: lambda i: head.greedy(hp[i % 8, :mm], tokens=tk[:mm],
                                                                  stream=stream))(m)
    for m in (1, 4, 5, 6, 8):
        cases[f"sample_fused_M{m}"] = (lambda mm: lambda i: head.sample(
            hp[i % 8, :mm], prm[:mm], history=hist, logits=lg[:mm], tokens=tk[:mm],
            stream=stream))(m)

        def two_pass(i, mm=m):
            head.logits(hp[i % 8, :mm], out=lg[:mm], stream=stream)
            sel.select(lg[:mm], prm[:mm], history=hist, tokens=tk[:mm], stream=stream)
        cases[f"logits_then_select_M{m}"] = two_pass
    got = {k: [] for k in cases}
    for _ in range(rounds):
        for k, fn in cases.items():
            got[k].append(time_loop(torch, n, 10, fn, min_warm_s=0.02) / n * 1e6)
    sel.close()
    print(json.dumps({"rows_sweep_us": {k: round(float(np.median(v)), 2) for k, v in got.items()},
                      "rounds": rounds, "calls_per_round": n,
                      "note": "back-to-back calls on one stream, median over interleaved rounds; "
                              "sample rows: rp 1.1 over 2048 ids each, T 0.7, k 40, p 0.9"}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--configs", default="1,2,3,4,5")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-power", action="store_true",
                    help="skip the amd-smi power sampling (skipped anyway when a profiler's library "
                         "is preloaded: it would initialise the GPU in the child processes too)")
    ap.add_argument("--cpu-rows", type=int, default=3,
                    help="full rows of config 2 in the CPU baseline (each about 1.7 s; the other "
                         "configs add about 15 s)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (FETCH_SIZE/WRITE_SIZE calibration)")
    ap.add_argument("--rows-sweep", action="store_true",
                    help="only time the head by rows (logits and greedy, M = 1..64) and the fused "
                         "sample pass against the logits pass + selector (M = 1, 4..8), back to "
                         "back in interleaved rounds; prints one JSON line of its own")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the vocabulary-sharded form across GPUs is a design, not built)", file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.copy_calibration:
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device=dev)
        b = torch.empty(n, dtype=torch.uint8, device=dev)
        a.fill_(1)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "launches": 5}))
        return

    sys.path.insert(0, ROOT)
    twd = importlib.import_module("turbo-winfare-dense_amd")
    if args.rows_sweep:
        rows_sweep(torch, dev, twd)
        return
    cfgs = {int(c) for c in args.configs.split(",") if c}
    cfgs.add(2)
    work = {}  # each config's inputs, for the CPU baseline

    log(f"generating the synthetic head V={V} d={D} ({HEAD_BYTES / 1e6:.1f} MB) on {dev}")
    wsb = torch.empty(HEAD_BYTES, dtype=torch.uint8, device=dev)
    twd.generate_head(wsb, V, D, SEED)
    head = twd.LMHead(wsb, V, D, CAP)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    results = {}

    # ---- config 2: M=1, fused head + softcap + greedy argmax -------------------------------------
    log("config 2: M=1 greedy")
    hp = hidden_pool(torch, dev, 64, 1, 2)
    tok = torch.empty(1, dtype=torch.int32, device=dev)

    def step2(i):
        head.greedy(hp[i % 64], tokens=tok, stream=stream)

    region_s = time_loop(torch, args.steps, args.warmup, step2)
    step_s = region_s / args.steps  # one launch per step: the mean launch-to-launch time
    rows_s = args.steps / region_s
    bytes2 = algorithmic_bytes(1)
    results[2] = {"rows_per_s": rows_s, "ms_per_step": step_s * 1e3,
                  "kernel_us_mean": step_s * 1e6, "hbm_frac": bytes2 / step_s / PEAK_HBM}
    results[2].update(launch_percentiles(torch, 200, step2))
    log(f"config 2: {rows_s:.1f} rows/s, {step_s * 1e6:.1f} us per launch, "
        f"{bytes2 / step_s / 1e12:.2f} TB/s")

    # the same row entering as the model's fp32 hidden state, with the final RMSNorm (eps 1e-6,
    # bf16 weight) computed as the head's prologue
    xr = torch.from_numpy(np.random.default_rng(22).uniform(-2, 2, (64, 1, D)).astype(np.float32)).to(dev)
    nw = torch.from_numpy(bf16_rne(np.random.default_rng(23).uniform(0.5, 1.5, D).astype(np.float32))
                          .view(np.int16)).to(dev)

    def step2n(i):
        head.greedy_rmsnorm(xr[i % 64], nw, tokens=tok, stream=stream)

    nn = max(100, args.steps // 4)
    r_n = time_loop(torch, nn, args.warmup, step2n)
    results[2]["rmsnorm_prologue_us_per_row"] = r_n / nn * 1e6

    # ---- config 1: selection only over one fp32 row (1 MB): greedy, then T=.8 k=64 p=.95 u=.37 ----
    if 1 in cfgs:
        log("config 1: select on one 1 MB row")
        sel = twd.Selector(V, 1)
        z = np.random.default_rng(1).standard_normal(V).astype(np.float32) * 4.0
        z = (30.0 * np.tanh(z / 30.0)).astype(np.float32)
        zr = torch.from_numpy(z).to(dev).view(1, V)
        work[1] = z
        t1 = torch.empty(1, dtype=torch.int32, device=dev)
        p_g = [twd.RowParams(0.0, 1.0, 0, 1.0, 0.0, CAP, 0, 0)]
        p_s = [twd.RowParams(0.8, 0.95, 64, 1.0, 0.37, CAP, 0, 0)]
        out = {}
        for name, pr in (("greedy", p_g), ("sampled", p_s)):
            def step1(i, pr=pr):
                sel.select(zr, pr, tokens=t1, stream=stream)
            n1 = max(50, args.steps // 4)
            r_s = time_loop(torch, n1, 10, step1)
            out[name] = {"us_per_row": r_s / n1 * 1e6}
        results[1] = out

    # ---- config 3: M=1 full chain, rp 1.1 over a 4096-id history, T=.7 k=40 p=.9, 1000 steps --
    if 3 in cfgs:
        log("config 3: M=1 sampled chain, 1000 steps")
        n3 = 1000
        hp3 = hidden_pool(torch, dev, n3, 1, 3)
        rng = np.random.default_rng(33)
        hist = torch.from_numpy(rng.integers(0, V, 4096 + n3 + 20, dtype=np.int64).astype(np.int32)).to(dev)
        lg3 = torch.empty(1, V, dtype=torch.float32, device=dev)
        t3 = torch.empty(1, dtype=torch.int32, device=dev)
        sp = twd.SamplingParams(0.7, 0.9, 40, 1.1, True, 12345)
        # the history is a sliding 4096-id window; uniforms follow seed_for(sp, position)
        prm = [[twd.RowParams(0.7, 0.9, 40, 1.1, twd.uniform_from_seed(twd.seed_for(sp, 4096 + i)),
                              CAP, i, 4096)] for i in range(n3 + 20)]
        work[3] = (hp3[:4].cpu().numpy().view(np.uint16).reshape(-1, D), hist.cpu().numpy().view(np.uint32),
                   [prm[i][0].uniform for i in range(4)])

        def step3(i):
            head.sample(hp3[i % n3], prm[i % len(prm)], history=hist, logits=lg3, tokens=t3,
                        stream=stream)

        r_s = time_loop(torch, n3, 20, step3)
        b3 = algorithmic_bytes(1, 4096)
        results[3] = {"rows_per_s": n3 / r_s, "ms_per_step": r_s * 1e3 / n3,
                      "hbm_frac": b3 / (r_s / n3) / PEAK_HBM}

        # the same chain through the decode-loop generator: a 4096-id prompt, each sampled id
        # appended to the device history as runner.cpp:2328 does, no host round trip per step
        prompt3 = [int(x) for x in rng.integers(0, V, 4096)]

        def gen_run(readback):
            g = twd.Generator(head, sp, prompt3, n3 + 200)
            step = (lambda i: g.step(hp3[i % n3], stream=stream)) if readback else (
                lambda i: twd.twd.lib.twd_generator_step(g.handle, hp3[i % n3].data_ptr(), stream,
                                                     None, None))
            r = time_loop(torch, n3, 20, step, min_warm_s=0.0)
            g.close()
            return r

        r_g = gen_run(False)
        r_gr = gen_run(True)
        results[3]["generator_rows_per_s"] = n3 / r_g
        results[3]["generator_with_token_readback_rows_per_s"] = n3 / r_gr

    # ---- config 4: M=5 greedy verify of 4 drafts ------------------------------------------------
    if 4 in cfgs:
        log("config 4: M=5 verify")
        hp4 = hidden_pool(torch, dev, 64, 5, 4)
        # the drafts as BASELINE config 4 draws them: position by position, the target row's
        # argmax with probability 0.6, otherwise a random id (the argmax from a greedy pass over
        # the same rows, outside the timed region)
        tgt = torch.empty(64, 5, dtype=torch.int32, device=dev)
        for c in range(64):
            head.greedy(hp4[c], tokens=tgt[c], stream=stream)
        tgt_np = tgt.cpu().numpy()
        drng = np.random.default_rng(4)
        dr = np.empty((64, 4), np.int32)
        for c in range(64):
            for i in range(4):
                dr[c, i] = tgt_np[c, i] if drng.random() < 0.6 else drng.integers(0, V)
        drafts = torch.from_numpy(dr).to(dev)
        res4 = torch.zeros(twd.twd.VERIFY_WORDS, dtype=torch.int32, device=dev)
        work[4] = (hp4[0].cpu().numpy().view(np.uint16), drafts[0].cpu().numpy().view(np.uint32))

        def step4(i):
            head.verify_greedy(hp4[i % 64], drafts[i % 64], result=res4, stream=stream)

        n4 = max(100, args.steps // 2)
        r_s = time_loop(torch, n4, 20, step4)
        k4 = r_s / n4
        results[4] = {"rows_per_s": 5 * n4 / r_s, "ms_per_step": k4 * 1e3,
                      "kernel_us_mean": k4 * 1e6, "hbm_frac": algorithmic_bytes(5) / k4 / PEAK_HBM}
        # the accepted counts of the 64 verify cases the steps cycle through (device results)
        acc = []
        for c in range(64):
            step4(c)
            acc.append(int(twd.decode_verify(res4)["num_accepted"]))
        results[4]["mean_accepted"] = float(np.mean(acc))
        results[4]["accepted_histogram"] = [acc.count(a) for a in range(5)]
        results[4]["drafts"] = "target argmax with p=0.6 per position, else a random id (64 cases)"

        # the same 5 rows verified with draft logits (rejection sampling, speculator.cpp:71-122):
        # the head's logits plus 4 synthetic draft rows, T=0.8, k=40, p=0.9
        lg4 = torch.empty(5, V, dtype=torch.float32, device=dev)
        head.logits(hp4[0], out=lg4, stream=stream)
        drng = np.random.default_rng(44)
        drows = [(0.8 * lg4[i] + torch.from_numpy(
            (drng.standard_normal(V) * 1.5).astype(np.float32)).to(dev)).contiguous()
            for i in range(4)]
        sel4 = twd.Selector(V, 5)
        p4 = twd.RowParams(0.8, 0.9, 40, 1.0, 0.0, CAP, 0, 0)

        dviews = [drafts[c] for c in range(64)]

        def step4d(i):
            sel4.verify_draft(lg4, drows, p4, 1000 + i, dviews[i % 64], result=res4,
                              stream=stream)

        nd = max(20, args.steps // 20)
        r_d = time_loop(torch, nd, 5, step4d)
        results[4]["draft_logits_verify_us"] = r_d / nd * 1e6
        # the same verify issued from C++ (tests/cpp/verify_timing, its own process): GPU time
        # back to back and alone, and the host time to issue one call, without the Python wrapper
        results[4]["draft_logits_verify_cpp"] = cpp_verify_timing()

    # ---- config 5: M=64 rows, each with own T/k/p, rp 1.1 over its own 2048-id history ---------
    if 5 in cfgs:
        log("config 5: M=64 sampled, MFMA path")
        hp5 = hidden_pool(torch, dev, 8, 64, 5)
        rng = np.random.default_rng(55)
        hist5 = torch.from_numpy(rng.integers(0, V, 64 * 2048, dtype=np.int64).astype(np.int32)).to(dev)
        prm5 = [twd.RowParams(float(rng.uniform(0.5, 1.2)), float(rng.uniform(0.8, 0.98)),
                              int(rng.integers(20, 101)), 1.1,
                              twd.uniform_from_seed(twd.splitmix64(m)), CAP, 2048 * m, 2048)
                for m in range(64)]
        lg5 = torch.empty(64, V, dtype=torch.float32, device=dev)
        t5 = torch.empty(64, dtype=torch.int32, device=dev)
        work[5] = (hp5[0].cpu().numpy().view(np.uint16), hist5.cpu().numpy().view(np.uint32),
                   [(p.temperature, p.top_p, p.top_k, p.uniform) for p in prm5])

        def step5(i):
            head.sample(hp5[i % 8], prm5, history=hist5, logits=lg5, tokens=t5, stream=stream)

        n5 = max(50, args.steps // 8)
        r_s = time_loop(torch, n5, 10, step5)

        def head5(i):
            head.logits(hp5[i % 8], out=lg5, stream=stream)

        kh = time_loop(torch, n5, 5, head5) / n5
        b5 = algorithmic_bytes(64, 2048) + 64 * V * 4  # the fp32 logits are written
        results[5] = {"rows_per_s": 64 * n5 / r_s, "ms_per_step": r_s * 1e3 / n5,
                      "head_kernel_us_mean": kh * 1e6,
                      "hbm_frac_full_step": b5 / (r_s / n5) / PEAK_HBM,
                      "head_hbm_frac": (HEAD_BYTES + 64 * D * 2 + 64 * V * 4) / kh / PEAK_HBM,
                      "head_mfma_frac": 2.0 * 64 * V * D / kh / PEAK_BF16}

    # socket power and clocks while config 2 (and the config-5 step) run back to back: both
    # reach the part's socket power limit, and the clocks they run at are reported beside them
    power = {}
    if not args.no_power:
        power["config2"] = power_during(torch, 3.0, step2)
        if 5 in cfgs:
            power["config5"] = power_during(torch, 3.0, step5)
    log(f"power: {power}")

    # the practical ceiling: a pure-read probe over the same 792 MB buffer (no arithmetic), the
    # best of several wave counts (more, shorter stripes read faster: 7.16 TB/s at 65536 waves
    # against 7.10 at 32768 in one sweep)
    best = None
    for waves in (8192, 32768, 65536, 131072):
        gbps, us, nb = twd.probe_read_bandwidth(wsb, waves=waves, launches=50, stream=stream)
        if best is None or gbps > best[0]:
            best = (gbps, us, nb, waves)
    ceiling = {"gbps": best[0], "frac_of_peak": best[0] * 1e9 / PEAK_HBM,
               "kernel_frac_of_ceiling": (bytes2 / step_s) / (best[0] * 1e9),
               "probe": f"{best[3]} waves streaming {best[2] / best[3] / 1024:.0f} KB stripes, "
                        f"16 B nt buffer loads, 8 KB in flight per wave"}
    log(f"read ceiling {best[0]:.0f} GB/s ({ceiling['frac_of_peak'] * 100:.1f}% of peak); "
        f"the head pass reaches {ceiling['kernel_frac_of_ceiling'] * 100:.1f}% of it")

    # the synthetic inputs, pinned by digest (outside every timed region)
    host = wsb.cpu().numpy()
    digests = {"weights_sha256": hashlib.sha256(memoryview(host)).hexdigest(),
               "hidden_sha256": hashlib.sha256(hp.cpu().numpy().tobytes()).hexdigest()}
    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline: every config's CPU path, config 2 on {args.cpu_rows} full rows")
        work[2] = hp[: args.cpu_rows].cpu().numpy().view(np.uint16).reshape(-1, D)
        cpu = cpu_baseline(host, work, args.cpu_rows)

    achieved = bytes2 / step_s
    traffic, traffic_src = measured_traffic()
    line = {
        "metric": "LM-head+sample rows/s at d=5376,V=262144 INT4; % HBM roofline",
        "value": results[2]["rows_per_s"],
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": results[2]["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 2: INT4 g64 LM head M=1, V=262144, d=5376, bf16 h "
                               "~N(0,1), fused softcap 30 + greedy argmax",
                   "vocab": V, "d_model": D, "group": G, "rows_per_step": 1,
                   "weights": "q~U{0..15}, s~U(1e-3,1e-2) bf16, b=-8s (twd_generate_head seed "
                              f"{SEED})",
                   "hidden": "64 bf16 rows ~N(0,1), numpy default_rng(2), cycled over the steps",
                   **digests},
        "roofline": {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": achieved / PEAK_HBM, "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "head_small_kernel<4,4,2,8,1> (M=1 greedy, single launch)",
                     "bytes_per_launch": bytes2,
                     "read_ceiling": ceiling},
        "cpu_baseline": cpu,
        "power": power,
        "configs": {str(k): results[k] for k in sorted(results)},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
