"""Writes tests/golden/*.json from the REFERENCE's own sampling.cpp and speculator.cpp.

The reference sources are compiled by oracle/Makefile (target `ref`) into oracle/_ref/libref.so
in this container; this script calls that build and commits only small fixtures: parameters,
generator seeds, SHA-256 digests of the large input rows, and the reference's outputs.

Input rows are regenerated at test time by oracle/gen_std.cpp (std::mt19937 through
std::normal_distribution<float>, the generator the reference's own tests use) and by the
counter formulas documented in oracle/oracle.h, so the fixtures stay a few KB.

Run:  make -C oracle all ref && python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

V_FULL = 262144


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def f32_hex(a) -> list[str]:
    return [f"{int(x):08x}" for x in np.asarray(a, np.float32).view(np.uint32)]


def draft_case_rows(seed: int, vocab: int, nrows: int) -> list:
    """Target rows of a verify_draft case: softcap(30) of N(0, 4^2) rows from std::mt19937."""
    return [O.softcap(O.gen_mt19937_normal(seed + j, 0.0, 4.0, vocab), 30.0) for j in range(nrows)]


def draft_case_drafts(seed: int, vocab: int, rows: list, alpha: float, sd: float, mask) -> list:
    """Draft rows: alpha * target + N(0, sd^2) noise in float32 (None where mask is False); a
    position past the target rows mixes with row 0."""
    out = []
    for i, m in enumerate(mask):
        if not m:
            out.append(None)
            continue
        base = rows[min(i, len(rows) - 1)]
        noise = O.gen_mt19937_normal(seed + 1000 + i, 0.0, sd, vocab)
        out.append((np.float32(alpha) * base + noise).astype(np.float32))
    return out


# A valid header in the shape of tests/test_format.cpp:33-66 (4 layers of 131072 bytes after a
# 65536-byte embedding at 4096), and the mutations its tests and validate_header's branches reject.
HEADER_BASE = dict(magic=0x4734444E, version=3, quant_type=1, num_layers=4, d_model=256, d_ff=512,
                   num_q_heads=4, num_kv_heads=2, head_dim=64, vocab_size=1024,
                   sliding_window=512, quant_group_size=64, scale_dtype=1, tied_embeddings=1,
                   global_layer_mask=(1 << 1) | (1 << 3), final_logit_softcapping=30.0,
                   embed_offset=4096, embed_size=65536, lm_head_offset=4096, lm_head_size=65536,
                   layer_offsets=[4096 + 65536 + 131072 * i for i in range(4)],
                   layer_sizes=[131072] * 4)
HEADER_END = 4096 + 65536 + 4 * 131072


def header_cases():
    lo = HEADER_BASE["layer_offsets"]
    ls = HEADER_BASE["layer_sizes"]
    return [
        ("valid", {}, HEADER_END),
        ("valid_no_file_size", {}, 0),
        ("bad_magic", {"magic": 0xDEADBEEF}, HEADER_END),
        ("version_2", {"version": 2}, HEADER_END),
        ("no_layers", {"num_layers": 0}, HEADER_END),
        ("61_layers", {"num_layers": 61}, HEADER_END),
        ("zero_d_model", {"d_model": 0}, HEADER_END),
        ("zero_vocab", {"vocab_size": 0}, HEADER_END),
        ("embed_unaligned", {"embed_offset": 4097}, HEADER_END),
        ("lm_head_unaligned", {"lm_head_offset": 8192 + 16}, HEADER_END),
        ("layer0_unaligned", {"layer_offsets": [4097] + lo[1:]}, HEADER_END),
        ("layer2_size_0", {"layer_sizes": ls[:2] + [0] + ls[3:]}, HEADER_END),
        ("past_file_end", {}, HEADER_END - 100),
        ("overflow", {"layer_offsets": lo[:3] + [2**64 - 4096], "layer_sizes": ls[:3] + [8192]},
         0),
    ]


def main() -> None:
    R = O.Reference()
    out: dict = {"source": "reference src/sampling.cpp + src/speculator.cpp via oracle/_ref"}

    # ---- seeding (sampling.cpp:56-72) --------------------------------------------------------
    xs = [0, 1, 2, 3, 0x9E3779B97F4A7C15, 0xFFFFFFFFFFFFFFFF, 12345, 1 << 63]
    out["splitmix64"] = [[str(x), str(R.splitmix64(x))] for x in xs]
    seeds = []
    for has_seed, seed in [(True, 12345), (True, 0), (True, 20260721), (False, 0), (False, 99)]:
        for pos in [0, 1, 2, 7, 100, 4095, 65535, -1]:
            seeds.append([int(has_seed), str(seed), pos, str(R.seed_for(has_seed, seed, pos))])
    out["seed_for"] = seeds

    # ---- validate_sampling (sampling.cpp:32-54) ------------------------------------------------
    grid = []
    for t in [0.0, 0.2, -0.1, float("inf"), float("nan"), 1.5]:
        for p in [1.0, 0.95, 0.0, 1.5, float("nan")]:
            for k in [0, 1, 64, 256, 257, -1]:
                for rp in [1.0, 1.1, 0.0, -1.0]:
                    grid.append([t, p, k, rp, R.validate_sampling(t, p, k, rp)])
    out["validate_sampling"] = [[repr(a), repr(b), c, repr(d), e] for a, b, c, d, e in grid]

    # ---- repetition penalty (sampling.cpp:74-90) ----------------------------------------------
    pen = []
    rng = np.random.default_rng(7)
    for case, (vocab, nhist, rp, cap, dup) in enumerate([
        (64, 40, 1.1, 30.0, True), (64, 200, 2.0, 30.0, True), (64, 50, 0.5, 30.0, True),
        (64, 50, 0.7, 0.0, True), (4096, 4096, 1.1, 30.0, False), (4096, 300, 1.3, 30.0, True),
    ]):
        logits = O.gen_mt19937_normal(1000 + case, 0.0, 12.0, vocab)
        logits = O.softcap(logits, 30.0)
        if dup:
            hist = rng.integers(0, vocab + 8, size=nhist, dtype=np.uint32)  # some out of range
        else:
            hist = rng.integers(0, vocab, size=nhist, dtype=np.uint32)
        got = R.apply_repetition_penalty(logits, hist, rp, cap)
        pen.append({
            "gen": ["mt19937_normal", 1000 + case, 0.0, 12.0, vocab, "softcap", 30.0],
            "history": [int(x) for x in hist], "penalty": rp, "softcap": cap,
            "in_sha256": sha(logits), "out_sha256": sha(got),
            "out_f32_hex": f32_hex(got) if vocab <= 64 else None,
        })
    out["penalty"] = pen

    # ---- sample_token, the reference test's own rows ---------------------------------------------
    # tests/test_sampling.cpp:238-265: mt19937(20260723), N(0, 6^2), V=262144, 5 configs x 40.
    lg = O.gen_mt19937_normal(20260723, 0.0, 6.0, V_FULL)
    cfgs = [(0.2, 0.95, 64, 1), (1.0, 0.90, 8, 2), (0.7, 1.00, 256, 3), (0.5, 1.00, 0, 4),
            (1.5, 0.99, 1, 5)]
    rows = []
    for t, p, k, s in cfgs:
        ids = []
        for i in range(40):
            sd = R.seed_for(True, s, i)
            ids.append([str(sd), R.sample_token(lg, t, p, k, sd)])
        rows.append({"t": t, "p": p, "k": k, "seed": s, "draws": ids})
    out["shortlist_vs_full_sort"] = {"gen": ["mt19937_normal", 20260723, 0.0, 6.0, V_FULL],
                                     "logits_sha256": sha(lg), "configs": rows}

    # ---- N(0, 4^2) row, softcap 30, greedy then T=.8/k=64/p=.95 -----------
    z = O.gen_mt19937_normal(1, 0.0, 4.0, V_FULL)
    zc = O.softcap(z, 30.0)
    c1 = {"gen": ["mt19937_normal", 1, 0.0, 4.0, V_FULL, "softcap", 30.0],
          "logits_sha256": sha(zc),
          "greedy": R.sample_token(zc, 0.0, 1.0, 0, 1),
          "sampled": []}
    for i in range(64):
        sd = R.seed_for(True, 20260801, i)
        c1["sampled"].append([str(sd), R.sample_token(zc, 0.8, 0.95, 64, sd)])
    out["config1"] = c1

    # ---- BASELINE config 3/5 style rows: softcapped, penalised, sampled ---------------------------
    c3 = []
    for case in range(6):
        zz = O.softcap(O.gen_mt19937_normal(300 + case, 0.0, 4.0, V_FULL), 30.0)
        hist = np.random.default_rng(300 + case).integers(0, V_FULL, size=4096, dtype=np.uint32)
        rp, t, p, k = [(1.1, 0.7, 0.9, 40), (1.1, 0.8, 0.95, 64), (1.3, 1.2, 0.98, 100),
                       (1.1, 0.5, 0.8, 20), (0.9, 0.7, 0.9, 40), (1.1, 0.0, 1.0, 0)][case]
        pz = R.apply_repetition_penalty(zz, hist, rp, 30.0)
        draws = []
        for i in range(16):
            sd = R.seed_for(True, 77 + case, i)
            draws.append([str(sd), R.sample_token(pz, t, p, k, sd)])
        c3.append({"gen": ["mt19937_normal", 300 + case, 0.0, 4.0, V_FULL, "softcap", 30.0],
                   "history_gen": ["numpy_default_rng_integers", 300 + case, 4096],
                   "history_sha256": sha(hist),
                   "rp": rp, "t": t, "p": p, "k": k, "penalised_sha256": sha(pz),
                   "draws": draws})
    out["penalised_sampling"] = c3

    # ---- greedy speculative verify (speculator.cpp:34-153) ------------------------------------
    ver = []
    vrng = np.random.default_rng(44)
    vocab = 4096
    for case in range(24):
        nrows = int(vrng.integers(1, 9))
        ndraft = int(vrng.integers(0, 9))
        rws = [O.softcap(O.gen_mt19937_normal(5000 + 16 * case + j, 0.0, 4.0, vocab), 30.0)
               for j in range(nrows)]
        arg = [int(np.argmax(r)) for r in rws]
        drafts = []
        for i in range(ndraft):
            if i < nrows and vrng.random() < 0.6:
                drafts.append(arg[i])
            else:
                drafts.append(int(vrng.integers(0, vocab)))
        t, p, k = [(0.0, 1.0, 0), (0.7, 0.9, 40)][case % 2]
        base = int(vrng.integers(0, 2**63))
        res = R.verify(drafts, rws, t, p, k, 1.0, base)
        ver.append({"rows_gen": ["mt19937_normal", 5000 + 16 * case, 0.0, 4.0, vocab, "softcap",
                                 30.0, nrows],
                    "drafts": drafts, "t": t, "p": p, "k": k, "base_seed": str(base),
                    "result": res})
    out["verify"] = ver

    # ---- verify with draft logits: the rejection branch (speculator.cpp:71-122) ---------------
    vd = []
    drng = np.random.default_rng(77)
    for case in range(40):
        vocab = V_FULL if case % 10 == 9 else 4096
        nrows = int(drng.integers(1, 7))
        ndraft = int(drng.integers(1, 7))
        seed_t = 9000 + 32 * case
        rws = draft_case_rows(seed_t, vocab, nrows)
        alpha = float(drng.choice([0.0, 0.5, 0.9, 1.0]))
        dsd = float(drng.choice([0.5, 2.0, 4.0]))
        mask = [bool(drng.random() < 0.85) for _ in range(ndraft)]
        drs = draft_case_drafts(seed_t, vocab, rws, alpha, dsd, mask)
        arg = [int(np.argmax(r)) for r in rws]
        drafts = [arg[i] if i < nrows and drng.random() < 0.5 else int(drng.integers(0, vocab))
                  for i in range(ndraft)]
        t, rp = [(0.8, 1.0), (1.0, 1.0), (0.5, 1.0), (1.3, 1.0), (0.0, 1.1)][case % 5]
        p, k = [(1.0, 0), (0.9, 40)][(case // 5) % 2]
        base = int(drng.integers(0, 2**63))
        res = R.verify_draft(drafts, rws, drs, t, p, k, rp, base)
        vd.append({"vocab": vocab, "rows_seed": seed_t, "nrows": nrows, "alpha": alpha,
                   "draft_sd": dsd, "mask": mask, "drafts": drafts, "t": t, "p": p, "k": k,
                   "rp": rp, "base_seed": str(base), "result": res})
    # A draft row equal to its target row except for one NaN: compute_softmax's sum is then NaN,
    # so q is left unnormalised (inv = 1), q >= p everywhere, p/q = 1/sum_p, and a rejection
    # finds (p - q)+ summing to 0 -- the fallback to sample_token (:113-115).
    for case in range(6):
        vocab = 4096
        seed_t = 12000 + 32 * case
        rws = draft_case_rows(seed_t, vocab, 3)
        drs = draft_case_drafts(seed_t, vocab, rws, 1.0, 0.0, [True, True])
        nan_at = [int(drng.integers(0, vocab)) for _ in drs]
        for r, j in zip(drs, nan_at):
            r[j] = np.nan
        drafts = [int(np.argsort(rws[i])[-2]) for i in range(2)]  # not the argmax, not NaN
        t, p, k = [(0.8, 1.0, 0), (1.0, 0.9, 40), (0.6, 1.0, 0)][case % 3]
        base = int(drng.integers(0, 2**63))
        res = R.verify_draft(drafts, rws, drs, t, p, k, 1.0, base)
        vd.append({"vocab": vocab, "rows_seed": seed_t, "nrows": 3, "alpha": 1.0,
                   "draft_sd": 0.0, "mask": [True, True], "nan_at": nan_at, "drafts": drafts,
                   "t": t, "p": p, "k": k, "rp": 1.0, "base_seed": str(base), "result": res})
    out["verify_draft"] = vd

    # ---- container header validation (src/format.cpp:6-65) -------------------------------------
    sys.path.insert(0, os.path.join(HERE, ".."))
    from helpers import container_header
    hv = []
    for name, over, fsize in header_cases():
        hdr = container_header(**{**HEADER_BASE, **over})
        hv.append({"case": name, "fields": over, "file_size": fsize,
                   "error": R.validate_header(hdr, fsize)})
    out["container_headers"] = hv

    path = os.path.join(HERE, "sampling_golden.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0, separators=(",", ":"))
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
