"""ctypes binding of the CPU oracle (liboracle.so) and of the reference build (_ref/libref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg as the checker. The product library never loads anything from this directory.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

OR_OK, OR_ERR_EMPTY_VOCAB, OR_ERR_DEGENERATE, OR_ERR_INVALID = 0, 1, 2, 3

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")


class SampleDiag(C.Structure):
    _fields_ = [
        ("max_logit", C.c_double),
        ("total", C.c_double),
        ("want", C.c_uint32),
        ("cut", C.c_uint32),
        ("cut_margin", C.c_double),
        ("draw_r", C.c_double),
        ("draw_margin", C.c_double),
        ("u", C.c_float),
    ]


OR_MAX_DRAFTS = 1024


class VerifyResult(C.Structure):
    _fields_ = [
        ("tokens", C.c_uint32 * (OR_MAX_DRAFTS + 1)),
        ("n_tokens", C.c_uint32),
        ("num_accepted", C.c_uint32),
        ("total_drafted", C.c_uint32),
        ("bonus_token_sampled", C.c_int),
        ("bonus_token", C.c_uint32),
        ("acceptance_rate", C.c_double),
    ]


class RejectDiag(C.Structure):
    _fields_ = [
        ("r", C.c_float),
        ("u1", C.c_float),
        ("u2", C.c_float),
        ("sum_p", C.c_float),
        ("sum_q", C.c_float),
        ("sum_diff", C.c_float),
        ("r_val", C.c_float),
        ("corr", C.c_uint32),
        ("accepted", C.c_int),
    ]


def build(ref: bool = True) -> None:
    """Compiles liboracle.so, and _ref/libref.so when the reference checkout is present."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if ref and os.path.isdir(os.environ.get("TWD_REFERENCE", "/root/reference")):
        subprocess.run(["make", "-s", "-C", HERE, "ref",
                        "REF=" + os.environ.get("TWD_REFERENCE", "/root/reference")], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build(ref=False)
    lib = C.CDLL(LIB_PATH)
    lib.or_splitmix64.restype = C.c_uint64
    lib.or_expf.argtypes = [_f32p, _f32p, C.c_size_t]
    lib.or_expf.restype = None
    lib.or_exp.argtypes = [_f64p, _f64p, C.c_size_t]
    lib.or_exp.restype = None
    lib.or_splitmix64.argtypes = [C.c_uint64]
    lib.or_seed_for.restype = C.c_uint64
    lib.or_seed_for.argtypes = [C.c_int, C.c_uint64, C.c_int]
    lib.or_uniform_from_seed.restype = C.c_float
    lib.or_uniform_from_seed.argtypes = [C.c_uint64]
    lib.or_validate_sampling.restype = C.c_int
    lib.or_validate_sampling.argtypes = [C.c_float, C.c_float, C.c_int, C.c_float]
    lib.or_apply_repetition_penalty.restype = None
    lib.or_apply_repetition_penalty.argtypes = [_f32p, C.c_uint32, _u32p, C.c_size_t,
                                                C.c_float, C.c_float]
    lib.or_sample_token.restype = C.c_int
    lib.or_sample_token.argtypes = [_f32p, C.c_uint32, C.c_float, C.c_float, C.c_int,
                                    C.c_uint64, C.POINTER(C.c_uint32), C.POINTER(SampleDiag)]
    lib.or_sample_token_u.restype = C.c_int
    lib.or_sample_token_u.argtypes = [_f32p, C.c_uint32, C.c_float, C.c_float, C.c_int,
                                      C.c_float, C.POINTER(C.c_uint32), C.POINTER(SampleDiag)]
    lib.or_argmax.restype = C.c_uint32
    lib.or_argmax.argtypes = [_f32p, C.c_uint32]
    lib.or_shortlist.restype = C.c_uint32
    lib.or_shortlist.argtypes = [_f32p, C.c_uint32, C.c_uint32, _u32p]
    lib.or_verify.restype = C.c_int
    lib.or_verify.argtypes = [_u32p, C.c_size_t, C.POINTER(C.c_void_p), C.c_size_t, C.c_uint32,
                              C.c_float, C.c_float, C.c_int, C.c_uint64, C.POINTER(VerifyResult)]
    lib.or_lm_head.restype = None
    lib.or_lm_head.argtypes = [_u32p, _u16p, _u16p, _f32p, C.c_uint32, C.c_uint32, C.c_uint32,
                               C.c_uint32, C.c_float, _f32p]
    lib.or_lm_head_f64.restype = None
    lib.or_lm_head_f64.argtypes = [_u32p, _u16p, _u16p, _f32p, C.c_uint32, C.c_uint32,
                                   C.c_uint32, C.c_uint32, _f64p]
    lib.or_rmsnorm.restype = None
    lib.or_rmsnorm.argtypes = [_f32p, _u16p, C.c_uint32, C.c_float, _f32p]
    lib.or_softcap.restype = None
    lib.or_softcap.argtypes = [_f32p, C.c_size_t, C.c_float]
    lib.or_gen_lm_head.restype = None
    lib.or_gen_lm_head.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                   _u32p, _u16p, _u16p]
    lib.or_gen_mt19937_normal.restype = None
    lib.or_gen_mt19937_normal.argtypes = [C.c_uint32, C.c_float, C.c_float, C.c_size_t, _f32p]
    lib.or_mt64_seed.restype = None
    lib.or_mt64_seed.argtypes = [C.c_void_p, C.c_uint64]
    lib.or_mt64_next.restype = C.c_uint64
    lib.or_mt64_next.argtypes = [C.c_void_p]
    lib.or_canonical_float.restype = C.c_float
    lib.or_canonical_float.argtypes = [C.c_uint64]
    lib.or_rejection_uniforms.restype = None
    lib.or_rejection_uniforms.argtypes = [C.c_uint64, C.POINTER(C.c_float), C.POINTER(C.c_float)]
    lib.or_softmax.restype = None
    lib.or_softmax.argtypes = [_f32p, C.c_uint32, C.c_float]
    lib.or_verify_draft.restype = C.c_int
    lib.or_verify_draft.argtypes = [_u32p, C.c_size_t, C.POINTER(C.c_void_p), C.c_size_t,
                                    C.POINTER(C.c_void_p), C.c_size_t, C.c_uint32, C.c_float,
                                    C.c_float, C.c_int, C.c_float, C.c_uint64,
                                    C.POINTER(VerifyResult), C.POINTER(RejectDiag)]
    lib.or_std_rejection_uniforms.restype = None
    lib.or_std_rejection_uniforms.argtypes = [C.POINTER(C.c_uint64), C.c_size_t, _f32p]
    lib.or_std_mt64_10000th.restype = C.c_uint64
    lib.or_std_mt64_10000th.argtypes = []
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


# ---- sampling.cpp restatement ---------------------------------------------------------------

def splitmix64(x: int) -> int:
    return int(lib().or_splitmix64(x & 0xFFFFFFFFFFFFFFFF))


def seed_for(has_seed: bool, seed: int, position: int) -> int:
    return int(lib().or_seed_for(1 if has_seed else 0, seed & 0xFFFFFFFFFFFFFFFF, position))


def uniform_from_seed(seed: int) -> float:
    return float(lib().or_uniform_from_seed(seed & 0xFFFFFFFFFFFFFFFF))


def validate_sampling(t: float, p: float, k: int, rp: float) -> bool:
    """True when the reference's validate_sampling accepts the parameters."""
    return lib().or_validate_sampling(t, p, k, rp) == OR_OK


def apply_repetition_penalty(logits, history, penalty: float, softcap: float) -> np.ndarray:
    out = _f32(logits).copy()
    h = _u32(history) if len(history) else np.zeros(1, np.uint32)
    lib().or_apply_repetition_penalty(out, out.size, h, len(history), penalty, softcap)
    return out


def sample_token(logits, t: float, p: float, k: int, seed: int = 0, u: float | None = None,
                 diag: bool = False):
    """sample_token of sampling.cpp:92-169. With `u` given, the draw uses it directly."""
    lg = _f32(logits)
    out = C.c_uint32(0)
    dg = SampleDiag()
    if u is None:
        rc = lib().or_sample_token(lg, lg.size, t, p, k, seed & 0xFFFFFFFFFFFFFFFF, C.byref(out),
                                   C.byref(dg))
    else:
        rc = lib().or_sample_token_u(lg, lg.size, t, p, k, u, C.byref(out), C.byref(dg))
    if rc != OR_OK:
        raise RuntimeError(f"oracle sample_token failed with code {rc}")
    if diag:
        return int(out.value), {f: getattr(dg, f) for f, _ in SampleDiag._fields_}
    return int(out.value)


def argmax(logits) -> int:
    lg = _f32(logits)
    return int(lib().or_argmax(lg, lg.size))


def shortlist(logits, want: int) -> np.ndarray:
    lg = _f32(logits)
    idx = np.zeros(max(1, want), np.uint32)
    n = lib().or_shortlist(lg, lg.size, want, idx)
    return idx[:n].copy()


def verify(drafts, rows, t=0.0, p=1.0, k=0, base_seed=0) -> dict:
    d = _u32(drafts) if len(drafts) else np.zeros(1, np.uint32)
    rows = [_f32(r) for r in rows]
    vocab = rows[0].size if rows else 0
    ptrs = (C.c_void_p * max(1, len(rows)))(*[r.ctypes.data for r in rows])
    res = VerifyResult()
    rc = lib().or_verify(d, len(drafts), ptrs, len(rows), vocab, t, p, k,
                         base_seed & 0xFFFFFFFFFFFFFFFF, C.byref(res))
    if rc != OR_OK:
        raise RuntimeError(f"oracle verify failed with code {rc}")
    return {
        "tokens": [int(res.tokens[i]) for i in range(res.n_tokens)],
        "num_accepted": int(res.num_accepted),
        "total_drafted": int(res.total_drafted),
        "bonus_token_sampled": bool(res.bonus_token_sampled),
        "bonus_token": int(res.bonus_token),
        "acceptance_rate": float(res.acceptance_rate),
    }


# ---- rejection-sampling verify (speculator.cpp:14-30, :71-122) -------------------------------

class MT64(C.Structure):
    _fields_ = [("mt", C.c_uint64 * 312), ("idx", C.c_int)]


def mt64_outputs(seed: int, n: int) -> list:
    g = MT64()
    lib().or_mt64_seed(C.byref(g), seed & 0xFFFFFFFFFFFFFFFF)
    return [int(lib().or_mt64_next(C.byref(g))) for _ in range(n)]


def canonical_float(x: int) -> float:
    return float(lib().or_canonical_float(x & 0xFFFFFFFFFFFFFFFF))


def rejection_uniforms(step_seed: int):
    u1, u2 = C.c_float(), C.c_float()
    lib().or_rejection_uniforms(step_seed & 0xFFFFFFFFFFFFFFFF, C.byref(u1), C.byref(u2))
    return float(u1.value), float(u2.value)


def std_rejection_uniforms(seeds) -> np.ndarray:
    """libstdc++'s own two draws per seed (gen_std.cpp): [n, 2] float32."""
    sd = (C.c_uint64 * len(seeds))(*[int(x) & 0xFFFFFFFFFFFFFFFF for x in seeds])
    out = np.zeros(2 * len(seeds), np.float32)
    lib().or_std_rejection_uniforms(sd, len(seeds), out)
    return out.reshape(-1, 2)


def std_mt64_10000th() -> int:
    return int(lib().or_std_mt64_10000th())


def expf(x) -> np.ndarray:
    """The host C library's expf, as compute_softmax's std::exp(float) (speculator.cpp:23)."""
    xs = _f32(x).copy()
    out = np.empty_like(xs)
    lib().or_expf(xs, out, xs.size)
    return out


def exp(x) -> np.ndarray:
    """The host C library's exp(double), elementwise (std::exp(double) of sampling.cpp)."""
    xs = np.ascontiguousarray(x, np.float64)
    out = np.empty_like(xs)
    lib().or_exp(xs, out, xs.size)
    return out


def softmax(logits, temp: float) -> np.ndarray:
    out = _f32(logits).copy()
    lib().or_softmax(out, out.size, temp)
    return out


def verify_draft(drafts, rows, draft_rows, t=0.8, p=1.0, k=0, rp=1.0, base_seed=0) -> dict:
    """evaluate_verification with draft logits; draft_rows entries may be None."""
    d = _u32(drafts) if len(drafts) else np.zeros(1, np.uint32)
    rows = [_f32(r) for r in rows]
    drs = [None if r is None else _f32(r) for r in draft_rows]
    vocab = rows[0].size if rows else 0
    ptrs = (C.c_void_p * max(1, len(rows)))(*[r.ctypes.data for r in rows])
    dptrs = (C.c_void_p * max(1, len(drs)))(*[None if r is None else r.ctypes.data for r in drs])
    res = VerifyResult()
    diag = (RejectDiag * max(1, len(drafts)))()
    for i in range(len(diag)):
        diag[i].r = -1.0
    rc = lib().or_verify_draft(d, len(drafts), ptrs, len(rows), dptrs, len(drs), vocab, t, p, k,
                               rp, base_seed & 0xFFFFFFFFFFFFFFFF, C.byref(res), diag)
    if rc != OR_OK:
        raise RuntimeError(f"oracle verify failed with code {rc}")
    return {
        "tokens": [int(res.tokens[i]) for i in range(res.n_tokens)],
        "num_accepted": int(res.num_accepted),
        "total_drafted": int(res.total_drafted),
        "bonus_token_sampled": bool(res.bonus_token_sampled),
        "bonus_token": int(res.bonus_token),
        "acceptance_rate": float(res.acceptance_rate),
        "diag": [None if diag[i].r == -1.0 else {f: getattr(diag[i], f) for f, _ in RejectDiag._fields_}
                 for i in range(len(drafts))],
    }


# ---- LM head (cpu_reference.cpp:643-665) -----------------------------------------------------

def rmsnorm(x, weight_bf16, eps: float = 1e-6) -> np.ndarray:
    """The final RMSNorm of cpu_reference.cpp:141-150 on one fp32 row."""
    xs = _f32(x)
    w = np.ascontiguousarray(weight_bf16, dtype=np.uint16)
    out = np.zeros_like(xs)
    lib().or_rmsnorm(xs, w, xs.size, eps, out)
    return out


def lm_head(W, S, B, hidden, d: int, group: int = 64, row0: int = 0, nrows: int | None = None,
            softcap: float = 0.0) -> np.ndarray:
    nrows = W.shape[0] if nrows is None else nrows
    out = np.zeros(nrows, np.float32)
    lib().or_lm_head(_u32(W).reshape(-1), np.ascontiguousarray(S, np.uint16).reshape(-1),
                     np.ascontiguousarray(B, np.uint16).reshape(-1), _f32(hidden), d, group,
                     row0, nrows, softcap, out)
    return out


def lm_head_f64(W, S, B, hidden, d: int, group: int = 64, row0: int = 0,
                nrows: int | None = None) -> np.ndarray:
    nrows = W.shape[0] if nrows is None else nrows
    out = np.zeros(nrows, np.float64)
    lib().or_lm_head_f64(_u32(W).reshape(-1), np.ascontiguousarray(S, np.uint16).reshape(-1),
                         np.ascontiguousarray(B, np.uint16).reshape(-1), _f32(hidden), d, group,
                         row0, nrows, out)
    return out


def softcap(z, cap: float) -> np.ndarray:
    out = _f32(z).copy()
    lib().or_softcap(out, out.size, cap)
    return out


def gen_lm_head(seed: int, V: int, d: int, group: int = 64, row0: int = 0):
    """Synthetic head rows [row0, row0+V) in the reference layout: (W [V, d/8] u32,
    S [V, d/group] bf16 bits, B [V, d/group] bf16 bits)."""
    W = np.zeros(V * (d // 8), np.uint32)
    S = np.zeros(V * (d // group), np.uint16)
    B = np.zeros(V * (d // group), np.uint16)
    lib().or_gen_lm_head(seed & 0xFFFFFFFFFFFFFFFF, d, group, row0, V, W, S, B)
    return W.reshape(V, d // 8), S.reshape(V, d // group), B.reshape(V, d // group)


def gen_mt19937_normal(seed: int, mean: float, sd: float, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().or_gen_mt19937_normal(seed, mean, sd, n, out)
    return out


# ---- the reference build ----------------------------------------------------------------------

class Reference:
    """The reference's own sampling.cpp + speculator.cpp behind oracle/ref_shim.cpp."""

    def __init__(self, path: str = REF_PATH):
        self.lib = C.CDLL(path)
        L = self.lib
        L.ref_splitmix64.restype = C.c_uint64
        L.ref_splitmix64.argtypes = [C.c_uint64]
        L.ref_seed_for.restype = C.c_uint64
        L.ref_seed_for.argtypes = [C.c_float, C.c_float, C.c_int, C.c_float, C.c_int,
                                   C.c_uint64, C.c_int]
        L.ref_validate_sampling.restype = C.c_int
        L.ref_validate_sampling.argtypes = [C.c_float, C.c_float, C.c_int, C.c_float,
                                            C.c_char_p, C.c_size_t]
        L.ref_apply_repetition_penalty.restype = None
        L.ref_apply_repetition_penalty.argtypes = [_f32p, C.c_uint32, _u32p, C.c_size_t,
                                                   C.c_float, C.c_float]
        L.ref_sample_token.restype = C.c_int
        L.ref_sample_token.argtypes = [_f32p, C.c_uint32, C.c_float, C.c_float, C.c_int,
                                       C.c_float, C.c_uint64, C.POINTER(C.c_uint32),
                                       C.c_char_p, C.c_size_t]
        L.ref_evaluate_verification_draft.restype = C.c_int
        L.ref_evaluate_verification_draft.argtypes = [_u32p, C.c_size_t, C.POINTER(C.c_void_p),
                                                      C.c_size_t, C.POINTER(C.c_void_p),
                                                      C.c_size_t, C.c_uint32, C.c_float,
                                                      C.c_float, C.c_int, C.c_float, C.c_uint64,
                                                      _u32p, _u32p, C.POINTER(C.c_double),
                                                      C.c_char_p, C.c_size_t]
        L.ref_validate_header.restype = C.c_int
        L.ref_validate_header.argtypes = [C.c_char_p, C.c_uint64, C.c_char_p, C.c_size_t]
        L.ref_evaluate_verification.restype = C.c_int
        L.ref_evaluate_verification.argtypes = [_u32p, C.c_size_t, C.POINTER(C.c_void_p),
                                                C.c_size_t, C.c_uint32, C.c_float, C.c_float,
                                                C.c_int, C.c_float, C.c_uint64, _u32p, _u32p,
                                                C.POINTER(C.c_double), C.c_char_p, C.c_size_t]

    @staticmethod
    def available(path: str = REF_PATH) -> bool:
        return os.path.exists(path)

    def splitmix64(self, x):
        return int(self.lib.ref_splitmix64(x & 0xFFFFFFFFFFFFFFFF))

    def seed_for(self, has_seed, seed, pos):
        return int(self.lib.ref_seed_for(0.7, 1.0, 0, 1.0, 1 if has_seed else 0,
                                         seed & 0xFFFFFFFFFFFFFFFF, pos))

    def validate_sampling(self, t, p, k, rp) -> bool:
        buf = C.create_string_buffer(256)
        return self.lib.ref_validate_sampling(t, p, k, rp, buf, 256) == 0

    def apply_repetition_penalty(self, logits, history, penalty, softcap):
        out = _f32(logits).copy()
        h = _u32(history) if len(history) else np.zeros(1, np.uint32)
        self.lib.ref_apply_repetition_penalty(out, out.size, h, len(history), penalty, softcap)
        return out

    def sample_token(self, logits, t, p, k, seed, rp=1.0):
        lg = _f32(logits)
        out = C.c_uint32(0)
        buf = C.create_string_buffer(256)
        rc = self.lib.ref_sample_token(lg, lg.size, t, p, k, rp, seed & 0xFFFFFFFFFFFFFFFF,
                                       C.byref(out), buf, 256)
        if rc != 0:
            raise RuntimeError(buf.value.decode())
        return int(out.value)

    def verify(self, drafts, rows, t=0.0, p=1.0, k=0, rp=1.0, base_seed=0):
        d = _u32(drafts) if len(drafts) else np.zeros(1, np.uint32)
        rows = [_f32(r) for r in rows]
        vocab = rows[0].size if rows else 0
        ptrs = (C.c_void_p * max(1, len(rows)))(*[r.ctypes.data for r in rows])
        toks = np.zeros(len(drafts) + 2, np.uint32)
        info = np.zeros(5, np.uint32)
        rate = C.c_double(0.0)
        buf = C.create_string_buffer(256)
        rc = self.lib.ref_evaluate_verification(d, len(drafts), ptrs, len(rows), vocab, t, p, k,
                                                rp, base_seed & 0xFFFFFFFFFFFFFFFF, toks, info,
                                                C.byref(rate), buf, 256)
        if rc != 0:
            raise RuntimeError(buf.value.decode())
        return {
            "tokens": [int(x) for x in toks[: info[0]]],
            "num_accepted": int(info[1]),
            "total_drafted": int(info[2]),
            "bonus_token_sampled": bool(info[3]),
            "bonus_token": int(info[4]),
            "acceptance_rate": float(rate.value),
        }

    def verify_draft(self, drafts, rows, draft_rows, t=0.8, p=1.0, k=0, rp=1.0, base_seed=0):
        d = _u32(drafts) if len(drafts) else np.zeros(1, np.uint32)
        rows = [_f32(r) for r in rows]
        drs = [None if r is None else _f32(r) for r in draft_rows]
        vocab = rows[0].size if rows else 0
        ptrs = (C.c_void_p * max(1, len(rows)))(*[r.ctypes.data for r in rows])
        dptrs = (C.c_void_p * max(1, len(drs)))(*[None if r is None else r.ctypes.data for r in drs])
        toks = np.zeros(len(drafts) + 2, np.uint32)
        info = np.zeros(5, np.uint32)
        rate = C.c_double(0.0)
        buf = C.create_string_buffer(256)
        rc = self.lib.ref_evaluate_verification_draft(d, len(drafts), ptrs, len(rows), dptrs,
                                                      len(drs), vocab, t, p, k, rp,
                                                      base_seed & 0xFFFFFFFFFFFFFFFF, toks, info,
                                                      C.byref(rate), buf, 256)
        if rc != 0:
            raise RuntimeError(buf.value.decode())
        return {
            "tokens": [int(x) for x in toks[: info[0]]],
            "num_accepted": int(info[1]),
            "total_drafted": int(info[2]),
            "bonus_token_sampled": bool(info[3]),
            "bonus_token": int(info[4]),
            "acceptance_rate": float(rate.value),
        }

    def validate_header(self, header: bytes, file_size: int = 0):
        """None when the reference's validate_header accepts the header, else its message."""
        buf = C.create_string_buffer(512)
        rc = self.lib.ref_validate_header(bytes(header), file_size, buf, 512)
        return None if rc == 0 else buf.value.decode()
