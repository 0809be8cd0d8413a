"""Python binding of libtwd_head.so, mirroring the reference's sampling/speculator interface.

Names, argument meaning and error behaviour follow include/g4dense/sampling.hpp:9-27 and
include/g4dense/speculator.hpp:10-43 of the reference (SamplingParams, validate_sampling,
splitmix64, seed_for, apply_repetition_penalty, sample_token,
SpeculativeCoordinator.evaluate_verification), plus LMHead for the fused INT4 head.

Device memory and streams come from PyTorch (ROCm); every computation runs in the HIP library.
If the library is missing this module raises at import -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
from typing import Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtwd_head.so")

TWD_OK, TWD_E_INVALID, TWD_E_HIP, TWD_E_DEGENERATE, TWD_E_UNSUPPORTED = 0, -1, -2, -3, -4
TOKEN_DEGENERATE = 0xFFFFFFFF
MAX_ROWS = 64
MAX_WANT = 256


class G4DenseFormatError(RuntimeError):
    """The reference's G4DenseFormatError (include/g4dense/format.hpp:249-253)."""


class TwdError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class RowParams(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_p", C.c_float),
        ("top_k", C.c_int32),
        ("repetition_penalty", C.c_float),
        ("uniform", C.c_float),
        ("softcap", C.c_float),
        ("history_offset", C.c_uint32),
        ("history_len", C.c_uint32),
    ]


class VerifyResult(C.Structure):
    _fields_ = [
        ("n_tokens", C.c_uint32),
        ("num_accepted", C.c_uint32),
        ("total_drafted", C.c_uint32),
        ("bonus_token_sampled", C.c_uint32),
        ("bonus_token", C.c_uint32),
        ("tokens", C.c_uint32 * (MAX_ROWS + 1)),
    ]


VERIFY_WORDS = C.sizeof(VerifyResult) // 4


class GenerationParams(C.Structure):
    """twd_generation_params: G4DenseGenerationOptions' sampling fields (c_api.h:24-36)."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_float), ("has_seed", C.c_int32),
                ("seed", C.c_uint64), ("max_tokens", C.c_uint32)]


class GenerationOptions(C.Structure):
    """G4DenseGenerationOptions, layout-identical to the reference's c_api.h:24-36."""
    _fields_ = [("max_tokens", C.c_int), ("temperature", C.c_float), ("top_p", C.c_float),
                ("top_k", C.c_int), ("repetition_penalty", C.c_float), ("has_seed", C.c_int),
                ("seed", C.c_ulonglong), ("system_prompt", C.c_char_p),
                ("stop_strings", C.POINTER(C.c_char_p)), ("stop_count", C.c_int),
                ("tier_id", C.c_int)]


# G4DenseTokenCallback (c_api.h:40): nonzero continues
TokenCallback = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_uint, C.c_char_p)

STOP_NONE, STOP_MAX_TOKENS, STOP_TOKEN, STOP_CALLBACK, STOP_CANCELLED, STOP_DEGENERATE = range(6)


def options_default() -> GenerationOptions:
    """The values g4dense_options_default writes (the reference's c_api.cpp:40-53)."""
    return GenerationOptions(512, 0.2, 0.95, 64, 1.0, 0, 0, None, None, 0, 1)


class ContainerInfo(C.Structure):
    """twd_container_info: the .g4dense header fields of this path (format.hpp:26-110)."""
    _fields_ = [(n, C.c_uint32) for n in ("version", "quant_type", "num_layers", "d_model", "d_ff",
                                           "vocab_size", "quant_group_size", "scale_dtype",
                                           "tied_embeddings")] + [
        ("final_logit_softcapping", C.c_float)] + [
        (n, C.c_uint64) for n in ("embed_offset", "embed_size", "lm_head_offset", "lm_head_size",
                                  "file_size")]

_vp, _u32, _u64, _f32, _i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_int32

_SIGS = {
    "twd_last_error": (C.c_char_p, []),
    "twd_head_create": (C.c_int, [_vp, _u64, _u32, _u32, _u32, _f32, C.POINTER(_vp)]),
    "twd_head_create_device": (C.c_int, [_vp, _u64, _u32, _u32, _u32, _f32, _vp, C.POINTER(_vp)]),
    "twd_head_destroy": (None, [_vp]),
    "twd_head_info": (C.c_int, [_vp, C.POINTER(_u32), C.POINTER(_u32), C.POINTER(_f32),
                                C.POINTER(_u64)]),
    "twd_head_logits": (C.c_int, [_vp, _vp, _u32, _vp, _vp]),
    "twd_head_greedy": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _vp]),
    "twd_head_sample": (C.c_int, [_vp, _vp, _u32, C.POINTER(RowParams), _vp, _vp, _vp, _vp]),
    "twd_head_verify_greedy": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp]),
    "twd_head_logits_rmsnorm": (C.c_int, [_vp, _vp, _vp, _f32, _u32, _vp, _vp]),
    "twd_head_greedy_rmsnorm": (C.c_int, [_vp, _vp, _vp, _f32, _u32, _vp, _vp, _vp]),
    "twd_head_verify_greedy_rmsnorm": (C.c_int, [_vp, _vp, _vp, _f32, _u32, _vp, _u32, _vp, _vp,
                                                 _vp]),
    "twd_head_sample_rmsnorm": (C.c_int, [_vp, _vp, _vp, _f32, _u32, C.POINTER(RowParams), _vp,
                                          _vp, _vp, _vp]),
    "twd_container_inspect": (C.c_int, [C.c_char_p, C.POINTER(ContainerInfo)]),
    "twd_head_load": (C.c_int, [C.c_char_p, _vp, C.POINTER(_vp)]),
    "twd_head_norm_weight": (_vp, [_vp]),
    "twd_generator_create": (C.c_int, [_vp, C.POINTER(GenerationParams), C.POINTER(_u32), _u32,
                                       C.POINTER(_u32), _u32, C.POINTER(_vp)]),
    "twd_generator_create_ex": (C.c_int, [_vp, C.POINTER(GenerationOptions), C.POINTER(_u32), _u32,
                                          C.POINTER(_u32), _u32, TokenCallback, _vp,
                                          C.POINTER(_vp)]),
    "twd_generator_cancel": (None, [_vp]),
    "twd_generator_stop_reason": (C.c_int, [_vp]),
    "twd_generator_sync": (C.c_int, [_vp, C.POINTER(C.c_int)]),
    "twd_head_finish_state": (_vp, [_vp]),
    "twd_generator_destroy": (None, [_vp]),
    "twd_generator_step": (C.c_int, [_vp, _vp, _vp, C.POINTER(_u32), C.POINTER(C.c_int)]),
    "twd_generator_step_rmsnorm": (C.c_int, [_vp, _vp, _vp, _f32, _vp, C.POINTER(_u32),
                                             C.POINTER(C.c_int)]),
    "twd_generator_history": (C.c_int, [_vp, C.POINTER(_vp), C.POINTER(_u32)]),
    "twd_generator_tokens": (C.c_int, [_vp, C.POINTER(_u32), _u32, C.POINTER(_u32)]),
    "twd_selector_create": (C.c_int, [_u32, _u32, C.POINTER(_vp)]),
    "twd_selector_destroy": (None, [_vp]),
    "twd_select": (C.c_int, [_vp, _vp, _u32, _u32, _u64, C.POINTER(RowParams), _vp, _vp, _vp]),
    "twd_select_noalloc": (C.c_int, [_vp, _u32, _u32, _u64, C.POINTER(RowParams), _vp, _vp, _vp]),
    "twd_verify": (C.c_int, [_vp, _vp, _u32, _u32, _u64, C.POINTER(RowParams), _u64, _vp, _u32,
                             _vp, _vp]),
    "twd_verify_draft": (C.c_int, [_vp, _vp, _u32, _u32, _u64, C.POINTER(_vp), _u32,
                                   C.POINTER(RowParams), _u64, _vp, _u32, _vp, _vp]),
    "twd_rejection_uniforms": (None, [_u64, C.POINTER(_f32), C.POINTER(_f32)]),
    "twd_verify_draft_sums": (C.c_int, [_vp, C.POINTER(_f32), C.POINTER(_u32), _u32, C.POINTER(_u32)]),
    "twd_selector_verify_state": (_vp, [_vp]),
    "twd_probe_expf": (C.c_int, [_vp, _vp, _u64, _vp]),
    "twd_probe_exp": (C.c_int, [_vp, _vp, _u64, _vp]),
    "twd_splitmix64": (_u64, [_u64]),
    "twd_seed_for": (_u64, [C.c_int, _u64, C.c_int]),
    "twd_uniform_from_seed": (_f32, [_u64]),
    "twd_validate_sampling": (C.c_int, [_f32, _f32, _i32, _f32]),
    "twd_generate_head": (C.c_int, [_vp, _u32, _u32, _u32, _u64, _vp]),
    "twd_head_bytes": (_u64, [_u32, _u32, _u32]),
    "twd_probe_read_bandwidth": (C.c_int, [_vp, _u64, _u32, _u32, _vp, C.POINTER(_f32),
                                           C.POINTER(_u64)]),
}


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                          "(or python turbo-winfare-dense_amd/build.py) first")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    return (lib.twd_last_error() or b"").decode()


def _check(rc: int) -> None:
    if rc != TWD_OK:
        raise TwdError(rc, last_error())


def _ptr(t) -> int | None:
    if t is None or isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream=None) -> int | None:
    if stream is not None:
        return stream
    import torch
    return torch.cuda.current_stream().cuda_stream


# ---- sampling.hpp mirror --------------------------------------------------------------------------

@dataclasses.dataclass
class SamplingParams:
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    repetition_penalty: float = 1.0
    has_seed: bool = False
    seed: int = 0

    def is_greedy(self) -> bool:
        import numpy as np
        return (np.float32(self.temperature) <= 0.0
                and np.float32(self.repetition_penalty) == np.float32(1.0))


def validate_sampling(p: SamplingParams) -> None:
    if lib.twd_validate_sampling(p.temperature, p.top_p, p.top_k, p.repetition_penalty) != TWD_OK:
        raise G4DenseFormatError(last_error())


def splitmix64(x: int) -> int:
    return int(lib.twd_splitmix64(x & 0xFFFFFFFFFFFFFFFF))


def seed_for(p: SamplingParams, position: int) -> int:
    return int(lib.twd_seed_for(1 if p.has_seed else 0, p.seed & 0xFFFFFFFFFFFFFFFF, position))


def uniform_from_seed(seed: int) -> float:
    return float(lib.twd_uniform_from_seed(seed & 0xFFFFFFFFFFFFFFFF))


def row_params(p: SamplingParams, uniform: float = 0.0, softcap: float = 0.0,
               history_offset: int = 0, history_len: int = 0,
               repetition_penalty: float | None = None) -> RowParams:
    rp = p.repetition_penalty if repetition_penalty is None else repetition_penalty
    return RowParams(p.temperature, p.top_p, p.top_k, rp, uniform, softcap, history_offset,
                     history_len)


def _params_array(params: Sequence[RowParams]):
    arr = (RowParams * len(params))(*params)
    return arr


class Selector:
    """Scratch for selection over caller-owned device logits (twd_selector)."""

    def __init__(self, max_vocab: int, max_rows: int = MAX_ROWS):
        h = C.c_void_p()
        _check(lib.twd_selector_create(max_vocab, max_rows, C.byref(h)))
        self.handle = h
        self.max_vocab = max_vocab
        self._draft_ptrs = None  # (addresses, ctypes array) of the last verify_draft's draft rows

    def close(self):
        if self.handle:
            lib.twd_selector_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def select(self, logits, params: Sequence[RowParams], history=None, tokens=None,
               stream=None):
        """Penalty (in place) + sample_token per row of a [rows, vocab] float32 device tensor."""
        import torch
        rows, vocab = logits.shape
        if tokens is None:
            tokens = torch.empty(rows, dtype=torch.int32, device=logits.device)
        arr = _params_array(params)
        if logits.stride(1) != 1:
            raise ValueError("logit rows must be contiguous")
        stride = logits.stride(0) if rows > 1 else vocab  # a size-1 dim may carry any stride
        _check(lib.twd_select(self.handle, _ptr(logits), vocab, rows, stride, arr,
                              _ptr(history), _ptr(tokens), _stream(stream)))
        return tokens

    def verify(self, logits, params: RowParams, base_seed: int, drafts, result=None,
               stream=None):
        import torch
        rows, vocab = logits.shape
        if result is None:
            result = torch.zeros(VERIFY_WORDS, dtype=torch.int32, device=logits.device)
        if logits.stride(1) != 1:
            raise ValueError("logit rows must be contiguous")
        stride = logits.stride(0) if rows > 1 else vocab
        _check(lib.twd_verify(self.handle, _ptr(logits), vocab, rows, stride,
                              C.byref(params), base_seed & 0xFFFFFFFFFFFFFFFF, _ptr(drafts),
                              0 if drafts is None else drafts.numel(), _ptr(result),
                              _stream(stream)))
        return result

    def draft_sums(self) -> dict:
        """{position: (target sum, draft sum)} of the last verify_draft that had draft rows."""
        sums = (_f32 * (2 * MAX_ROWS))()
        pos = (_u32 * MAX_ROWS)()
        n = _u32()
        _check(lib.twd_verify_draft_sums(self.handle, sums, pos, MAX_ROWS, C.byref(n)))
        return {int(pos[i]): (float(sums[2 * i]), float(sums[2 * i + 1])) for i in range(n.value)}

    def verify_draft(self, logits, draft_rows, params: RowParams, base_seed: int, drafts,
                     result=None, stream=None):
        """evaluate_verification with draft logits (speculator.cpp:34-153): draft_rows[i] is a
        float32 device row of position i's draft logits, or None."""
        rows, vocab = logits.shape
        if result is None:
            import torch
            result = torch.zeros(VERIFY_WORDS, dtype=torch.int32, device=logits.device)
        if logits.stride(1) != 1:
            raise ValueError("logit rows must be contiguous")
        # the pointer array of the last list of draft rows is kept, so repeated calls with the
        # same rows only compare their addresses
        key = tuple(0 if r is None else r.data_ptr() for r in draft_rows)
        cached = self._draft_ptrs
        if cached is None or cached[0] != key:
            for r in draft_rows:
                if r is not None and (r.numel() != vocab or not r.is_contiguous()):
                    raise ValueError("each draft row must be a contiguous row of vocab floats")
            cached = (key, (_vp * max(1, len(key)))(*[k or None for k in key]))
            self._draft_ptrs = cached
        stride = logits.stride(0) if rows > 1 else vocab
        _check(lib.twd_verify_draft(self.handle, logits.data_ptr(), vocab, rows, stride, cached[1],
                                    len(key), C.byref(params),
                                    base_seed & 0xFFFFFFFFFFFFFFFF, _ptr(drafts),
                                    0 if drafts is None else drafts.numel(), result.data_ptr(),
                                    _stream(stream)))
        return result


def probe_expf(x, out=None, stream=None):
    """The draft verify's device expf over a float32 device tensor (twd_probe_expf)."""
    import torch
    if out is None:
        out = torch.empty_like(x)
    _check(lib.twd_probe_expf(_ptr(x), _ptr(out), x.numel(), _stream(stream)))
    return out


def probe_exp(x, out=None, stream=None):
    """The sampled shortlist's device exp(double) over a float64 device tensor (twd_probe_exp)."""
    import torch
    if out is None:
        out = torch.empty_like(x)
    _check(lib.twd_probe_exp(_ptr(x), _ptr(out), x.numel(), _stream(stream)))
    return out


def rejection_uniforms(step_seed: int):
    """The two draws of speculator.cpp:87-89,105 for one step seed."""
    u1, u2 = _f32(), _f32()
    lib.twd_rejection_uniforms(step_seed & 0xFFFFFFFFFFFFFFFF, C.byref(u1), C.byref(u2))
    return float(u1.value), float(u2.value)


_default_selector: Selector | None = None


def _selector(vocab: int) -> Selector:
    global _default_selector
    if _default_selector is None or _default_selector.max_vocab < vocab:
        _default_selector = Selector(max(vocab, 262144), MAX_ROWS + 1)
    return _default_selector


def apply_repetition_penalty(logits, vocab: int, history, penalty: float, softcap: float):
    """In place on a float32 device tensor holding one row (sampling.cpp:74-90)."""
    import torch
    if float(penalty) == 1.0 or history is None or len(history) == 0:
        return logits
    hist = torch.as_tensor(history, dtype=torch.int64).to(torch.int32).to(logits.device)
    p = RowParams(0.0, 1.0, 0, penalty, 0.0, softcap, 0, hist.numel())
    sel = _selector(vocab)
    tok = torch.empty(1, dtype=torch.int32, device=logits.device)
    sel.select(logits.view(1, -1)[:, :vocab], [p], hist, tok)
    return logits


def sample_token(logits, vocab: int, p: SamplingParams, seed: int) -> int:
    """sample_token (sampling.cpp:92-169) on a float32 device tensor holding one row."""
    if vocab == 0:
        raise G4DenseFormatError("sample_token: empty vocabulary")
    sel = _selector(vocab)
    rp = row_params(p, uniform_from_seed(seed), repetition_penalty=1.0)
    tok = sel.select(logits.view(1, -1)[:, :vocab], [rp])
    t = int(tok.cpu().item()) & 0xFFFFFFFF
    if t == TOKEN_DEGENERATE:
        raise G4DenseFormatError("sample_token: logit distribution is degenerate")
    return t


def decode_verify(result) -> dict:
    v = [int(x) & 0xFFFFFFFF for x in result.cpu().tolist()]
    n = v[0]
    if n == TOKEN_DEGENERATE:
        raise G4DenseFormatError("sample_token: logit distribution is degenerate")
    total = v[2]
    return {
        "tokens": v[5:5 + n],
        "num_accepted": v[1],
        "total_drafted": total,
        "bonus_token_sampled": bool(v[3]),
        "bonus_token": v[4],
        "acceptance_rate": 0.0 if total == 0 else v[1] / total,
    }


class SpeculativeCoordinator:
    """speculator.hpp:19-43 over device logit rows."""

    def __init__(self):
        self.total_draft_tokens = 0
        self.total_accepted_tokens = 0

    def cumulative_acceptance_rate(self) -> float:
        return 0.0 if self.total_draft_tokens == 0 else (
            self.total_accepted_tokens / self.total_draft_tokens)

    def evaluate_verification(self, draft_tokens, target_logits, vocab_size: int,
                              sampling: SamplingParams, base_seed: int, draft_logits=()):
        """target_logits: float32 device tensor [rows, vocab]. draft_logits: per position a
        float32 device row of vocab entries, or an empty sequence / None for none.

        Any number of drafts, as speculator.cpp:34-153: the device verifies at most MAX_ROWS
        positions per call, so longer drafts go in batches of MAX_ROWS positions, each with
        base_seed + its first position (the seeds stay base_seed + i), until a correction or
        the end; only the last batch adds the bonus row."""
        import torch
        n = len(draft_tokens)
        self.total_draft_tokens += n
        out = {"tokens": [], "num_accepted": 0, "total_drafted": n,
               "bonus_token_sampled": False, "bonus_token": 0, "acceptance_rate": 0.0}
        rows_all = target_logits.shape[0]
        if n == 0 or rows_all == 0:
            return out
        k = min(n, rows_all)
        drafts_all = [int(x) for x in draft_tokens]
        sel = _selector(vocab_size)
        rows = [None if d is None or len(d) == 0 else d for d in draft_logits]
        use_draft = not sampling.is_greedy() and any(r is not None for r in rows)
        for b0 in range(0, k, MAX_ROWS):
            kb = min(MAX_ROWS, k - b0)
            last = b0 + kb == k
            nrows = min(rows_all, k + 1) - b0 if last else kb
            drafts = torch.tensor(drafts_all[b0:b0 + kb], dtype=torch.int64).to(torch.int32).to(
                target_logits.device)
            tl = target_logits[b0:b0 + nrows, :vocab_size]
            seed = base_seed + b0
            batch_rows = rows[b0:b0 + kb]
            if use_draft and any(r is not None for r in batch_rows):
                res = sel.verify_draft(tl, batch_rows, row_params(sampling), seed, drafts)
            else:
                res = sel.verify(tl, row_params(sampling), seed, drafts)
            got = decode_verify(res)
            out["tokens"] += got["tokens"]
            out["num_accepted"] += got["num_accepted"]
            out["bonus_token_sampled"] = got["bonus_token_sampled"]
            out["bonus_token"] = got["bonus_token"]
            if got["num_accepted"] < kb:
                break
        out["acceptance_rate"] = out["num_accepted"] / n
        self.total_accepted_tokens += out["num_accepted"]
        return out


# ---- the fused LM head --------------------------------------------------------------------------

def head_bytes(vocab: int, d_model: int, group: int = 64) -> int:
    return int(lib.twd_head_bytes(vocab, d_model, group))


def generate_head(buf, vocab: int, d_model: int, seed: int, group: int = 64, stream=None):
    """Fills a uint8 device tensor with the synthetic [W|S|B] head (formula in twd_head.h)."""
    _check(lib.twd_generate_head(_ptr(buf), vocab, d_model, group,
                                 seed & 0xFFFFFFFFFFFFFFFF, _stream(stream)))
    return buf


class Generator:
    """The decode loop around the head (runner.cpp:2312-2344) with a device-resident history."""

    def __init__(self, head: "LMHead", sampling: SamplingParams, prompt, max_tokens: int,
                 stop_ids=()):
        p = GenerationParams(sampling.temperature, sampling.top_p, sampling.top_k,
                             sampling.repetition_penalty, 1 if sampling.has_seed else 0,
                             sampling.seed & 0xFFFFFFFFFFFFFFFF, max_tokens)
        pr = (_u32 * max(1, len(prompt)))(*[int(t) for t in prompt])
        st = (_u32 * max(1, len(stop_ids)))(*[int(t) for t in stop_ids])
        h = C.c_void_p()
        _check(lib.twd_generator_create(head.handle, C.byref(p), pr, len(prompt), st,
                                        len(stop_ids), C.byref(h)))
        self.handle = h
        self.head = head
        self._cb = None

    @classmethod
    def from_options(cls, head: "LMHead", options: GenerationOptions | None, prompt,
                     stop_ids=(), on_token=None) -> "Generator":
        """twd_generator_create_ex: the reference's G4DenseGenerationOptions (None = its
        GenerationOptions defaults) and an optional on_token(index, token_id, delta) -> bool
        that ends the generation when it returns False (c_api.cpp:148-155)."""
        self = cls.__new__(cls)
        pr = (_u32 * max(1, len(prompt)))(*[int(t) for t in prompt])
        st = (_u32 * max(1, len(stop_ids)))(*[int(t) for t in stop_ids])
        self._cb = None
        if on_token is not None:
            self._cb = TokenCallback(lambda user, i, tok, delta: 1 if on_token(i, tok, delta) else 0)
        h = C.c_void_p()
        _check(lib.twd_generator_create_ex(head.handle, None if options is None else C.byref(options),
                                           pr, len(prompt), st, len(stop_ids),
                                           self._cb if self._cb is not None else TokenCallback(),
                                           None, C.byref(h)))
        self.handle = h
        self.head = head
        return self

    def cancel(self):
        lib.twd_generator_cancel(self.handle)

    def stop_reason(self) -> int:
        return int(lib.twd_generator_stop_reason(self.handle))

    def sync(self) -> bool:
        """Applies the stop rules to ids of steps taken without readback; returns finished."""
        fin = C.c_int()
        _check(lib.twd_generator_sync(self.handle, C.byref(fin)))
        return bool(fin.value)

    def step_async(self, hidden_bf16, stream=None):
        """A step that only enqueues (no readback, no stop rules until sync())."""
        _check(lib.twd_generator_step(self.handle, _ptr(hidden_bf16), _stream(stream), None, None))

    def close(self):
        if self.handle:
            lib.twd_generator_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, hidden_bf16, stream=None):
        """One step; returns (token, finished)."""
        tok, fin = _u32(), C.c_int()
        _check(lib.twd_generator_step(self.handle, _ptr(hidden_bf16), _stream(stream),
                                      C.byref(tok), C.byref(fin)))
        return int(tok.value), bool(fin.value)

    def step_rmsnorm(self, x, norm_weight, eps=1e-6, stream=None):
        tok, fin = _u32(), C.c_int()
        _check(lib.twd_generator_step_rmsnorm(self.handle, _ptr(x), _ptr(norm_weight), eps,
                                              _stream(stream), C.byref(tok), C.byref(fin)))
        return int(tok.value), bool(fin.value)

    def history(self):
        """(device address, length) of the history."""
        ptr, n = _vp(), _u32()
        _check(lib.twd_generator_history(self.handle, C.byref(ptr), C.byref(n)))
        return ptr.value, n.value

    def tokens(self) -> list:
        """The history (prompt, then the sampled ids), copied to the host."""
        _, n = self.history()
        buf = (_u32 * max(1, n))()
        got = _u32()
        _check(lib.twd_generator_tokens(self.handle, buf, n, C.byref(got)))
        return [int(buf[i]) for i in range(got.value)]


def container_info(path: str) -> dict:
    """The validated header of a .g4dense container (validate_header, format.cpp:6-65)."""
    info = ContainerInfo()
    _check(lib.twd_container_inspect(os.fsencode(path), C.byref(info)))
    return {n: getattr(info, n) for n, _ in ContainerInfo._fields_}


class LMHead:
    """The tied INT4 g64 LM head resident in HBM (twd_head)."""

    @classmethod
    def load(cls, path: str, stream=None) -> "LMHead":
        """The head of a .g4dense container (runner.cpp:423-443), with its final norm weight."""
        h = C.c_void_p()
        _check(lib.twd_head_load(os.fsencode(path), _stream(stream), C.byref(h)))
        self = cls.__new__(cls)
        self.handle = h
        vocab, d, cap, nbytes = _u32(), _u32(), _f32(), _u64()
        _check(lib.twd_head_info(h, C.byref(vocab), C.byref(d), C.byref(cap), C.byref(nbytes)))
        self.vocab, self.d_model, self.softcap = vocab.value, d.value, cap.value
        self.nbytes = head_bytes(self.vocab, self.d_model)
        return self

    def norm_weight(self) -> int | None:
        """Device address of the container's final RMSNorm weight (bf16 [d]), or None."""
        return lib.twd_head_norm_weight(self.handle)

    def __init__(self, wsb, vocab: int, d_model: int, softcap: float, group: int = 64,
                 stream=None):
        """wsb: the reference layout [W|S|B] as a uint8 device tensor (or host numpy array)."""
        h = C.c_void_p()
        nbytes = head_bytes(vocab, d_model, group)
        if hasattr(wsb, "data_ptr") and wsb.is_cuda:
            _check(lib.twd_head_create_device(_ptr(wsb), wsb.numel() * wsb.element_size(),
                                              vocab, d_model, group, softcap, _stream(stream),
                                              C.byref(h)))
        else:
            import numpy as np
            arr = np.ascontiguousarray(wsb)
            _check(lib.twd_head_create(arr.ctypes.data, arr.nbytes, vocab, d_model, group,
                                       softcap, C.byref(h)))
        self.handle = h
        self.vocab, self.d_model, self.softcap = vocab, d_model, softcap
        self.nbytes = nbytes

    def close(self):
        if self.handle:
            lib.twd_head_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def logits(self, hidden, out=None, stream=None):
        import torch
        rows = hidden.shape[0]
        if out is None:
            out = torch.empty(rows, self.vocab, dtype=torch.float32, device=hidden.device)
        _check(lib.twd_head_logits(self.handle, _ptr(hidden), rows, _ptr(out), _stream(stream)))
        return out

    def greedy(self, hidden, logits=None, tokens=None, stream=None):
        import torch
        rows = hidden.shape[0]
        if tokens is None:
            tokens = torch.empty(rows, dtype=torch.int32, device=hidden.device)
        _check(lib.twd_head_greedy(self.handle, _ptr(hidden), rows, _ptr(logits), _ptr(tokens),
                                   _stream(stream)))
        return tokens

    def sample(self, hidden, params: Sequence[RowParams], history=None, logits=None,
               tokens=None, stream=None):
        import torch
        rows = hidden.shape[0]
        if logits is None:
            logits = torch.empty(rows, self.vocab, dtype=torch.float32, device=hidden.device)
        if tokens is None:
            tokens = torch.empty(rows, dtype=torch.int32, device=hidden.device)
        arr = _params_array(params)
        _check(lib.twd_head_sample(self.handle, _ptr(hidden), rows, arr, _ptr(history),
                                   _ptr(logits), _ptr(tokens), _stream(stream)))
        return tokens, logits

    def verify_greedy(self, hidden, drafts, logits=None, result=None, stream=None):
        import torch
        rows = hidden.shape[0]
        if result is None:
            result = torch.zeros(VERIFY_WORDS, dtype=torch.int32, device=hidden.device)
        nd = 0 if drafts is None else drafts.numel()
        _check(lib.twd_head_verify_greedy(self.handle, _ptr(hidden), rows, _ptr(drafts), nd,
                                          _ptr(logits), _ptr(result), _stream(stream)))
        return result

    # ---- with the final RMSNorm as the prologue: x fp32 [rows, d], norm_weight bf16 bits [d] ----

    def logits_rmsnorm(self, x, norm_weight, eps=1e-6, out=None, stream=None):
        import torch
        rows = x.shape[0]
        if out is None:
            out = torch.empty(rows, self.vocab, dtype=torch.float32, device=x.device)
        _check(lib.twd_head_logits_rmsnorm(self.handle, _ptr(x), _ptr(norm_weight), eps, rows,
                                           _ptr(out), _stream(stream)))
        return out

    def greedy_rmsnorm(self, x, norm_weight, eps=1e-6, logits=None, tokens=None, stream=None):
        import torch
        rows = x.shape[0]
        if tokens is None:
            tokens = torch.empty(rows, dtype=torch.int32, device=x.device)
        _check(lib.twd_head_greedy_rmsnorm(self.handle, _ptr(x), _ptr(norm_weight), eps, rows,
                                           _ptr(logits), _ptr(tokens), _stream(stream)))
        return tokens

    def verify_greedy_rmsnorm(self, x, norm_weight, drafts, eps=1e-6, logits=None, result=None,
                              stream=None):
        import torch
        rows = x.shape[0]
        if result is None:
            result = torch.zeros(VERIFY_WORDS, dtype=torch.int32, device=x.device)
        nd = 0 if drafts is None else drafts.numel()
        _check(lib.twd_head_verify_greedy_rmsnorm(self.handle, _ptr(x), _ptr(norm_weight), eps,
                                                  rows, _ptr(drafts), nd, _ptr(logits),
                                                  _ptr(result), _stream(stream)))
        return result

    def sample_rmsnorm(self, x, norm_weight, params: Sequence[RowParams], eps=1e-6, history=None,
                       logits=None, tokens=None, stream=None):
        import torch
        rows = x.shape[0]
        if logits is None:
            logits = torch.empty(rows, self.vocab, dtype=torch.float32, device=x.device)
        if tokens is None:
            tokens = torch.empty(rows, dtype=torch.int32, device=x.device)
        arr = _params_array(params)
        _check(lib.twd_head_sample_rmsnorm(self.handle, _ptr(x), _ptr(norm_weight), eps, rows, arr,
                                           _ptr(history), _ptr(logits), _ptr(tokens),
                                           _stream(stream)))
        return tokens, logits


def probe_read_bandwidth(buf, waves: int = 32768, launches: int = 50, stream=None):
    """Pure-read ceiling over a uint8 device tensor: (GB/s, us per launch, bytes per launch)."""
    us, nbytes = _f32(), _u64()
    _check(lib.twd_probe_read_bandwidth(_ptr(buf), buf.numel(), waves, launches, _stream(stream),
                                        C.byref(us), C.byref(nbytes)))
    return nbytes.value / us.value / 1e3, us.value, nbytes.value
