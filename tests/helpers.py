"""Shared helpers of the test suite (data generation in the BASELINE configs' shapes)."""
from __future__ import annotations

import importlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def twd():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    return importlib.import_module("turbo-winfare-dense_amd")


def bf16_rne(x) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def hidden_bf16(seed: int, rows: int, d: int) -> np.ndarray:
    """h ~ N(0,1) rounded to bf16, as BASELINE configs 2-5 specify."""
    return bf16_rne(np.random.default_rng(seed).standard_normal((rows, d)).astype(np.float32))


def wsb_bytes(W, S, B) -> np.ndarray:
    return np.concatenate([np.ascontiguousarray(W).reshape(-1).view(np.uint8),
                           np.ascontiguousarray(S).reshape(-1).view(np.uint8),
                           np.ascontiguousarray(B).reshape(-1).view(np.uint8)])


def allclose_report(got, want, atol, rtol):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    err = np.abs(got - want)
    ratio = err / (atol + rtol * np.abs(want))
    i = int(np.argmax(ratio))
    return float(ratio[i]), float(err.max()), i


# ---- a .g4dense container writer (include/g4dense/format.hpp:26-110) --------------------------

HEADER_FIELDS_U32 = ["magic", "version", "quant_type", "num_layers", "d_model", "d_ff",
                     "num_q_heads", "num_kv_heads", "head_dim", "vocab_size", "sliding_window",
                     "quant_group_size", "scale_dtype", "tied_embeddings"]


def container_header(**f) -> bytes:
    """The 4096-byte header: 14 u32, global_layer_mask u64, four floats, four u64, then
    layer_offsets[60], layer_sizes[60], the payload SHA-256 and zero padding."""
    import struct
    out = struct.pack("<14I", *[int(f.get(k, 0)) for k in HEADER_FIELDS_U32])
    out += struct.pack("<Q", int(f.get("global_layer_mask", 0)))
    out += struct.pack("<4f", f.get("rope_theta_local", 10000.0), f.get("rope_theta_global", 1e6),
                       f.get("rope_scaling", 1.0), f.get("final_logit_softcapping", 30.0))
    out += struct.pack("<4Q", *[int(f.get(k, 0)) for k in ("embed_offset", "embed_size",
                                                             "lm_head_offset", "lm_head_size")])
    lo = list(f.get("layer_offsets", [])) + [0] * 60
    ls = list(f.get("layer_sizes", [])) + [0] * 60
    out += struct.pack("<60Q", *lo[:60]) + struct.pack("<60Q", *ls[:60])
    out += bytes(f.get("payload_sha256", b"\0" * 32))
    assert len(out) == 0x450
    return out + b"\0" * (4096 - len(out))


def write_container(path, W, S, B, norm_w, vocab, d, softcap=30.0, num_layers=2, **overrides):
    """A tied-embedding container: [header | embedding W|S|B|final norm, padded to 4096 |
    num_layers dummy layer blocks of 4096 bytes], with lm_head_offset = embed_offset as the
    reference's writer sets it (tools/make_synthetic_model.py)."""
    embed = wsb_bytes(W, S, B).tobytes() + np.ascontiguousarray(norm_w, np.uint16).tobytes()
    embed += b"\0" * (-len(embed) % 4096)
    layers_at = 4096 + len(embed)
    fields = dict(magic=0x4734444E, version=3, quant_type=1, num_layers=num_layers, d_model=d,
                  d_ff=4 * d, num_q_heads=8, num_kv_heads=4, head_dim=128, vocab_size=vocab,
                  sliding_window=1024, quant_group_size=64, scale_dtype=1, tied_embeddings=1,
                  final_logit_softcapping=softcap, embed_offset=4096, embed_size=len(embed),
                  lm_head_offset=4096, lm_head_size=len(embed),
                  layer_offsets=[layers_at + 4096 * i for i in range(num_layers)],
                  layer_sizes=[4096] * num_layers)
    fields.update(overrides)
    with open(path, "wb") as fh:
        fh.write(container_header(**fields))
        fh.write(embed)
        fh.write(b"\x5a" * (4096 * num_layers))
    return fields
