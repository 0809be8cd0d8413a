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
