"""Seeded synthetic inputs of the benchmark workloads (numpy, host side).

    dense_plumbing     B1 H8 T4096, 16-bit uniform codes, d_v 64 fp32 ~N(0,1)
    zipf_prefill       B8 H16 T16384, 24-bit codes: per (b, h) a book of 4096 distinct codes,
                       ranks drawn from a truncated Zipf p(r) ~ r^-1.1 independently for
                       queries and keys; d_v 64 bf16 ~N(0,1)
    uniform_decode     per step fresh uniform 32-bit query/key codes (the reference's
                       worst-case access pattern, code/experiments/main_inference/common.py:170-196)

Values come back as float32 numpy arrays; callers convert to the value dtype.
"""
from __future__ import annotations

import numpy as np

__all__ = ["dense_plumbing", "zipf_codes", "zipf_prefill", "normal_values",
           "ZIPF_PREFILL", "DENSE_PLUMBING"]

DENSE_PLUMBING = dict(B=1, H=8, T=4096, bits=16, dv=64)
ZIPF_PREFILL = dict(B=8, H=16, T=16384, bits=24, distinct=4096, s=1.1, dv=64)


def dense_plumbing(seed: int = 0, B: int = 1, H: int = 8, T: int = 4096, bits: int = 16,
                   dv: int = 64):
    """qc, kc int64 [B, H, T] uniform in [0, 2^bits); v float32 [B, H, T, dv]."""
    rng = np.random.default_rng(seed)
    qc = rng.integers(0, 1 << bits, size=(B, H, T), dtype=np.int64)
    kc = rng.integers(0, 1 << bits, size=(B, H, T), dtype=np.int64)
    v = rng.standard_normal((B, H, T, dv), dtype=np.float32)
    return qc, kc, v


def zipf_codes(rng: np.random.Generator, rows: int, T: int, bits: int = 24,
               distinct: int = 4096, s: float = 1.1):
    """Per row a book of `distinct` distinct codes of `bits` bits; query and key ranks drawn
    independently from p(r) ~ r^-s, r = 1..distinct. Returns qc, kc int64 [rows, T]."""
    p = np.arange(1, distinct + 1, dtype=np.float64) ** -s
    cdf = np.cumsum(p / p.sum())
    cdf[-1] = 1.0
    book = np.stack([rng.choice(1 << bits, size=distinct, replace=False) for _ in range(rows)])
    book = book.astype(np.int64)
    rq = np.minimum(np.searchsorted(cdf, rng.random((rows, T)), side="right"), distinct - 1)
    rk = np.minimum(np.searchsorted(cdf, rng.random((rows, T)), side="right"), distinct - 1)
    return np.take_along_axis(book, rq, 1), np.take_along_axis(book, rk, 1)


def normal_values(rng: np.random.Generator, shape) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32)


def zipf_prefill(seed: int = 0, B: int = 8, H: int = 16, T: int = 16384, bits: int = 24,
                 distinct: int = 4096, s: float = 1.1, dv: int = 64, values: bool = True):
    """qc, kc int64 [B, H, T] and v float32 [B, H, T, dv] (or None)."""
    rng = np.random.default_rng(seed)
    qc, kc = zipf_codes(rng, B * H, T, bits, distinct, s)
    v = normal_values(rng, (B, H, T, dv)) if values else None
    return qc.reshape(B, H, T), kc.reshape(B, H, T), v
