"""Seeded synthetic inputs of the benchmark workloads (numpy, host side).

    dense_plumbing     B1 H8 T4096, 16-bit uniform codes, d_v 64 fp32 ~N(0,1)
    zipf_prefill       B8 H16 T16384, 24-bit codes: per (b, h) a book of 4096 distinct codes,
                       ranks drawn from a truncated Zipf p(r) ~ r^-1.1 independently for
                       queries and keys; d_v 64 bf16 ~N(0,1)
    uniform_decode     per step fresh uniform 32-bit query/key codes (the reference's
                       worst-case access pattern, code/experiments/main_inference/common.py:170-196)
    long_context       B1 H64 T = 2^24 fed in calls of 2^20 positions, 32-bit codes: each key
                       is uniform with probability 0.9, else a copy of the key d positions back,
                       d ~ Geometric(1e-5) (mean 1e5); each query likewise copies an earlier key
                       (so copies hit) or is uniform. Counter-based: every position's codes are
                       a pure function of (seed, head, position), computed in torch on any
                       device for any slice of positions, so a 2^24-position run never has to
                       be held anywhere.

Values come back as float32 numpy arrays; callers convert to the value dtype.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = ["dense_plumbing", "zipf_codes", "zipf_prefill", "normal_values",
           "long_context_codes", "long_context_code_at", "ZIPF_PREFILL", "DENSE_PLUMBING",
           "LONG_CONTEXT"]

DENSE_PLUMBING = dict(B=1, H=8, T=4096, bits=16, dv=64)
ZIPF_PREFILL = dict(B=8, H=16, T=16384, bits=24, distinct=4096, s=1.1, dv=64)
LONG_CONTEXT = dict(B=1, H=64, T=1 << 24, call=1 << 20, p_copy=0.1, p_geom=1e-5, dv=24)


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


# ----------------------------------------------------------------- long-context codes
# splitmix64's finaliser over a counter (seed, stream, head, position); in int64 torch
# arithmetic (multiplication wraps, right shifts are made logical with a mask).
_GOLD = 0x9E3779B97F4A7C15
_MASK64 = (1 << 64) - 1


def _s64(v: int) -> int:
    v &= _MASK64
    return v - (1 << 64) if v >> 63 else v


def _srl(x, k: int):
    return (x >> k) & ((1 << (64 - k)) - 1)


def _mix(x):
    x = (x ^ _srl(x, 30)) * _s64(0xBF58476D1CE4E5B9)
    x = (x ^ _srl(x, 27)) * _s64(0x94D049BB133111EB)
    return x ^ _srl(x, 31)


def _ctr_hash(seed: int, stream: int, head, pos):
    """64-bit hash of (seed, stream, head, position): head, pos int64 tensors."""
    key = _s64(_GOLD * (seed * 8 + stream + 1))
    return _mix(_mix(pos ^ key) ^ (head * _s64(_GOLD)))


def _unit(h):
    return _srl(h, 11).double() * (2.0 ** -53)


def _geometric(h, p: float):
    """d >= 1 with P(d = k) = p (1 - p)^(k - 1)."""
    import torch
    u = (_srl(h, 11) + 1).double() * (2.0 ** -53)            # (0, 1]
    return 1 + torch.floor(torch.log(u) / math.log1p(-p)).long()


def _key_codes(seed, head, pos, p_copy, p_geom):
    import torch
    pos = pos.clone()
    for _ in range(256):                     # follow copy links back to an original key
        link = (_unit(_ctr_hash(seed, 0, head, pos)) < p_copy)
        back = pos - _geometric(_ctr_hash(seed, 1, head, pos), p_geom)
        move = link & (back >= 0)
        if not bool(move.any()):
            break
        pos = torch.where(move, back, pos)
    return _ctr_hash(seed, 2, head, pos) & 0xFFFFFFFF


def long_context_codes(seed: int, H: int, t0: int, t1: int, device=None,
                       p_copy: float = 0.1, p_geom: float = 1e-5):
    """qc, kc int64 [H, t1 - t0] (values in [0, 2^32)) of positions [t0, t1) of every head.

    Key j is original (uniform 32-bit code) with probability 1 - p_copy, else a copy of key
    j - d, d ~ Geometric(p_geom), when j - d >= 0. Query i is uniform with probability
    1 - p_copy, else the code of key i - d (d >= 1, so the copy has a strictly earlier
    match)."""
    import torch
    head = torch.arange(H, dtype=torch.int64, device=device).view(H, 1)
    pos = torch.arange(t0, t1, dtype=torch.int64, device=device).view(1, -1).expand(H, -1)
    kc = _key_codes(seed, head, pos, p_copy, p_geom)
    copy = _unit(_ctr_hash(seed, 3, head, pos)) < p_copy
    src = pos - _geometric(_ctr_hash(seed, 4, head, pos), p_geom)
    copy = copy & (src >= 0)
    qc = _ctr_hash(seed, 5, head, pos) & 0xFFFFFFFF
    if bool(copy.any()):
        hh = head.expand(H, pos.shape[1])[copy]
        qc[copy] = _key_codes(seed, hh, src[copy], p_copy, p_geom)
    return qc, kc


def long_context_code_at(seed: int, head: int, pos: int, kind: str,
                         p_copy: float = 0.1, p_geom: float = 1e-5) -> int:
    """One position's key ("k") or query ("q") code, computed through the same tensor
    arithmetic (a scalar convenience for checks)."""
    import torch
    h = torch.tensor([[head]], dtype=torch.int64)
    p = torch.tensor([[pos]], dtype=torch.int64)
    if kind == "k":
        return int(_key_codes(seed, h, p, p_copy, p_geom))
    qc, _ = long_context_codes(seed, head + 1, pos, pos + 1, None, p_copy, p_geom)
    return int(qc[head, 0])
