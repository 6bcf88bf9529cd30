"""ctypes bindings of the C oracle plus pure-Python restatements. Test infrastructure only.

Values are numpy arrays. bfloat16 has no numpy dtype, so a bf16 tensor is carried as its
uint16 bit patterns (the same carrier the reference uses, code/lema/cache.py:98-103) and the
value dtype is named separately: "f32", "f16" or "bf16".
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import subprocess
from pathlib import Path

import numpy as np

__all__ = ["lib", "pack_codes", "latest_prev_match", "gather", "store_exchange",
           "store_home", "dict_rule", "brute_force", "DictStore", "HostStore", "ref_store",
           "DTYPES", "num_threads", "ORACLE_DIR"]

ORACLE_DIR = Path(__file__).resolve().parent
_SO = ORACLE_DIR / "liblema_oracle.so"
_REF_SO = ORACLE_DIR / "_ref" / "lema_store_ref.so"
DTYPES = {"f32": 0, "f16": 1, "bf16": 2}
_LIB = None
_REF = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64


def lib():
    """The oracle library, built with `make -C oracle oracle` if it is not there yet."""
    global _LIB
    if _LIB is None:
        if not _SO.exists():
            subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "oracle"], check=True)
        L = ctypes.CDLL(str(_SO))
        L.lo_pack_codes.argtypes = [_p, ctypes.c_int, _i64, ctypes.c_int, _p]
        L.lo_latest_prev_match.argtypes = [_p, _p, _i64, _i64, _p]
        L.lo_gather.argtypes = [_p, ctypes.c_int, _i64, _i64, _i64, _p, ctypes.c_int, _p]
        L.lo_store_exchange.argtypes = [_p, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _p,
                                        ctypes.c_int]
        L.lo_store_home.argtypes = [ctypes.c_uint64, ctypes.c_uint64, _i64]
        L.lo_store_home.restype = _i64
        L.lo_num_threads.restype = ctypes.c_int
        for f in ("lo_pack_codes", "lo_latest_prev_match", "lo_gather", "lo_store_exchange"):
            getattr(L, f).restype = ctypes.c_int
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def num_threads() -> int:
    return int(lib().lo_num_threads())


def pack_codes(z: np.ndarray, dtype: str) -> np.ndarray:
    """attention.py:82-97 on contiguous `[..., D]` values: one uint64 code per row."""
    z = np.ascontiguousarray(z)
    D = z.shape[-1]
    rows = z.size // D if D else 0
    out = np.empty(z.shape[:-1], dtype=np.uint64)
    rc = lib().lo_pack_codes(_ptr(z), DTYPES[dtype], rows, D, _ptr(out))
    if rc:
        raise ValueError(f"d_qk {D} > 64 cannot pack into a uint64")
    return out


def latest_prev_match(qc: np.ndarray, kc: np.ndarray) -> np.ndarray:
    """The dictionary rule on `[N, T]` codes (any integer dtype, compared as 64-bit
    patterns): for each i the largest j < i with kc[j] == qc[i], else -1."""
    qc = np.ascontiguousarray(qc).view(np.uint64) if qc.dtype.itemsize == 8 else \
        np.ascontiguousarray(qc.astype(np.uint64))
    kc = np.ascontiguousarray(kc).view(np.uint64) if kc.dtype.itemsize == 8 else \
        np.ascontiguousarray(kc.astype(np.uint64))
    N, T = qc.shape
    src = np.empty((N, T), dtype=np.int64)
    rc = lib().lo_latest_prev_match(_ptr(qc), _ptr(kc), N, T, _ptr(src))
    if rc:
        raise RuntimeError(f"oracle latest_prev_match failed ({rc})")
    return src


def gather(v: np.ndarray, dtype: str, src: np.ndarray, miss_mode: int = 0) -> np.ndarray:
    """attention.py:157-158 on contiguous `[N, T, dv]` values and `[N, T]` src.
    miss_mode 0: the dense path's v[row, 0] * 0; 1: the store path's zero bytes."""
    v = np.ascontiguousarray(v)
    src = np.ascontiguousarray(src, dtype=np.int64)
    N, T, dv = v.shape
    y = np.empty_like(v)
    rc = lib().lo_gather(_ptr(v), DTYPES[dtype], N, T, dv, _ptr(src), miss_mode, _ptr(y))
    if rc:
        raise RuntimeError(f"oracle gather failed ({rc})")
    return y


def store_home(code: int, group: int, cap: int) -> int:
    return int(lib().lo_store_home(ctypes.c_uint64(code & (2**64 - 1)),
                                   ctypes.c_uint64(group), cap))


def store_exchange(table: np.ndarray, cap: int, vbytes: int, qc: np.ndarray,
                   kc: np.ndarray, values: np.ndarray, out: np.ndarray, T: int, g0: int,
                   added: np.ndarray, nthreads: int = 1) -> bool:
    """store.cpp:127-162 on host arrays. Returns True when the table was found full."""
    for a in (table, qc, kc, values, out, added):
        assert a.flags.c_contiguous
    n = qc.size
    rc = lib().lo_store_exchange(_ptr(table), cap, vbytes, _ptr(qc), _ptr(kc), _ptr(values),
                                 _ptr(out), n, T, g0, _ptr(added), nthreads)
    if rc == 2:
        raise ValueError("items must be partitions x T, vbytes a multiple of 8")
    return rc == 1


class HostStore:
    """A host-RAM table driven by the C restatement of store.cpp: the shape of the
    reference's HashStore (code/lema/cache.py:129-201), for checking and CPU timing."""

    def __init__(self, vbytes: int, groups: int, capacity: int, nthreads: int = 1):
        if vbytes % 8:
            raise ValueError("vbytes must be a multiple of 8")
        self.vbytes, self.groups, self.nthreads = vbytes, groups, nthreads
        self.cap = max(16, int(capacity))
        self.table = np.zeros((self.cap, 16 + vbytes), dtype=np.uint8)
        self.counts = np.zeros(groups, dtype=np.int64)

    def exchange(self, qc: np.ndarray, kc: np.ndarray, values: np.ndarray, out: np.ndarray,
                 T: int, g0: int):
        P = qc.size // T
        added = np.zeros(P, dtype=np.int64)
        full = store_exchange(self.table, self.cap, self.vbytes, qc.view(np.uint64),
                              kc.view(np.uint64), values, out, T, g0, added, self.nthreads)
        self.counts[g0:g0 + P] += added
        if full:
            raise RuntimeError("hash table full: the store is presized and never grows -- "
                               "provision more capacity")

    def __len__(self):
        return int(self.counts.sum())


# ------------------------------------------------------------ pure-Python restatements
def dict_rule(qc, kc) -> list:
    """verification/lema.py:26-29 verbatim in spirit: look the query up, then insert the
    key. One row."""
    src, last = [], {}
    for i in range(len(qc)):
        src.append(last.get(int(qc[i]), -1))
        last[int(kc[i])] = i
    return src


def brute_force(qc, kc) -> np.ndarray:
    """O(T^2): src[i] = max{j < i : kc[j] == qc[i]} or -1, straight from the definition
    (code/lema/attention.py:101)."""
    qc = np.asarray(qc)
    kc = np.asarray(kc)
    T = len(qc)
    eq = qc[:, None] == kc[None, :]
    eq &= np.tri(T, T, -1, dtype=bool)          # strictly causal: j < i
    j = np.arange(T)
    return np.where(eq.any(1), np.where(eq, j[None, :], -1).max(1), -1)


class DictStore:
    """code/tests/test_store.py:17-41: one dict per partition, latest write wins, every
    query looked up before its key is inserted."""

    def __init__(self, groups: int, vbytes: int):
        self.ref = [dict() for _ in range(groups)]
        self.vbytes = vbytes

    def exchange(self, qc: np.ndarray, kc: np.ndarray, values: np.ndarray, T: int, g0: int):
        """qc, kc `[n]` 64-bit, values `[n, vbytes]` uint8. Returns out `[n, vbytes]`."""
        n = qc.size
        out = np.zeros((n, self.vbytes), dtype=np.uint8)
        zeros = np.zeros(self.vbytes, dtype=np.uint8)
        for i in range(n):
            d = self.ref[g0 + i // T]
            out[i] = d.get(int(qc[i]), zeros)
            d[int(kc[i])] = values[i].copy()
        return out

    def counts(self) -> np.ndarray:
        return np.array([len(d) for d in self.ref], dtype=np.int64)


def ref_store():
    """The reference's `lema_store` module (store.cpp compiled into oracle/_ref/), or None
    where it was not built."""
    global _REF
    if _REF is None and _REF_SO.exists() and os.environ.get("LEMA_NO_REF") != "1":
        spec = importlib.util.spec_from_file_location("lema_store_ref", str(_REF_SO))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _REF = mod
    return _REF
