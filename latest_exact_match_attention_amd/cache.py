"""The LEMA retrieval state in HBM: the reference's `HashStore`, `LayerStore` and `LemaCache`
(code/lema/cache.py:129-378) with the same names, arguments, results and errors, whose table
lives in device memory and is exchanged against by the HIP kernels of liblema_hip.so.

A LEMA head's whole state after position i is the map code -> value of the latest position
that emitted it, so a decode step is one lookup and one insert per (layer, stream, head). The
reference keeps ONE shared open-addressing table in host RAM and crosses PCIe for every layer;
here the same table (same slot format, same home-slot hash) sits in HBM, so an exchange is one
kernel launch with no host round trip, and a decode step can be captured into a HIP graph.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib

__all__ = ["HashStore", "LayerStore", "LemaCache"]

# value dtypes a table can carry; numpy has no bfloat16, the reference names it uint16
_ITEMSIZE = {np.dtype(np.float16): 2, np.dtype(np.float32): 4, np.dtype(np.uint16): 2,
             torch.float16: 2, torch.float32: 4, torch.bfloat16: 2, torch.uint16: 2}


def _itemsize(dtype) -> int:
    key = dtype if isinstance(dtype, torch.dtype) else np.dtype(dtype)
    if key not in _ITEMSIZE:
        raise ValueError(f"store dtype must be float16, float32, or uint16 (the carrier for "
                         f"bfloat16), got {dtype}")
    return _ITEMSIZE[key]


def _codes(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    if t.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"codes must be int64 or int32, got {t.dtype}")
    return t.contiguous(), t.element_size()


class HashStore:
    """ONE open-addressing table (linear probing, fixed capacity) for every (layer, stream,
    head) partition; an entry's key is (group, code) (code/lema/cache.py:129-201).

    `capacity` is slots, exact (the home slot is a multiply, not a mask). The table is a zeroed
    allocation -- zero is the free state, so it is empty as allocated -- of
    capacity x (16 + d_v * itemsize) bytes, never resized; a key that finds no free slot makes
    `exchange` raise RuntimeError("hash table full ...").

    `place` puts the table in device memory ("hbm") or in pinned host RAM ("ram", the
    reference's placement, for tables larger than device memory): the same kernels then read,
    write and claim slots in host memory over the host link, in place. "ram" needs a link that
    carries the device's atomics to host memory, and is refused otherwise. Codes, values, counts
    and the full flag stay on the device either way.
    """

    def __init__(self, d_v: int, groups: int, dtype=np.float16, capacity: int = 256,
                 device=None, place: str = "hbm"):
        self.d_v, self.dtype, self.groups = d_v, dtype, groups
        self.vbytes = d_v * _itemsize(dtype)
        if self.vbytes % 8:
            raise ValueError(f"value row of {self.vbytes} bytes breaks slot alignment "
                             f"(d_v * itemsize must be a multiple of 8)")
        self.stride = 16 + self.vbytes
        self.cap = max(16, int(capacity))
        self.device = torch.device(device) if device is not None else torch.device("cuda", 0)
        if self.device.type != "cuda":
            raise TypeError(f"the store lives in device memory; got device {self.device}")
        if place not in ("hbm", "ram"):
            raise ValueError(f"place must be 'hbm' (device memory) or 'ram' (host memory), "
                             f"got {place!r}")
        self.place = place
        self._host = None
        if place == "ram":
            dev_index = self.device.index if self.device.index is not None else 0
            if not _lib.host_atomics_supported(dev_index):
                raise RuntimeError("a store in host RAM needs device atomics on host memory, "
                                   "which this system's host link does not carry")
            self._host = _lib.HostTable(self.cap * self.stride)
            self.table = self._host.tensor().view(self.cap, self.stride)
        else:
            self.table = torch.zeros((self.cap, self.stride), dtype=torch.uint8,
                                     device=self.device)
        self.counts_device = torch.zeros(groups, dtype=torch.int64, device=self.device)
        self.full_flag = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._ws = None          # scratch of long calls (bulk path), kept while small

    @property
    def counts(self) -> torch.Tensor:
        """Entries per partition (a host copy, like the reference's CPU tensor)."""
        return self.counts_device.cpu()

    def __len__(self):
        return int(self.counts_device.sum())

    def nbytes(self) -> int:
        return self.table.numel()

    def load(self) -> float:
        """Fraction of slots occupied (linear probing's cost is set by this alone)."""
        return len(self) / self.cap

    def exchange(self, qcodes: torch.Tensor | None, kcodes: torch.Tensor, values: torch.Tensor,
                 out: torch.Tensor | None, T: int, g0: int, check: bool = True):
        """One pass of P partitions x T positions (code/lema/cache.py:184-201): item i
        (partition i // T, position i % T, group g0 + i // T) looks `qcodes[i]` up into
        `out[i]` (zeros on a miss) and then inserts `kcodes[i] -> values[i]`, each partition in
        position order. Device tensors: codes int64 (or int32 for codes below 2^32), values and
        out rows of `vbytes` bytes in any dtype. `qcodes=None` only inserts. With `check` the
        full flag is read back (a device sync) and a full table raises like the reference;
        without it, call `check_full()` later (e.g. after a graph replay). A long call
        (T > 1024 with at most 128 partitions, T > 2048 with more) takes the bulk path with
        a device workspace, kept for the next call when at most KEEP_WORKSPACE_BYTES."""
        kc, cb = _codes(kcodes)
        n = kc.numel()
        if qcodes is not None:
            qc, qcb = _codes(qcodes)
            if qcb != cb:
                qc, kc, cb = _lib.widen_codes(qc), _lib.widen_codes(kc), 8
            if qc.numel() != n:
                raise ValueError("query and key codes differ in count")
        else:
            qc = None
        if T <= 0 or n % T:
            raise ValueError(f"items must be partitions x T (n={n}, T={T})")
        if g0 < 0 or g0 + n // T > self.groups:
            raise ValueError(f"groups [{g0}, {g0 + n // T}) outside the store's {self.groups}")
        _lib.require_device(kc, values)
        values = values.contiguous()
        if values.numel() * values.element_size() != n * self.vbytes:
            raise ValueError(f"values hold {values.numel() * values.element_size()} bytes, "
                             f"need {n} x {self.vbytes}")
        if qc is not None:
            if out is None or not out.is_contiguous() or \
                    out.numel() * out.element_size() != n * self.vbytes:
                raise ValueError(f"out must be a contiguous buffer of {n} x {self.vbytes} bytes")
        if check:
            self.full_flag.zero_()
        L = _lib.lib()
        ws_bytes = L.lema_store_workspace_bytes(n, T, cb)
        ws = self._workspace(ws_bytes) if ws_bytes > 0 else None
        _lib.check(L.lema_store_exchange_ws(
            self.table_ptr(), self.cap, self.vbytes,
            qc.data_ptr() if qc is not None else None, kc.data_ptr(), cb, values.data_ptr(),
            out.data_ptr() if qc is not None else None, n, T, g0,
            self.counts_device.data_ptr(), self.full_flag.data_ptr(),
            ws.data_ptr() if ws is not None else None, ws_bytes, _lib.stream_of(kc)))
        if ws is not None and ws.numel() > self.KEEP_WORKSPACE_BYTES:
            self._ws = None       # freed once the call's kernels are done (stream-ordered)
        if check:
            self.check_full()

    # Scratch of long calls above this size is handed back to torch's allocator after the call
    # instead of being kept for the next one (a 1,024-partition prefill's is a few GB, which
    # later decode steps do not need).
    KEEP_WORKSPACE_BYTES = 256 << 20

    def table_ptr(self) -> int:
        """The table's address for the kernels (the device-side address of a host table)."""
        return self._host.dev_ptr if self._host is not None else self.table.data_ptr()

    def _workspace(self, nbytes: int) -> torch.Tensor:
        """Device scratch of a long call (small ones are kept for the next call)."""
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = None
            self._ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self._ws

    def release_workspace(self) -> None:
        """Hand the kept scratch of long calls back to torch's allocator."""
        self._ws = None

    def check_full(self):
        """Raise like the reference (code/lema/csrc/store.cpp:159-160) if some key since the
        last clear found no free slot; clears the flag."""
        full = bool(self.full_flag.item())
        self.full_flag.zero_()
        if full:
            raise RuntimeError(_lib.FULL_MESSAGE)

    def dump(self):
        """The published entries (group, code, value rows), on the table's side (host tensors
        for a table in RAM): the table read the way
        code/experiments/app_retrieval/fixedpoint.py:72-82 reads the reference's."""
        if self._host is not None:
            torch.cuda.synchronize(self.device)   # the kernels write host memory in place
        words = self.table[:, :16].contiguous().view(torch.int64).view(self.cap, 2)
        state = words[:, 1]
        live = state >= 2
        return state[live] - 2, words[live, 0], self.table[live, 16:]


class LayerStore:
    """One layer's view of the cache: its slice of partitions in the shared store
    (code/lema/cache.py:248-302). `exchange(qc, kc, v)` is what a LEMA block is handed: the
    `[B, H, T]` codes and `[B, H, T, d_v]` values flatten partition-major, position-minor
    (partition b * H + h, group g0 + partition); the retrieved values come back like `v`, zeros
    where nothing matched -- with no staging through host memory."""

    __slots__ = ("store", "g0", "partitions", "codes_hook", "layer_index")

    def __init__(self, store: HashStore, g0: int, partitions: int, codes_hook=None,
                 layer_index: int = 0):
        self.store, self.g0, self.partitions = store, g0, partitions
        self.codes_hook, self.layer_index = codes_hook, layer_index

    def exchange(self, qc: torch.Tensor, kc: torch.Tensor, v: torch.Tensor,
                 check: bool = True) -> torch.Tensor:
        if self.codes_hook is not None:       # on the device, inside a captured step
            qc, kc = self.codes_hook(self.layer_index, qc, kc)
        n, d_v = qc.numel(), v.shape[-1]
        got = torch.empty(v.shape, dtype=v.dtype, device=v.device)
        self.store.exchange(qc.reshape(-1), kc.reshape(-1), v.reshape(-1, d_v),
                            got.view(-1, d_v), n // self.partitions, self.g0, check=check)
        return got


class LemaCache:
    """The retrieval state of a model: one shared table, viewed per layer
    (code/lema/cache.py:305-378), in device memory (place "hbm") or host RAM ("ram"). Sized
    once: `capacity` slots, or ceil(depth * batch * heads * max_cache_len / max_load) for the
    worst case of one new code per token per head; it never resizes."""

    def __init__(self, cfg, dtype=torch.bfloat16, pin: bool = True, max_cache_len: int = 8192,
                 max_load: float = 0.7, batch: int = 1, capacity: int | None = None,
                 codes_hook=None, device=None, place: str = "hbm"):
        if dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise ValueError(f"cache dtype must be one of "
                             f"{[torch.float32, torch.float16, torch.bfloat16]}, got {dtype}")
        if not 0 < max_load <= 0.95:
            raise ValueError(f"max_load must be in (0, 0.95], got {max_load}")
        P = batch * cfg.num_heads
        slots = int(capacity) if capacity else math.ceil(cfg.depth * P * max_cache_len
                                                         / max_load)
        self.cfg, self.batch, self.dtype = cfg, batch, dtype
        self.store = HashStore(cfg.d_v, groups=cfg.depth * P, dtype=dtype, capacity=slots,
                               device=device, place=place)
        self.t = 0
        self.codes_hook = codes_hook
        self._views = [LayerStore(self.store, i * P, P, codes_hook, i) for i in range(cfg.depth)]

    def layer(self, i: int) -> LayerStore:
        return self._views[i]

    def counts(self) -> torch.Tensor:
        """Entries per partition as `[depth, batch, heads]` (host copy)."""
        return self.store.counts.view(self.cfg.depth, self.batch, self.cfg.num_heads)

    def entries(self) -> int:
        return len(self.store)

    def nbytes(self) -> int:
        return self.store.nbytes()

    def load(self) -> float:
        return self.store.load()
