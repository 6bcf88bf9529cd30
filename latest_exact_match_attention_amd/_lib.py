"""ctypes binding of liblema_hip.so (the C ABI declared in include/lema_hip.h).

The library is the only compute path: there is no CPU or eager-torch fallback. If it has not
been built, `lib()` raises and names the build command.
"""
from __future__ import annotations

import ctypes
import weakref
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "liblema_hip.so"
# the diagnostics build (decode-step clock readings); loaded only when a caller asks for it
STAMPS_LIB_PATH = Path(__file__).resolve().parent / "liblema_hip_stamps.so"

OK, TABLE_FULL, BAD_ARG, HIP_ERROR = 0, 1, 2, 3
F32, F16, BF16 = 0, 1, 2
MISS_DENSE, MISS_ZERO = 0, 1
NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024   # LEMA_NOALLOC_SCRATCH_BYTES of the header

DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

FULL_MESSAGE = "hash table full: the store is presized and never grows -- provision more capacity"

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64

# name -> argument types, exactly the prototypes of include/lema_hip.h
PROTOTYPES = {
    "lema_last_error": ([], ctypes.c_char_p),
    "lema_abi_version": ([], ctypes.c_int),
    "lema_device_copy": ([_p, _p, _i64, _p], ctypes.c_int),
    "lema_pack_codes": ([_p, _i32, _i64, _i64, _i64, _i32, _i64, _i64, _i64, _p, _i32, _p],
                        ctypes.c_int),
    "lema_latest_prev_match": ([_p, _p, _i32, _i64, _i64, _p, _i32, _p], ctypes.c_int),
    "lema_hard": ([_p, _p, _i32, _p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64,
                   _i64, _i64, _i32, _p, _i32, _p], ctypes.c_int),
    "lema_latest_prev_match_ws": ([_p, _p, _i32, _i64, _i64, _p, _i32, _p, _i64, _p],
                                  ctypes.c_int),
    "lema_resolve_workspace_bytes": ([_i64, _i64], ctypes.c_int64),
    "lema_hard_ws": ([_p, _p, _i32, _p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p,
                      _i64, _i64, _i64, _i32, _p, _i32, _p, _i64, _p], ctypes.c_int),
    "lema_gather": ([_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i32, _p, _i64,
                     _i64, _i64, _i32, _p], ctypes.c_int),
    "lema_store_exchange": ([_p, _i64, _i64, _p, _p, _i32, _p, _p, _i64, _i64, _i64, _p, _p, _p],
                            ctypes.c_int),
    "lema_store_workspace_bytes": ([_i64, _i64, _i32], ctypes.c_int64),
    "lema_swiglu_bf16": ([_p, _p, _p, _i64, _p], ctypes.c_int),
    "lema_rmsnorm_bf16": ([_p, _p, _p, ctypes.c_float, _i64, _i64, _p, _p, _p], ctypes.c_int),
    "lema_argmax_bf16": ([_p, _i64, _i64, _i64, _p, _i64, _p], ctypes.c_int),
    "lema_embedding_bf16": ([_p, _i64, _i64, _p, _i64, _p, _p], ctypes.c_int),
    "lema_cross_entropy_bf16": ([_p, _i64, _i64, _i64, _p, _p, _p], ctypes.c_int),
    "lema_skinny_gemm_bf16": ([_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p], ctypes.c_int),
    "lema_skinny_pack_bf16": ([_p, _i64, _p, _i64, _i64, _i64, _i64, _i32, _i64, _p, _i32, _p],
                              ctypes.c_int),
    "lema_qk_pack_bf16": ([_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32, _i64, _p, _p, _i32,
                           _p], ctypes.c_int),
    "lema_skinny_gemm_add_bf16": ([_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p],
                                  ctypes.c_int),
    "lema_skinny_qkv_bf16": ([_p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i64,
                              _p, _p, _i32, _p, _p], ctypes.c_int),
    "lema_skinny_swiglu_bf16": ([_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _p], ctypes.c_int),
    "lema_skinny_norm_swiglu_bf16": ([_p, _p, _p, ctypes.c_float, _p, _p, _p, _i64, _i64, _i64,
                                      _i64, _p, _p], ctypes.c_int),
    "lema_skinny_norm_qkv_bf16": ([_p, _p, ctypes.c_float, _p, _p, _p, _i64, _i64, _i64, _i64,
                                   _i64, _i32, _i64, _p, _p, _i32, _p, _p], ctypes.c_int),
    "lema_store_exchange_noalloc": ([_p, _i64, _i64, _p, _p, _i32, _p, _p, _i64, _i64, _i64, _p,
                                     _p, _p], ctypes.c_int),
    "lema_store_exchange_ws": ([_p, _i64, _i64, _p, _p, _i32, _p, _p, _i64, _i64, _i64, _p, _p,
                                _p, _i64, _p], ctypes.c_int),
}

_LIB = None


def use_stamps_library() -> ctypes.CDLL:
    """Load the diagnostics build in place of the product library (before any other use of
    the library in this process): the same kernels, with the decode step's clock readings."""
    global _LIB, LIB_PATH
    if _LIB is not None and LIB_PATH != STAMPS_LIB_PATH:
        raise RuntimeError("the product library is already loaded in this process")
    LIB_PATH = STAMPS_LIB_PATH
    L = lib()
    L.lema_debug_step_stamps.argtypes = [_p]
    L.lema_debug_step_stamps.restype = None
    L.lema_debug_empty_step.argtypes = [_i64, _p]
    L.lema_debug_empty_step.restype = ctypes.c_int
    return L


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built: the LEMA kernels have no fallback. Build it "
                f"with `python -m latest_exact_match_attention_amd.build` (hipcc, gfx950).")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in PROTOTYPES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _LIB = L
    return _LIB


def check(status: int) -> None:
    """Map a library status to the exception the reference raises for the same failure."""
    if status == OK:
        return
    msg = (lib().lema_last_error() or b"").decode(errors="replace")
    if status == TABLE_FULL:
        raise RuntimeError(FULL_MESSAGE)
    if status == BAD_ARG:
        raise ValueError(msg)
    raise RuntimeError(f"HIP error in liblema_hip: {msg}")


def stream_of(t: torch.Tensor) -> int:
    """The raw hipStream_t of the current torch stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


# ---- host memory the GPU works on in place (a store table in host RAM) ----
# The HIP runtime this process already uses (torch's; the library links the same soname).
_HIP = None
HIP_HOST_MALLOC_COHERENT = 0x40000000        # hipHostMallocCoherent
HIP_ATTR_HOST_NATIVE_ATOMIC = 15             # hipDeviceAttributeHostNativeAtomicSupported


def hip_runtime() -> ctypes.CDLL:
    global _HIP
    if _HIP is None:
        torch.cuda.init()
        H = ctypes.CDLL("libamdhip64.so.7")
        H.hipHostMalloc.argtypes = [ctypes.POINTER(_p), ctypes.c_size_t, ctypes.c_uint]
        H.hipHostFree.argtypes = [_p]
        H.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(_p), _p, ctypes.c_uint]
        H.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                            ctypes.c_int]
        for f in ("hipHostMalloc", "hipHostFree", "hipHostGetDevicePointer",
                  "hipDeviceGetAttribute"):
            getattr(H, f).restype = ctypes.c_int
        _HIP = H
    return _HIP


def host_atomics_supported(device: int) -> bool:
    """Whether the link between `device` and the host carries the device's atomic operations
    on host memory (a claim in a host-RAM table is a 64-bit compare-and-swap)."""
    v = ctypes.c_int(0)
    rc = hip_runtime().hipDeviceGetAttribute(ctypes.byref(v), HIP_ATTR_HOST_NATIVE_ATOMIC,
                                             device)
    return rc == 0 and v.value == 1


class HostTable:
    """`nbytes` of zeroed, pinned, coherent host memory that the GPU reads, writes and updates
    atomically in place (no copies), freed with the object. `tensor()` views it from the CPU;
    `dev_ptr` is the address kernels use."""

    def __init__(self, nbytes: int):
        H = hip_runtime()
        ptr = _p()
        rc = H.hipHostMalloc(ctypes.byref(ptr), max(1, nbytes), HIP_HOST_MALLOC_COHERENT)
        if rc != 0 or not ptr.value:
            raise RuntimeError(f"hipHostMalloc of {nbytes} bytes failed (status {rc})")
        self.ptr, self.nbytes = ptr.value, nbytes
        self._finalizer = weakref.finalize(self, H.hipHostFree, ptr.value)
        ctypes.memset(self.ptr, 0, nbytes)
        dev = _p()
        rc = H.hipHostGetDevicePointer(ctypes.byref(dev), ptr.value, 0)
        if rc != 0 or not dev.value:
            raise RuntimeError(f"hipHostGetDevicePointer failed (status {rc})")
        self.dev_ptr = dev.value
        self._buf = (ctypes.c_uint8 * nbytes).from_address(self.ptr)

    def tensor(self) -> torch.Tensor:
        return torch.frombuffer(self._buf, dtype=torch.uint8)


def widen_codes(t: torch.Tensor) -> torch.Tensor:
    """Codes in the int64 carrier, for calls that mix widths. An int32 code stands for its
    32-bit pattern, which the kernels read as an unsigned word (a d_qk <= 32 code of the
    reference is an int64 below 2^32), so it is zero-extended, never sign-extended."""
    if t.dtype == torch.int64:
        return t
    if t.dtype == torch.int32:
        return t.to(torch.int64) & 0xFFFFFFFF
    return t.to(torch.int64)


def require_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise TypeError("liblema_hip runs on HIP devices only: got a tensor on "
                            f"{t.device}; move the inputs to the GPU")
