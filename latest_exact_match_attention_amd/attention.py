"""The exact LEMA op on MI355X: the reference's `pack_codes`, `latest_prev_match` and
`lema_hard` (code/lema/attention.py:82-158) with the same names, arguments, results and
errors, computed by the HIP kernels of liblema_hip.so.

Conventions (code/lema/attention.py:3-8): codes are sign patterns with sign(0) := +1; the
match is STRICTLY causal (a query never matches its own key); no match => output 0.
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["pack_codes", "latest_prev_match", "lema_hard", "lema_from_codes", "gather_values",
           "resolve_workspace",
           "code_dtype_for"]


def code_dtype_for(d_qk: int) -> torch.dtype:
    """The narrowest code carrier: int32 holds the 32-bit pattern for d_qk <= 32."""
    return torch.int32 if d_qk <= 32 else torch.int64


def _rows4(z: torch.Tensor) -> torch.Tensor:
    """z as a [B, H, T, D] view with a contiguous last dim (copying only if it must)."""
    if z.dim() == 4 and (z.stride(-1) == 1 or z.shape[-1] == 1):
        return z
    if z.dim() == 4:
        return z.contiguous()
    return z.reshape(1, 1, -1, z.shape[-1])


def pack_codes(z: torch.Tensor, code_dtype: torch.dtype = torch.int64) -> torch.Tensor:
    """[..., D] -> one integer code per row, on z's device (code/lema/attention.py:82-97).

    Bit j is set iff z[..., j] >= 0, so raw pre-activations and +-1 codes give the same
    code; -0.0 sets the bit and NaN does not. D <= 64; at D == 64 the top bit is the int64
    sign bit, as in the reference. `code_dtype` int32 (D <= 32) returns the same bit pattern
    in a 4-byte carrier, which the kernels here read faster.
    """
    D = z.shape[-1]
    if D > 64:
        raise ValueError(f"d_qk {D} > 64 cannot pack into a uint64")
    if code_dtype not in (torch.int64, torch.int32):
        raise ValueError(f"code_dtype must be torch.int64 or torch.int32, got {code_dtype}")
    if code_dtype == torch.int32 and D > 32:
        raise ValueError(f"d_qk {D} > 32 does not fit an int32 code")
    _lib.require_device(z)
    if z.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"pack_codes takes float32, float16 or bfloat16, got {z.dtype}")
    out = torch.empty(z.shape[:-1], dtype=code_dtype, device=z.device)
    if out.numel() == 0:
        return out
    if D == 0:
        return out.zero_()
    z4 = _rows4(z)
    B, H, T, _ = z4.shape
    cb = 4 if code_dtype == torch.int32 else 8
    _lib.check(_lib.lib().lema_pack_codes(
        z4.data_ptr(), _lib.DTYPE_CODE[z.dtype], B, H, T, D, z4.stride(0), z4.stride(1),
        z4.stride(2), out.data_ptr(), cb, _lib.stream_of(z)))
    return out


def _codes_pair(qc: torch.Tensor, kc: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, int]:
    if qc.shape != kc.shape:
        raise ValueError(f"query and key codes differ in shape: {tuple(qc.shape)} vs "
                         f"{tuple(kc.shape)}")
    if qc.dtype != kc.dtype:
        qc, kc = _lib.widen_codes(qc), _lib.widen_codes(kc)
    if qc.dtype not in (torch.int64, torch.int32, torch.uint32, torch.uint64):
        raise TypeError(f"codes must be int64 or int32, got {qc.dtype}")
    return qc.contiguous(), kc.contiguous(), qc.element_size()


def latest_prev_match(qc: torch.Tensor, kc: torch.Tensor,
                      out_dtype: torch.dtype = torch.int64) -> torch.Tensor:
    """For each i, the largest j < i with kc[j] == qc[i], else -1
    (code/lema/attention.py:100-132).

    qc, kc: [N, T] integer codes, N independent streams (batch x heads). Returns [N, T]
    int64 like the reference (`out_dtype=torch.int32` halves the index bytes).
    """
    if qc.dim() != 2:
        raise ValueError(f"codes must be [N, T], got shape {tuple(qc.shape)}")
    _lib.require_device(qc, kc)
    qc, kc, cb = _codes_pair(qc, kc)
    N, T = qc.shape
    if out_dtype not in (torch.int64, torch.int32):
        raise ValueError("out_dtype must be torch.int64 or torch.int32")
    src = torch.empty((N, T), dtype=out_dtype, device=qc.device)
    if src.numel() == 0:
        return src
    ws = resolve_workspace(N, T, qc.device)
    _lib.check(_lib.lib().lema_latest_prev_match_ws(
        qc.data_ptr(), kc.data_ptr(), cb, N, T, src.data_ptr(), src.element_size(),
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _lib.stream_of(qc)))
    return src


def resolve_workspace(N: int, T: int, device) -> torch.Tensor | None:
    """Scratch for the chunk summaries of N rows of T positions (None when rows are short
    enough for the backward scan): 8 KB per 1024 positions."""
    n = _lib.lib().lema_resolve_workspace_bytes(N, T)
    return torch.empty(n, dtype=torch.uint8, device=device) if n > 0 else None


def _value4(v: torch.Tensor) -> torch.Tensor:
    if v.dim() != 4:
        raise ValueError(f"values must be [B, H, T, d_v], got shape {tuple(v.shape)}")
    if v.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"values must be float32, float16 or bfloat16, got {v.dtype}")
    return v if v.stride(-1) == 1 or v.shape[-1] == 1 else v.contiguous()


def _hard_forward(qc: torch.Tensor, kc: torch.Tensor, v: torch.Tensor,
                  want_src: bool) -> tuple[torch.Tensor, torch.Tensor | None]:
    """The fused resolve + gather kernel: y (laid out like v) and optionally src int32."""
    B, H, T, dv = v.shape
    qc, kc, cb = _codes_pair(qc.reshape(B * H, T), kc.reshape(B * H, T))
    y = torch.empty_like(v)
    if y.stride(-1) != 1 and dv > 1:
        y = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    src = torch.empty((B, H, T), dtype=torch.int32, device=v.device) if want_src else None
    if y.numel() == 0:
        if src is not None:
            src.fill_(-1)
        return y, src
    launch_hard(qc, kc, v, y, src)
    return y, src


def launch_hard(qc: torch.Tensor, kc: torch.Tensor, v: torch.Tensor, y: torch.Tensor,
                src: torch.Tensor | None = None, miss: int = _lib.MISS_DENSE,
                workspace: torch.Tensor | None = None) -> None:
    """Enqueue the fused kernels on preallocated buffers: qc, kc contiguous [B*H, T] (int32 or
    int64), v and y [B, H, T, dv] with a contiguous last dim, src None or contiguous
    int32/int64 [B, H, T], workspace None or `resolve_workspace(B*H, T)` (allocated here when
    needed and not given; pass it to keep the call allocation-free)."""
    B, H, T, dv = v.shape
    cb = qc.element_size()
    ws = workspace if workspace is not None else resolve_workspace(B * H, T, v.device)
    _lib.check(_lib.lib().lema_hard_ws(
        qc.data_ptr(), kc.data_ptr(), cb, v.data_ptr(), _lib.DTYPE_CODE[v.dtype], B, H, T, dv,
        v.stride(0), v.stride(1), v.stride(2), y.data_ptr(), y.stride(0), y.stride(1),
        y.stride(2), miss, src.data_ptr() if src is not None else None,
        src.element_size() if src is not None else 4,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _lib.stream_of(v)))


def lema_from_codes(qc: torch.Tensor, kc: torch.Tensor, v: torch.Tensor,
                    return_src: bool = False):
    """`lema_hard` after pack_codes (code/lema/attention.py:155-158), from [B, H, T] codes:
    y = v[latest match] with the dense path's miss fill. With `return_src` also the int32
    match indices [B, H, T] (-1 = no match). No gradient."""
    v = _value4(v)
    _lib.require_device(qc, kc, v)
    if qc.shape != v.shape[:3]:
        raise ValueError(f"codes {tuple(qc.shape)} do not match values {tuple(v.shape)}")
    y, src = _hard_forward(qc, kc, v, want_src=return_src)
    return (y, src) if return_src else y


def gather_values(v: torch.Tensor, src: torch.Tensor, miss: str = "dense") -> torch.Tensor:
    """y[b, h, i] = v[b, h, src[b, h, i]] (code/lema/attention.py:157-158). A miss (-1) is
    v[b, h, 0] * 0 for miss="dense" and +0 for miss="zero" (the store path,
    code/lema/csrc/store.cpp:92). Indices must lie in [-1, T)."""
    v = _value4(v)
    _lib.require_device(v, src)
    B, H, T, dv = v.shape
    if src.shape != (B, H, T):
        raise ValueError(f"src {tuple(src.shape)} does not match values {tuple(v.shape)}")
    if miss not in ("dense", "zero"):
        raise ValueError(f"miss must be 'dense' or 'zero', got {miss!r}")
    if src.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"src must be int32 or int64, got {src.dtype}")
    src = src.contiguous()
    if src.numel() and (int(src.min()) < -1 or int(src.max()) >= T):
        raise ValueError(f"src entries must lie in [-1, {T})")
    y = torch.empty_like(v)
    if y.stride(-1) != 1 and dv > 1:
        y = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    if y.numel() == 0:
        return y
    _lib.check(_lib.lib().lema_gather(
        v.data_ptr(), _lib.DTYPE_CODE[v.dtype], B, H, T, dv, v.stride(0), v.stride(1),
        v.stride(2), src.data_ptr(), src.element_size(), y.data_ptr(), y.stride(0),
        y.stride(1), y.stride(2), _lib.MISS_DENSE if miss == "dense" else _lib.MISS_ZERO,
        _lib.stream_of(v)))
    return y


class _LemaGather(torch.autograd.Function):
    """The value path stays differentiable (code/lema/attention.py:146-148): the gradient
    of y = v[src] * (src >= 0) sends each dy row to its source row."""

    @staticmethod
    def forward(ctx, qc, kc, v):
        y, src = _hard_forward(qc, kc, v, want_src=True)
        ctx.save_for_backward(src)
        ctx.v_shape = v.shape
        return y

    @staticmethod
    def backward(ctx, gy):
        (src,) = ctx.saved_tensors
        B, H, T, dv = ctx.v_shape
        hit = (src >= 0).unsqueeze(-1)
        idx = src.clamp_min(0).to(torch.int64).view(B * H, T, 1).expand(B * H, T, dv)
        gv = torch.zeros((B * H, T, dv), dtype=gy.dtype, device=gy.device)
        gv.scatter_add_(1, idx, (gy * hit).reshape(B * H, T, dv))
        return None, None, gv.view(B, H, T, dv)


def lema_hard(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, store=None) -> torch.Tensor:
    """Exact latest match: o_i = v_j for the largest j < i with k_j == q_i, else 0
    (code/lema/attention.py:135-158).

    q, k: [B, H, T, d_qk] pre-activations or +-1 codes; v: [B, H, T, d_v]. Without a store
    the window is resolved and gathered by one fused kernel; a miss yields v[b, h, 0] * 0
    like the reference's dense path. With a `store` the codes are exchanged against it
    (looked up, then inserted, in position order) and it returns the values.
    """
    B, H, T, D = q.shape
    if D > 64:
        raise ValueError(f"d_qk {D} > 64 cannot pack into a uint64")
    with torch.no_grad():
        ct = code_dtype_for(D)
        qc, kc = pack_codes(q, ct), pack_codes(k, ct)
    if store is not None:
        return store.exchange(qc, kc, v)
    v = _value4(v)
    if v.shape[:3] != (B, H, T):
        raise ValueError(f"values {tuple(v.shape)} do not match codes {(B, H, T)}")
    _lib.require_device(v)
    if v.requires_grad and torch.is_grad_enabled():
        return _LemaGather.apply(qc, kc, v)
    y, _ = _hard_forward(qc, kc, v, want_src=False)
    return y
