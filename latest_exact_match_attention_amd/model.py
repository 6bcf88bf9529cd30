"""The LEMA transformer on MI355X: the reference's `ModelConfig` / `Transformer`
(code/lema/model.py) for an all-LEMA model in hard mode, the configuration in which the
exact op runs and a retrieval cache can be attached.

Pre-RMSNorm, SwiGLU MLP, untied head, no biases, no positional encoding
(code/lema/model.py:1-9). The projections, MLP and head are bf16 (or fp32) GEMMs on the
matrix cores through torch; the attention of every block is the exact op of this package
(sign-pack, latest-match resolve and gather in HIP), and a cached forward exchanges each
layer's codes against the HBM store with no host round trip.

Parameters are created and initialised in the reference's module order (embedding, then per
block norm1, q, k, v, o, norm2, gate, up, down, then norm_f, lm_head; Gaussian std
1/sqrt(fan_in) for every Linear and 1/sqrt(dim) for the embedding, the two residual-branch
outputs scaled by 1/sqrt(2 * depth): code/lema/model.py:258-281), so the same seed gives the
same weights.

In bf16 on the GPU the SwiGLU product, both pre-norms (the MLP's with the attention residual
add), the final norm and the loss run as fused HIP kernels (the reference compiles these
segments with torch.compile). The norm kernel rounds like torch's RMSNorm (one rounding of
x * rstd * w from fp32) but adds up the mean of squares in its own order, so a rare element
of the attention input lands one bf16 ulp from torch's. The codes, the signs of that input's
projections, can then differ from the ones torch's norm gives, only at pre-activations
within 1e-3 of zero (the stated binarization tolerance; at the full LM shape 9 of 1e8 code
bits of the first layer).

Only the hard (exact) op is implemented: the training surrogate (stick-breaking relaxation,
straight-through binarization) and the softmax / gated-deltanet baselines are not part of the
exact-match path.
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from .attention import code_dtype_for, lema_from_codes, lema_hard, pack_codes

__all__ = ["ModelConfig", "SwiGLU", "Attention", "Block", "Transformer", "lm_loss", "rms_norm",
           "embed", "argmax_into", "load_trained",
           "swiglu", "cross_entropy_sum"]

# ------------------------------------------------------------------ fused bf16 segments
# On the GPU in bf16 the SwiGLU product, the residual add with the next pre-norm, and the loss
# run as one HIP kernel each (liblema_hip.so); other dtypes and devices use the torch ops.

def _fused(*ts: torch.Tensor) -> bool:
    return all(t.is_cuda and t.dtype == torch.bfloat16 and t.is_contiguous() for t in ts)


def rms_norm(x: torch.Tensor, norm: nn.RMSNorm, d: torch.Tensor | None = None):
    """norm(x + d) and x + d (or norm(x), x when d is None), one pass in bf16."""
    if d is not None and not (_fused(x, d) and _fused(norm.weight)):
        x, d = x + d, None
    if not (_fused(x) and _fused(norm.weight) and x.shape[-1] % 8 == 0
            and x.shape[-1] <= 4096):
        return norm(x), x
    D = x.shape[-1]
    h = torch.empty_like(x)
    xo = torch.empty_like(x) if d is not None else x
    eps = norm.eps if norm.eps is not None else torch.finfo(x.dtype).eps
    _lib.check(_lib.lib().lema_rmsnorm_bf16(
        x.data_ptr(), d.data_ptr() if d is not None else None, norm.weight.data_ptr(),
        float(eps), x.numel() // D, D, xo.data_ptr() if d is not None else None, h.data_ptr(),
        _lib.stream_of(x)))
    return h, xo


def embed(emb: nn.Embedding, ids: torch.Tensor) -> torch.Tensor:
    """emb(ids) for a decode step: bf16 rows gathered by one workgroup each. The ids must lie
    in [0, vocab) (an id outside it gives a zero row where nn.Embedding raises)."""
    w = emb.weight
    if not (_fused(w) and ids.is_cuda and ids.dtype == torch.long and ids.is_contiguous()
            and w.shape[1] % 8 == 0 and w.data_ptr() % 16 == 0):
        return emb(ids)
    out = torch.empty(ids.shape + (w.shape[1],), dtype=w.dtype, device=w.device)
    _lib.check(_lib.lib().lema_embedding_bf16(w.data_ptr(), w.shape[0], w.shape[1],
                                              ids.data_ptr(), ids.numel(), out.data_ptr(),
                                              _lib.stream_of(w)))
    return out


def argmax_into(logits: torch.Tensor, out: torch.Tensor) -> None:
    """out[...] = logits.argmax(-1) (the first index of the maximum, NaN above every number),
    written in place: one workgroup per row of bf16 logits."""
    V = logits.shape[-1]
    if not (_fused(logits) and V % 8 == 0 and logits.data_ptr() % 16 == 0 and out.is_cuda
            and out.dtype == torch.long and out.is_contiguous()
            and out.numel() == logits.numel() // V):
        out.copy_(logits.argmax(-1).view(out.shape))
        return
    _lib.check(_lib.lib().lema_argmax_bf16(logits.data_ptr(), logits.numel() // V, V, V,
                                           out.data_ptr(), 1, _lib.stream_of(logits)))


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    if not (_fused(g, u) and g.numel() % 8 == 0):
        return F.silu(g) * u
    out = torch.empty_like(g)
    _lib.check(_lib.lib().lema_swiglu_bf16(g.data_ptr(), u.data_ptr(), out.data_ptr(),
                                           g.numel(), _lib.stream_of(g)))
    return out


def cross_entropy_sum(logits: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Sum over rows of logsumexp(logits) - logits[y] (fp32)."""
    V = logits.shape[-1]
    if not (_fused(logits) and V % 8 == 0 and y.is_cuda):
        return F.cross_entropy(logits.float(), y, reduction="sum")
    rows = logits.numel() // V
    loss = torch.empty(rows, dtype=torch.float32, device=logits.device)
    yy = y.reshape(-1).to(torch.int64).contiguous()
    _lib.check(_lib.lib().lema_cross_entropy_bf16(
        logits.data_ptr(), rows, V, V, yy.data_ptr(), loss.data_ptr(), _lib.stream_of(logits)))
    return loss.sum()


SKINNY_ROWS = 32  # products with at most this many token rows run on the skinny MFMA kernel


def _skinny(x: torch.Tensor, weight: torch.Tensor) -> bool:
    K = x.shape[-1]
    return (_fused(x, weight) and K % 32 == 0 and 0 < x.numel() // K <= SKINNY_ROWS
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


def linear(x: torch.Tensor, lin: nn.Linear) -> torch.Tensor:
    """lin(x); a decode-shaped product (<= 32 rows, bf16) on the skinny MFMA kernel."""
    if not _skinny(x, lin.weight):
        return lin(x)
    K, N = x.shape[-1], lin.weight.shape[0]
    M = x.numel() // K
    y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
    _lib.check(_lib.lib().lema_skinny_gemm_bf16(
        x.data_ptr(), K, lin.weight.data_ptr(), K, y.data_ptr(), N, M, N, K, _lib.stream_of(x)))
    return y


def project_codes(x: torch.Tensor, lin: nn.Linear, d: int, code_dtype: torch.dtype):
    """[B, T, dim] -> [B, H, T] codes of lin(x) viewed as H heads of d, or None when the
    shape is not decode-sized (the caller then projects and packs)."""
    if not (_skinny(x, lin.weight) and x.dim() == 3 and _pack_tiles(d)):
        return None
    B, T, K = x.shape
    N = lin.weight.shape[0]
    codes = torch.empty((B, N // d, T), dtype=code_dtype, device=x.device)
    _lib.check(_lib.lib().lema_skinny_pack_bf16(
        x.data_ptr(), K, lin.weight.data_ptr(), K, B * T, N, K, d, T, codes.data_ptr(),
        codes.element_size(), _lib.stream_of(x)))
    return codes


def _pack_tiles(d: int) -> bool:
    """Whether the skinny kernel packs d-bit codes: heads split over 16-column blocks when d
    is a multiple of 8, else whole heads in blocks of up to 64 columns."""
    return d % 8 == 0 or any((16 * c) % d == 0 for c in (1, 2, 3, 4))


def project_qkv(x: torch.Tensor, at, code_dtype: torch.dtype, norm: nn.RMSNorm | None = None):
    """[B, T, dim] -> (qc, kc [B, H, T] codes, v [B, H, T, d_v] view) with all three
    projections in one launch (skinny MFMA kernel, pack epilogues for q and k), or None when
    the shape is not decode-sized or the heads differ in count. With `norm`, x is the layer's
    input and the launch normalises it first, rounded as rms_norm rounds it (the same codes and
    v as rms_norm followed by this, with one launch fewer); None also where that does not
    apply."""
    c = at.cfg
    wq, wk, wv = at.q_proj.weight, at.k_proj.weight, at.v_proj.weight
    if not (_skinny(x, wq) and x.dim() == 3 and wq.shape == wk.shape and _pack_tiles(c.d_qk)
            and wk.data_ptr() % 16 == 0 and wv.data_ptr() % 16 == 0
            and wv.dtype == wq.dtype and wv.is_contiguous() and wk.is_contiguous()):
        return None
    B, T, K = x.shape
    Nqk, Nv = wq.shape[0], wv.shape[0]
    if norm is not None:
        M = B * T
        ct = 1 if c.d_qk % 8 == 0 else next(k for k in range(1, 5) if (16 * k) % c.d_qk == 0)
        if not (_fused(norm.weight) and norm.weight.data_ptr() % 16 == 0 and x.is_contiguous()
                and K <= 2048
                and M * (K + 8) * 2 + 8 * (16 if M <= 16 else 32) * (16 * ct + 1) * 4 <= 160 * 1024):
            return None
    qc = torch.empty((B, Nqk // c.d_qk, T), dtype=code_dtype, device=x.device)
    kc = torch.empty_like(qc)
    v = torch.empty((B, T, Nv), dtype=x.dtype, device=x.device)
    if norm is not None:
        eps = norm.eps if norm.eps is not None else torch.finfo(x.dtype).eps
        _lib.check(_lib.lib().lema_skinny_norm_qkv_bf16(
            x.data_ptr(), norm.weight.data_ptr(), float(eps), wq.data_ptr(), wk.data_ptr(),
            wv.data_ptr(), K, B * T, Nqk, Nv, K, c.d_qk, T, qc.data_ptr(), kc.data_ptr(),
            qc.element_size(), v.data_ptr(), _lib.stream_of(x)))
    else:
        _lib.check(_lib.lib().lema_skinny_qkv_bf16(
            x.data_ptr(), K, wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), K, B * T, Nqk, Nv, K,
            c.d_qk, T, qc.data_ptr(), kc.data_ptr(), qc.element_size(), v.data_ptr(),
            _lib.stream_of(x)))
    return qc, kc, v.view(B, T, c.num_kv_heads, c.d_v).transpose(1, 2)


# Rows of a prefill projection taken by lema_qk_pack_bf16 (q and k straight to codes): its
# 256 x 256 tiles cover the rows in 8 row groups, one per XCD.
QK_PACK_ROWS = 2048
# Whether the model's prefill takes its q and k codes from lema_qk_pack_bf16 (the codes are
# identical either way). Off: on the 4 x 16384-token, dim-1536 prefill the launch takes
# 494.5-541 us against 526-560 us for the two hipBLASLt GEMMs and two packs when timed alone,
# but 572 us against 525 us inside the forward, where both run at the clock a sustained matrix
# load holds (it spends ~30% more cycles per FLOP than the library's GEMMs); the forward's step
# time is the same with it on or off (114.5-114.8 ms).
FUSED_QK_PACK = False


def project_qk_prefill(x: torch.Tensor, at, code_dtype: torch.dtype):
    """[B, T, dim] -> (qc, kc [B, H, T] codes) of a prefill-sized input (B * T a multiple of
    2048 rows, bf16, no autograd): the query and key projections and the sign-pack in one
    persistent MFMA launch whose epilogue writes the codes, so the pre-activations zq and zk
    never reach memory. The same codes as project + pack_codes (bit j = bf16(z_j) >= 0); None
    where the launch does not apply (the caller then projects and packs)."""
    c = at.cfg
    wq, wk = at.q_proj.weight, at.k_proj.weight
    if torch.is_grad_enabled() and (x.requires_grad or wq.requires_grad or wk.requires_grad):
        return None
    if not (_fused(x, wq, wk) and x.dim() == 3 and wq.shape == wk.shape):
        return None
    B, T, K = x.shape
    N, d = wq.shape[0], c.d_qk
    cb = torch.iinfo(code_dtype).bits // 8
    if ((B * T) % QK_PACK_ROWS or N % 256 or N > 65536 or K % 64 or d % 8 or d > 64 or N % d
            or cb != (4 if d <= 32 else 8) or B * T * (N // d) * cb >= 1 << 31
            or x.data_ptr() % 16 or wq.data_ptr() % 16 or wk.data_ptr() % 16):
        return None
    qc = torch.empty((B, N // d, T), dtype=code_dtype, device=x.device)
    kc = torch.empty_like(qc)
    _lib.check(_lib.lib().lema_qk_pack_bf16(
        x.data_ptr(), K, wq.data_ptr(), wk.data_ptr(), K, B * T, N, K, d, T, qc.data_ptr(),
        kc.data_ptr(), qc.element_size(), _lib.stream_of(x)))
    return qc, kc


ATTN_KINDS = ("lema",)
POS_KINDS = ("nope",)


def _pad128(n) -> int:
    return -(-int(n) // 128) * 128


@dataclass
class ModelConfig:
    """Geometry of a LEMA model (code/lema/model.py:33-82). `d_qk`, `d_v` default to
    dim // num_heads, `dim_ff` to 8 * dim / 3; `vocab_size` and `dim_ff` are rounded up to a
    multiple of 128 (the padded vocabulary rows are never targets)."""
    vocab_size: int
    depth: int
    dim: int
    num_heads: int
    d_qk: int = 0
    d_v: int = 0
    dim_ff: int = 0
    num_kv_heads: int = 0
    attn: str = "lema"
    pos: str = "nope"
    norm_eps: float = 1e-5

    def __post_init__(self):
        if self.attn not in ATTN_KINDS:
            raise ValueError(f"attn must be one of {ATTN_KINDS} (the exact-match path), "
                             f"got {self.attn!r}")
        if self.pos not in POS_KINDS:
            raise ValueError(f"pos must be one of {POS_KINDS}, got {self.pos!r}")
        if (not self.d_qk or not self.d_v) and self.dim % self.num_heads:
            raise ValueError(f"dim {self.dim} is not divisible by num_heads {self.num_heads}")
        head = self.dim // self.num_heads
        self.d_qk = self.d_qk or head
        self.d_v = self.d_v or head
        self.dim_ff = _pad128(self.dim_ff or 8 * self.dim / 3)
        self.vocab_size = _pad128(self.vocab_size)
        self.num_kv_heads = self.num_kv_heads or self.num_heads
        if self.num_kv_heads != self.num_heads:
            raise ValueError("grouped-query attention (num_kv_heads < num_heads) is "
                             "implemented for softmax attention only")
        if self.d_qk > 64:
            raise ValueError(f"d_qk {self.d_qk} > 64: codes must pack into one uint64")

    @classmethod
    def from_dict(cls, d: dict) -> "ModelConfig":
        names = {f.name for f in dataclasses.fields(cls)}
        return cls(**{k: v for k, v in d.items() if k in names})

    def summary(self) -> str:
        return (f"{self.depth}L d{self.dim} h{self.num_heads} d_qk {self.d_qk} d_v {self.d_v} "
                f"dim_ff {self.dim_ff} attn {self.attn} pos {self.pos}")


class SwiGLU(nn.Module):
    def __init__(self, dim: int, dim_ff: int):
        super().__init__()
        self.gate = nn.Linear(dim, dim_ff, bias=False)
        self.up = nn.Linear(dim, dim_ff, bias=False)
        self.down = nn.Linear(dim_ff, dim, bias=False)

    def forward(self, x, residual=None):
        """down(silu(gate(x)) * up(x)), plus `residual` when given (Block's x + mlp(h)). On
        decode shapes the gate, up and product are one launch and the down projection adds
        the residual in its epilogue; on longer bf16 inputs without autograd the down GEMM
        accumulates into `residual` itself, which is then returned."""
        g, u, dn = self.gate.weight, self.up.weight, self.down.weight
        if _skinny(x, g) and g.shape == u.shape and u.data_ptr() % 16 == 0 and u.is_contiguous():
            K, N = x.shape[-1], g.shape[0]
            M = x.numel() // K
            a = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
            _lib.check(_lib.lib().lema_skinny_swiglu_bf16(
                x.data_ptr(), K, g.data_ptr(), u.data_ptr(), K, M, N, K, a.data_ptr(),
                _lib.stream_of(x)))
            if residual is not None and _skinny(a, dn) and residual.is_contiguous() \
                    and residual.shape == x.shape[:-1] + (dn.shape[0],) \
                    and residual.dtype == a.dtype and residual.data_ptr() % 16 == 0:
                y = torch.empty_like(residual)
                _lib.check(_lib.lib().lema_skinny_gemm_add_bf16(
                    a.data_ptr(), N, dn.data_ptr(), N, residual.data_ptr(), y.data_ptr(),
                    dn.shape[0], M, dn.shape[0], N, _lib.stream_of(x)))
                return y
        else:
            a = swiglu(linear(x, self.gate), linear(x, self.up))
            if residual is not None and not _skinny(a, dn) and a.is_cuda and \
                    a.dtype == residual.dtype == dn.dtype == torch.bfloat16 and \
                    residual.is_contiguous() and not torch.is_grad_enabled():
                # the residual add in the GEMM's epilogue, accumulating into `residual` in
                # place (one rounding of x + a . W^T where the two torch ops round twice;
                # within the forward's tolerance), 2-D operands
                D = dn.shape[0]
                residual.view(-1, D).addmm_(a.reshape(-1, a.shape[-1]), dn.t())
                return residual
        y = linear(a, self.down)
        return y if residual is None else residual + y

    def forward_normed(self, x, d, norm: nn.RMSNorm):
        """x + d + self(norm(x + d)), Block.forward's MLP half, on decode shapes: the norm runs
        inside the gate/up launch, rounded as rms_norm rounds it, so the result equals
        `self(*reversed(rms_norm(x, norm, d)))` bit for bit with one launch fewer. None where
        that launch does not apply."""
        g, u, dn = self.gate.weight, self.up.weight, self.down.weight
        K, N = x.shape[-1], g.shape[0]
        M = x.numel() // K
        if not (_skinny(x, g) and _fused(d, norm.weight) and d.shape == x.shape
                and g.shape == u.shape and _fused(u) and u.data_ptr() % 16 == 0
                and d.data_ptr() % 16 == 0 and norm.weight.data_ptr() % 16 == 0 and K <= 2048
                and M * (K + 8) * 2 + 8 * (16 if M <= 16 else 32) * 33 * 4 <= 160 * 1024
                and _fused(dn) and dn.data_ptr() % 16 == 0 and N % 32 == 0):
            return None
        xo = torch.empty_like(x)
        a = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
        eps = norm.eps if norm.eps is not None else torch.finfo(x.dtype).eps
        _lib.check(_lib.lib().lema_skinny_norm_swiglu_bf16(
            x.data_ptr(), d.data_ptr(), norm.weight.data_ptr(), float(eps), xo.data_ptr(),
            g.data_ptr(), u.data_ptr(), K, M, N, K, a.data_ptr(), _lib.stream_of(x)))
        y = torch.empty_like(xo)
        _lib.check(_lib.lib().lema_skinny_gemm_add_bf16(
            a.data_ptr(), N, dn.data_ptr(), N, xo.data_ptr(), y.data_ptr(), dn.shape[0], M,
            dn.shape[0], N, _lib.stream_of(x)))
        return y


class Attention(nn.Module):
    """A LEMA attention block (code/lema/model.py:143-210): q, k, v projections viewed as
    `[B, H, T, d]` (transposed views, read in place by the kernels), the exact op, o_proj."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.kind = cfg.attn
        self.q_proj = nn.Linear(cfg.dim, cfg.num_heads * cfg.d_qk, bias=False)
        self.k_proj = nn.Linear(cfg.dim, cfg.num_kv_heads * cfg.d_qk, bias=False)
        self.v_proj = nn.Linear(cfg.dim, cfg.num_kv_heads * cfg.d_v, bias=False)
        self.o_proj = nn.Linear(cfg.num_heads * cfg.d_v, cfg.dim, bias=False)
        self.hard = False

    def project(self, x):
        """`[B, T, dim]` -> query and key pre-activations and values, `[B, H, T, d]`."""
        B, T, _ = x.shape
        c = self.cfg
        zq = linear(x, self.q_proj).view(B, T, c.num_heads, c.d_qk).transpose(1, 2)
        zk = linear(x, self.k_proj).view(B, T, c.num_kv_heads, c.d_qk).transpose(1, 2)
        v = linear(x, self.v_proj).view(B, T, c.num_kv_heads, c.d_v).transpose(1, 2)
        return zq, zk, v

    def merge(self, y):
        B, _, T, _ = y.shape
        return linear(y.transpose(1, 2).reshape(B, T, -1).contiguous(), self.o_proj)

    def forward(self, x):
        if not self.hard:
            raise NotImplementedError("only the exact (hard) op is implemented: call "
                                      "model.set_hard(True)")
        codes = (project_qk_prefill(x, self, code_dtype_for(self.cfg.d_qk))
                 if FUSED_QK_PACK else None)
        if codes is not None:  # q and k straight to codes; v by its own product
            B, T, _ = x.shape
            c = self.cfg
            v = linear(x, self.v_proj).view(B, T, c.num_kv_heads, c.d_v).transpose(1, 2)
            return self.merge(lema_from_codes(codes[0], codes[1], v))
        zq, zk, v = self.project(x)
        return self.merge(lema_hard(zq, zk, v))


class Block(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.norm1 = nn.RMSNorm(cfg.dim, eps=cfg.norm_eps)
        self.attn = Attention(cfg)
        self.norm2 = nn.RMSNorm(cfg.dim, eps=cfg.norm_eps)
        self.mlp = SwiGLU(cfg.dim, cfg.dim_ff)
        self.seg = None

    def pre_attn(self, x):
        """The attention's input norm1(x): in bf16 on the device the fused norm kernel, which
        rounds x * rsqrt(mean(x^2) + eps) * w once from fp32 as torch's RMSNorm does (the
        codes are the signs of its projections)."""
        return rms_norm(x, self.norm1)[0]

    def gpu_pre(self, x):
        """Normalise, project, pack both codes (code/lema/model.py:224-227). On decode shapes
        the norm and the three projections are one launch, q and k going straight to codes
        (skinny MFMA kernel: pre-norm prologue, pack epilogues); with FUSED_QK_PACK set, on
        prefill chunks of 2048 or more rows q and k go straight to codes in one persistent
        MFMA launch."""
        at, c = self.attn, self.attn.cfg
        ct = code_dtype_for(c.d_qk)
        fused = project_qkv(x, at, ct, norm=self.norm1)
        if fused is not None:
            return fused
        h = self.pre_attn(x)
        fused = project_qkv(h, at, ct)
        if fused is not None:
            return fused
        codes = project_qk_prefill(h, at, ct) if FUSED_QK_PACK else None
        if codes is not None:  # prefill chunks of 2048+ rows
            B, T, _ = h.shape
            v = linear(h, at.v_proj).view(B, T, c.num_kv_heads, c.d_v).transpose(1, 2)
            return codes[0], codes[1], v
        qc = project_codes(h, at.q_proj, c.d_qk, ct)
        kc = project_codes(h, at.k_proj, c.d_qk, ct) if qc is not None else None
        if kc is not None:
            B, T, _ = h.shape
            v = linear(h, at.v_proj).view(B, T, c.num_kv_heads, c.d_v).transpose(1, 2)
            return qc, kc, v
        zq, zk, v = at.project(h)
        return pack_codes(zq, ct), pack_codes(zk, ct), v

    def gpu_post(self, x, got):
        """Merge the retrieved values and finish the layer (code/lema/model.py:229-232); on
        decode shapes the MLP's pre-norm runs inside its gate/up launch."""
        d = self.attn.merge(got)
        y = self.mlp.forward_normed(x, d, self.norm2)
        if y is not None:
            return y
        h, x = rms_norm(x, self.norm2, d)
        return self.mlp(h, residual=x)

    def forward(self, x, store=None):
        if store is not None:
            pre, post = self.seg or (self.gpu_pre, self.gpu_post)
            qc, kc, v = pre(x)
            return post(x, store.exchange(qc, kc, v))
        h, x = rms_norm(x, self.norm2, self.attn(self.pre_attn(x)))
        return self.mlp(h, residual=x)


class Transformer(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.tok_emb = nn.Embedding(cfg.vocab_size, cfg.dim)
        self.blocks = nn.ModuleList(Block(cfg) for _ in range(cfg.depth))
        self.norm_f = nn.RMSNorm(cfg.dim, eps=cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.dim, cfg.vocab_size, bias=False)
        self.checkpoint_blocks = False
        self._init_weights()

    def _init_weights(self):
        for m in self.modules():
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, mean=0.0, std=1.0 / math.sqrt(m.weight.shape[1]))
            elif isinstance(m, nn.Embedding):
                nn.init.normal_(m.weight, mean=0.0, std=1.0 / math.sqrt(self.cfg.dim))
        for b in self.blocks:
            for lin in (b.attn.o_proj, b.mlp.down):
                lin.weight.data.mul_(1.0 / math.sqrt(2 * self.cfg.depth))

    def lema_layers(self):
        return [b.attn for b in self.blocks if b.attn.kind == "lema"]

    def set_hard(self, hard: bool = True):
        for att in self.lema_layers():
            att.hard = hard

    def new_cache(self, place: str = "hbm", **kw):
        """A retrieval cache for this model (code/lema/model.py:306-324): in device memory
        (place "hbm", or "vram"), or in pinned host RAM ("ram", the reference's placement,
        for caches larger than device memory; the same kernels work on it in place over the
        host link). `max_cache_len=` or `capacity=` slots, `batch=`, `max_load=`,
        `codes_hook=` as in `LemaCache`."""
        from .cache import LemaCache
        if place not in ("hbm", "vram", "ram"):
            raise ValueError(f"a LEMA cache lives in device memory (place='hbm') or host RAM "
                             f"(place='ram'); place={place!r} is not an implementation of it")
        p = next(self.parameters())
        kw.setdefault("dtype", p.dtype)
        kw.pop("pin", None)
        return LemaCache(self.cfg, device=p.device, place="ram" if place == "ram" else "hbm",
                         **kw)

    def forward(self, idx, *, cache=None, return_logits=True):
        """Run `idx` through the model (code/lema/model.py:337-363).

            forward(x)                                batched, no state
            forward(x, cache=c, return_logits=False)  prefill: fills c, no logits
            forward(next, cache=c)                    extending c

        With a cache, queries match keys from before this call too, so a sequence can be fed
        in pieces; any chunking gives the one-shot result.
        """
        if cache is not None and not (self.lema_layers()
                                      and all(a.hard for a in self.lema_layers())):
            raise ValueError("a cache needs an all-LEMA model in hard mode")
        x = self.tok_emb(idx)
        for li, blk in enumerate(self.blocks):
            x = blk(x, store=(cache.layer(li) if cache is not None else None))
        if cache is not None:
            cache.t += idx.shape[-1]
        return linear(rms_norm(x, self.norm_f)[0], self.lm_head) if return_logits else None

    def hidden(self, idx):
        """The final normalised hidden states (the input of lm_head), without a cache."""
        x = self.tok_emb(idx)
        for blk in self.blocks:
            x = blk(x)
        return rms_norm(x, self.norm_f)[0]

    def n_params(self, embedding: bool = True) -> int:
        n = sum(p.numel() for p in self.parameters())
        if not embedding:
            n -= self.tok_emb.weight.numel() + self.lm_head.weight.numel()
        return n


def lm_loss(model: Transformer, x: torch.Tensor, y: torch.Tensor, chunk: int = 4096):
    """Mean next-token cross-entropy without holding the full `[B, T, vocab]` logits: the
    head and the loss run `chunk` positions at a time on the final hidden states, in fp32
    (code/lema/train.py:131-152, forward only). At B4 T16384 with a 50,304-word vocabulary,
    chunks of 4096 positions (head GEMMs of 16,384 rows, 1.65 GB of bf16 logits at a time)
    took the whole forward from 119.9-120.4 to 118.2-118.8 ms against chunks of 1024."""
    h = model.hidden(x)
    total = torch.zeros((), dtype=torch.float32, device=h.device)
    for a in range(0, x.shape[1], chunk):
        # a contiguous 2-D block: the head is then one plain GEMM (a strided 3-D slice would
        # make matmul broadcast the transposed weight into a batched product instead)
        hc = h[:, a:a + chunk].reshape(-1, h.shape[-1]).contiguous()
        total += cross_entropy_sum(model.lm_head(hc), y[:, a:a + chunk].reshape(-1))
    return total / y.numel()


def load_trained(path, device="cuda") -> tuple[Transformer, ModelConfig]:
    """A finished training run, ready to evaluate (code/lema/model.py:420-436): `path` is the
    run directory (its `model.pt`) or a checkpoint file, a dict holding `config` (the
    ModelConfig fields) and `state_dict`. The model comes back in hard mode, fp32, in eval
    mode; parameters the checkpoint holds beyond this model's are dropped.

    The file is read with `torch.load(weights_only=True)`, which builds tensors and plain
    containers only and executes nothing from the file; a checkpoint that needs arbitrary
    objects to load raises instead. Only all-LEMA configurations load (ModelConfig raises
    ValueError for the others)."""
    path = Path(path)
    if path.is_dir():
        path = path / "model.pt"
    ck = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(ck, dict) or "config" not in ck or "state_dict" not in ck:
        raise ValueError(f"{path}: expected a dict with 'config' and 'state_dict'")
    cfg = ModelConfig.from_dict(dict(ck["config"]))
    model = Transformer(cfg).to(device).eval()
    keep = model.state_dict().keys()
    model.load_state_dict({k: v for k, v in ck["state_dict"].items() if k in keep})
    model.set_hard(True)
    return model, cfg
