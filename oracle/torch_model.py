"""The LEMA language model's forward restated functionally in plain torch -- TEST
INFRASTRUCTURE ONLY (the oracle of the model path; the product never imports it).

Follows code/lema/model.py:143-363 in hard mode from a state dict with the reference's
parameter names: embedding; per block pre-RMSNorm, q/k/v projections viewed as
`[B, H, T, d]`, codes packed as sum_j [z_j >= 0] << j (code/lema/attention.py:95-97), the
exact op by the reference's sort-based algorithm (`torch_port`, attention.py:100-158),
o_proj, residual, pre-RMSNorm SwiGLU, residual; final RMSNorm and the untied head; the
mean cross-entropy in fp32 (code/lema/train.py:120-152). Runs on whatever device the
tensors are on.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .torch_port import latest_prev_match_sorted


def pack(z: torch.Tensor) -> torch.Tensor:
    """code/lema/attention.py:92-97 (int64 codes)."""
    D = z.shape[-1]
    pw = torch.ones((), dtype=torch.int64, device=z.device) << torch.arange(
        D, device=z.device, dtype=torch.int64)
    return ((z >= 0).to(torch.int64) * pw).sum(-1)


def lema_exact(zq, zk, v):
    """code/lema/attention.py:151-158: codes, latest match, gather, miss mask. Returns the
    output and the match indices."""
    B, H, T, _ = v.shape
    qc, kc = pack(zq), pack(zk)
    src = latest_prev_match_sorted(qc.reshape(B * H, T), kc.reshape(B * H, T)).view(B, H, T)
    y = torch.gather(v, 2, src.clamp_min(0).unsqueeze(-1).expand_as(v))
    return y * (src >= 0).unsqueeze(-1).to(v.dtype), src


def forward_hidden(sd: dict, cfg, idx: torch.Tensor, record=None):
    """Final normalised hidden states; `record` (a list) receives each layer's indices."""
    c = cfg
    x = F.embedding(idx, sd["tok_emb.weight"])
    B, T, _ = x.shape
    for i in range(c.depth):
        p = f"blocks.{i}."
        h = F.rms_norm(x, (c.dim,), sd[p + "norm1.weight"], c.norm_eps)
        zq = F.linear(h, sd[p + "attn.q_proj.weight"]).view(B, T, c.num_heads, c.d_qk)
        zk = F.linear(h, sd[p + "attn.k_proj.weight"]).view(B, T, c.num_heads, c.d_qk)
        v = F.linear(h, sd[p + "attn.v_proj.weight"]).view(B, T, c.num_heads, c.d_v)
        y, src = lema_exact(zq.transpose(1, 2), zk.transpose(1, 2), v.transpose(1, 2))
        if record is not None:
            record.append(src)
        x = x + F.linear(y.transpose(1, 2).reshape(B, T, -1), sd[p + "attn.o_proj.weight"])
        h = F.rms_norm(x, (c.dim,), sd[p + "norm2.weight"], c.norm_eps)
        g = F.linear(h, sd[p + "mlp.gate.weight"])
        u = F.linear(h, sd[p + "mlp.up.weight"])
        x = x + F.linear(F.silu(g) * u, sd[p + "mlp.down.weight"])
    return F.rms_norm(x, (c.dim,), sd["norm_f.weight"], c.norm_eps)


def loss(sd: dict, cfg, x: torch.Tensor, y: torch.Tensor, chunk: int = 1024, record=None):
    h = forward_hidden(sd, cfg, x, record)
    total = torch.zeros((), dtype=torch.float32, device=h.device)
    for a in range(0, x.shape[1], chunk):
        hc = h[:, a:a + chunk].reshape(-1, h.shape[-1]).contiguous()   # 2-D: a plain GEMM
        logits = F.linear(hc, sd["lm_head.weight"])
        total += F.cross_entropy(logits.float(), y[:, a:a + chunk].reshape(-1),
                                 reduction="sum")
    return total / y.numel()
