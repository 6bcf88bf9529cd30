"""The reference's CPU "library attention" restated with torch ops, for the CPU baseline only
(test infrastructure: the product never imports this).

`latest_prev_match_sorted` follows code/lema/attention.py:100-132 step for step -- two
stable argsorts order the 2T events by (code, position, query before key), a cumulative
maximum of key positions runs inside each code's segment, and a scatter sends the answers
back to query positions -- so timing it on the host's cores times the reference's own
algorithm. `lema_hard_codes` adds the gather and mask of attention.py:157-158. Both run
on the tensors' device (the CPU baseline times them on the host's cores; the model oracle
runs them on the GPU).
"""
from __future__ import annotations

import torch


def latest_prev_match_sorted(qc: torch.Tensor, kc: torch.Tensor) -> torch.Tensor:
    N, T = qc.shape
    codes = torch.cat([qc, kc], dim=1)                                  # [N, 2T] events
    dev = qc.device
    pos = torch.arange(T, device=dev).repeat(2)
    kind = torch.cat([torch.zeros(T, dtype=torch.long, device=dev),
                      torch.ones(T, dtype=torch.long, device=dev)])
    # stable sort by the secondary key (position, then query before key), then by code
    by_pos = (2 * pos + kind).expand(N, -1).argsort(dim=1, stable=True)
    by_code = codes.gather(1, by_pos).argsort(dim=1, stable=True)
    order = by_pos.gather(1, by_code)
    c = codes.gather(1, order)
    is_key = kind.expand(N, -1).gather(1, order).bool()
    p = pos.expand(N, -1).gather(1, order)
    starts = torch.ones_like(c, dtype=torch.bool)
    starts[:, 1:] = c[:, 1:] != c[:, :-1]
    seg = starts.long().cumsum(1) - 1
    stride = T + 2                                  # keeps segments from mixing in the max
    run = torch.where(is_key, p + 1, torch.zeros_like(p)) + seg * stride
    latest = run.cummax(dim=1).values - seg * stride - 1
    dest = torch.where(is_key, torch.full_like(p, T), p)     # keys go to a dump column
    return p.new_full((N, T + 1), -1).scatter_(1, dest, latest)[:, :T]


def lema_hard_codes(qc: torch.Tensor, kc: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """y = v[src] * (src >= 0) on [B, H, T] codes and [B, H, T, d_v] values."""
    B, H, T, _ = v.shape
    src = latest_prev_match_sorted(qc.reshape(B * H, T), kc.reshape(B * H, T)).view(B, H, T)
    y = torch.gather(v, 2, src.clamp_min(0).unsqueeze(-1).expand_as(v))
    return y * (src >= 0).unsqueeze(-1).to(v.dtype)
