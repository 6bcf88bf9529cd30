"""Consumers of the exact op that look inside a model, on the HIP path: the reference's
`lema.analysis.trace` (code/lema/analysis.py:1-61), the distinct-code census of
code/experiments/main_codes_count/count_codes.py:39-57, and the generation state of
code/experiments/app_retrieval/gen_eval.py:211-275, each with the same interface.

    trace(model, x)        per layer {"qc", "kc", "src"} from the same pre-activations the
                           forward uses (codes and latest-match indices, int64)
    prefix_distinct(kc)    [H, T] -> distinct key codes among positions <= t, for every t
    census(model, x)       [depth, H, T] entry counts of every head after each prefix
    LemaState              prefill + single-token steps of a hard-mode model, the state kept
                           in the device store
"""
from __future__ import annotations

import torch

from .attention import latest_prev_match, pack_codes
from .model import rms_norm

__all__ = ["trace", "prefix_distinct", "census", "LemaState"]


@torch.no_grad()
def trace(model, x, reduce=None, return_logits=True):
    """Run `x` ([B, T] tokens) through `model` and return (logits, records), one record per
    layer: {"qc", "kc"} [B, H, T] int64 codes and "src" [B, H, T] int64, the position each
    query reads (-1 on no match). `reduce(layer, rec)`, if given, replaces the record by its
    result inside the hook (code/lema/analysis.py:29-61)."""
    recs = [None] * model.cfg.depth

    def hook(li):
        def fn(blk, inp, _out):
            zq, zk, _ = blk.attn.project(blk.pre_attn(inp[0]))
            qc, kc = pack_codes(zq), pack_codes(zk)
            B, H, T = qc.shape
            src = latest_prev_match(qc.reshape(B * H, T), kc.reshape(B * H, T))
            rec = {"qc": qc, "kc": kc, "src": src.view(B, H, T)}
            recs[li] = reduce(li, rec) if reduce is not None else rec
        return fn

    handles = [blk.register_forward_hook(hook(li)) for li, blk in enumerate(model.blocks)]
    try:
        logits = model(x, return_logits=return_logits)
    finally:
        for h in handles:
            h.remove()
    return logits, recs


def prefix_distinct(codes: torch.Tensor) -> torch.Tensor:
    """[H, T] codes -> [H, T] int64: the number of distinct codes among positions <= t
    (code/experiments/main_codes_count/count_codes.py:39-48). Position t holds the first
    occurrence of its code exactly when no earlier position has the same code, i.e. when its
    latest earlier match against the codes themselves is -1: one resolver pass and a running
    sum, no sort."""
    if codes.dim() != 2:
        raise ValueError(f"codes must be [H, T], got shape {tuple(codes.shape)}")
    first = latest_prev_match(codes, codes) < 0
    return first.long().cumsum(1)


@torch.no_grad()
def census(model, x: torch.Tensor):
    """[depth, heads, T] entry counts after each prefix of `x` ([1, T] tokens)
    (code/experiments/main_codes_count/count_codes.py:51-57)."""
    _, counts = trace(model, x, return_logits=False,
                      reduce=lambda li, r: prefix_distinct(r["kc"][0]))
    return torch.stack(counts)


class LemaState:
    """A hard-mode LEMA model's generation state (code/experiments/app_retrieval/
    gen_eval.py:211-275): `prefill(x)` feeds a prompt and `step(tok)` one token per stream,
    each returning the final normalised hidden state of the last position. The reference
    keeps every position's key code and value and scans them per step; here the state is the
    device store of `model.new_cache` -- one entry per distinct (layer, stream, head, code) --
    and a step is one exchange per layer."""

    @staticmethod
    def bytes_per_row(cfg, T: int, max_load: float = 0.7) -> int:
        """Store bytes provisioned per stream for T positions (worst case: a new code per
        position per head)."""
        return int(cfg.depth * T * cfg.num_heads * (16 + 2 * cfg.d_v) / max_load)

    def __init__(self, model, B: int, maxlen: int, device="cuda"):
        self.model, self.n = model, 0
        self.cache = model.new_cache("hbm", max_cache_len=maxlen, batch=B)

    def _run(self, x):
        m, cache = self.model, self.cache
        h = m.tok_emb(x)
        for li, blk in enumerate(m.blocks):
            qc, kc, v = blk.gpu_pre(h)
            h = blk.gpu_post(h, cache.layer(li).exchange(qc, kc, v))
        cache.t += x.shape[1]
        self.n += x.shape[1]
        return h

    @torch.no_grad()
    def prefill(self, x):
        return rms_norm(self._run(x)[:, -1:].contiguous(), self.model.norm_f)[0]

    @torch.no_grad()
    def step(self, tok):
        return rms_norm(self._run(tok), self.model.norm_f)[0]
