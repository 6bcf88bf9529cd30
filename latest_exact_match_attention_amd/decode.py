"""Single-token decoding of a LEMA model with the whole step in ONE HIP graph.

The reference's `LemaDecoder` (code/lema/decode.py:183-240) replays depth + 1 CUDA graphs
per token with the host hash-table exchange between them (a device sync, a D2H and an H2D
copy per layer). Here the store lives in HBM and each layer's exchange is one kernel on the
step's stream, so the complete step -- embedding, every layer's projections, code packing,
store exchange, merge and MLP, the head and the choice of the next token -- is captured
once and replayed as a single graph launch per token.

The captured work is exactly `Transformer.forward(tok, cache=...)`: the same
`Block.gpu_pre` / `gpu_post` segments and the same store exchange, so a replay reproduces an
eager step. The graph ends by writing the chosen token into `tok`, which the next replay
reads.
"""
from __future__ import annotations

import contextlib

import torch

from .cache import HashStore, LemaCache
from .model import argmax_into, embed, linear, rms_norm

__all__ = ["LemaDecoder", "decoder", "worst_case_codes"]


def _chooser(temperature: float):
    """(logits, tok) -> next token written into tok: argmax, or a draw from
    softmax(logits / temperature) by the Gumbel-max trick (code/lema/decode.py:71-93):
    argmax(logits / T + g) with g = -log(E), E ~ Exponential(1). In fp32, so near-tied bf16
    logits stay distinct. Inside a graph the generator advances on every replay."""
    if temperature <= 0:
        return argmax_into

    def pick(logits, tok):
        z = logits.float() / temperature
        g = torch.empty_like(z).exponential_().log().neg_()
        tok.copy_((z + g).argmax(-1))
    return pick


@contextlib.contextmanager
def _scratch_store(cache: LemaCache):
    """Point every layer view at a throw-away store of the same partitions while the step is
    warmed up (first calls load kernels and allocate), so the real table is not touched."""
    real = cache.store
    scratch = HashStore(real.d_v, groups=real.groups, dtype=real.dtype,
                        capacity=max(16, 4 * real.groups), device=real.device)
    views = [cache.layer(i) for i in range(cache.cfg.depth)]
    for v in views:
        v.store = scratch
    try:
        yield
    finally:
        for v in views:
            v.store = real


class LemaDecoder:
    """A LEMA model decoding `cache.batch` streams one token per `step()`: one graph replay
    per token, the store exchanges inside it."""

    def __init__(self, model, cache: LemaCache, tok: torch.Tensor | None = None,
                 temperature: float = 0.0):
        cfg = model.cfg
        if not model.lema_layers() or not all(a.hard for a in model.lema_layers()):
            raise ValueError("LemaDecoder needs an all-LEMA model in hard mode")
        if not isinstance(cache, LemaCache):
            raise TypeError("LemaDecoder needs a LemaCache of this package (model.new_cache())")
        self.model, self.cache = model, cache
        B, L = cache.batch, cfg.depth
        dev = next(model.parameters()).device
        self.tok = torch.zeros(B, 1, dtype=torch.long, device=dev)
        if tok is not None:
            if bool(((tok < 0) | (tok >= cfg.vocab_size)).any()):
                raise ValueError(f"tokens must lie in [0, {cfg.vocab_size})")
            self.tok.copy_(tok)
        views = [cache.layer(i) for i in range(L)]
        segs = [b.seg or (b.gpu_pre, b.gpu_post) for b in model.blocks]
        choose = _chooser(temperature)

        def step_fn():
            x = embed(model.tok_emb, self.tok)
            for i in range(L):
                qc, kc, v = segs[i][0](x)
                x = segs[i][1](x, views[i].exchange(qc, kc, v, check=False))
            logits = linear(rms_norm(x, model.norm_f)[0], model.lm_head)
            choose(logits, self.tok)
            return logits

        tok0 = self.tok.clone()
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with _scratch_store(cache), torch.cuda.stream(s):
            for _ in range(2):
                step_fn()
        torch.cuda.current_stream(dev).wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = step_fn()
        self.tok.copy_(tok0)
        cache.store.check_full()

    def step(self, check: bool = True) -> torch.Tensor:
        """Decode one token for every stream; returns `tok` ([batch, 1], on the device). With
        `check` the store's full flag is read back (a sync) and a full table raises like the
        reference; without it call `cache.store.check_full()` later."""
        self.graph.replay()
        self.cache.t += 1
        if check:
            self.cache.store.check_full()
        return self.tok


def decoder(model, cache, tok=None, temperature: float = 0.0):
    """The decoder for a cache (code/lema/decode.py:243-248); a LEMA cache here."""
    return LemaDecoder(model, cache, tok, temperature)


def worst_case_codes(depth: int):
    """A `LemaCache` codes hook replacing every layer's query AND key codes with fresh
    uniformly random 64-bit codes (code/experiments/main_inference/common.py:170-196): every
    lookup probes to the end of a random run and every insert claims a fresh random slot,
    the worst access pattern a model can produce. All layers' codes are drawn at layer 0 by
    one kernel into a buffer the later layers view; inside a graph every replay draws
    afresh."""
    bufs = {}

    def hook(layer, qc, kc):
        key = (qc.device, tuple(qc.shape))
        if layer == 0 or key not in bufs:
            if key not in bufs:
                bufs[key] = torch.empty((depth, 2) + tuple(qc.shape), dtype=torch.int64,
                                        device=qc.device)
            bufs[key].random_()
        b = bufs[key]
        return b[layer, 0], b[layer, 1]
    return hook
