"""Write tests/golden/model.npz from the reference's own LEMA language model.

The model's forward and its same-seed initialisation (code/lema/model.py:143-363,
code/lema/attention.py:82-158) have no closed form and no golden vectors in the reference,
so this script imports the reference package from its checkout (`code/` on sys.path, CPU,
fp32, hard mode) and records, at two tiny geometries:

  * every parameter's name, shape, float32 byte digest (sha256) and sum, as drawn by
    `Transformer(cfg)` right after `torch.manual_seed(seed)`;
  * then, so that codes repeat and the exact op matches often, every block's k_proj
    weight is set to a copy of its q_proj weight (a query then matches the latest earlier
    position with the same normalised hidden state's sign pattern);
  * a [2, 65] token batch (row 0 over 12 distinct ids, so codes repeat and matches occur;
    row 1 uniform), x = tok[:, :-1], y = tok[:, 1:];
  * each layer's query and key codes and match indices, captured by wrapping the
    reference's `pack_codes` and `latest_prev_match` inside `lema_hard`;
  * the logits [2, 64, vocab] and the mean cross-entropy of the logits against y
    (code/lema/train.py:131-152, in fp32).

Geometry "d16" has 16-bit codes (int32 carrier here), "d40" 40-bit codes (int64 carrier).
Run once in a container that holds the reference:

    python tests/golden/make_model_golden.py /root/reference/code

It only reads the reference (no bytecode is written). The fixture is data; no reference
source is stored.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "model.npz"

GEOMETRIES = {
    "d16": (0, dict(vocab_size=256, depth=2, dim=128, num_heads=4, d_qk=16, d_v=32)),
    "d40": (1, dict(vocab_size=200, depth=2, dim=96, num_heads=2, d_qk=40, d_v=24)),
}


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().float().contiguous().numpy().tobytes()).hexdigest()


def tokens(seed: int, vocab: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(1000 + seed)
    few = torch.randint(0, vocab, (12,), generator=g)
    row0 = few[torch.randint(0, 12, (65,), generator=g)]
    row1 = torch.randint(0, vocab, (65,), generator=g)
    return torch.stack([row0, row1])


def main(ref_code: str) -> None:
    sys.dont_write_bytecode = True
    sys.path.insert(0, ref_code)
    import lema.attention as ref_attention
    from lema.model import ModelConfig, Transformer

    torch.set_num_threads(1)
    out = {}
    for name, (seed, geo) in GEOMETRIES.items():
        cfg = ModelConfig(attn="lema", **geo)
        torch.manual_seed(seed)
        model = Transformer(cfg).eval()
        model.set_hard(True)
        sd = model.state_dict()
        out[f"{name}/param_names"] = np.array(list(sd))
        out[f"{name}/param_shapes"] = np.array([list(t.shape) + [0] * (2 - t.dim())
                                                for t in sd.values()], dtype=np.int64)
        out[f"{name}/param_sha256"] = np.array([digest(t) for t in sd.values()])
        out[f"{name}/param_sums"] = np.array([t.double().sum().item() for t in sd.values()])

        with torch.no_grad():
            for blk in model.blocks:
                blk.attn.k_proj.weight.copy_(blk.attn.q_proj.weight)
        tok = tokens(seed, geo["vocab_size"])
        x, y = tok[:, :-1], tok[:, 1:]
        codes, srcs = [], []
        pack0, match0 = ref_attention.pack_codes, ref_attention.latest_prev_match

        def pack_rec(z):
            c = pack0(z)
            codes.append(c.clone())
            return c

        def match_rec(qc, kc):
            s = match0(qc, kc)
            srcs.append(s.clone())
            return s

        ref_attention.pack_codes, ref_attention.latest_prev_match = pack_rec, match_rec
        try:
            with torch.no_grad():
                logits = model(x)
        finally:
            ref_attention.pack_codes, ref_attention.latest_prev_match = pack0, match0
        B, T = x.shape
        H = cfg.num_heads
        assert len(codes) == 2 * cfg.depth and len(srcs) == cfg.depth
        loss = F.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), y.reshape(-1))
        out[f"{name}/config"] = np.array([cfg.vocab_size, cfg.depth, cfg.dim, cfg.num_heads,
                                          cfg.d_qk, cfg.d_v, cfg.dim_ff, seed],
                                         dtype=np.int64)
        out[f"{name}/tokens"] = tok.numpy()
        out[f"{name}/qc"] = torch.stack(codes[0::2]).reshape(cfg.depth, B, H, T).numpy()
        out[f"{name}/kc"] = torch.stack(codes[1::2]).reshape(cfg.depth, B, H, T).numpy()
        out[f"{name}/src"] = torch.stack(srcs).reshape(cfg.depth, B, H, T).numpy()
        out[f"{name}/logits"] = logits.float().numpy()
        out[f"{name}/loss"] = np.array(loss.item(), dtype=np.float64)
        hits = (out[f"{name}/src"] >= 0).mean()
        print(f"{name}: loss {loss.item():.6f}, match rate {hits:.3f}, "
              f"{len(sd)} tensors")
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/code")
