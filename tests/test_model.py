"""The model host code and its oracle on the CPU: configuration rules, parameter names and
init (code/lema/model.py:33-82, 258-281), and pins of the functional model oracle."""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_model
from latest_exact_match_attention_amd.model import ModelConfig, Transformer


def reference_param_names(depth):
    """The reference's state-dict keys in module order (code/lema/model.py:152-265)."""
    names = ["tok_emb.weight"]
    for i in range(depth):
        p = f"blocks.{i}."
        names += [p + "norm1.weight", p + "attn.q_proj.weight", p + "attn.k_proj.weight",
                  p + "attn.v_proj.weight", p + "attn.o_proj.weight", p + "norm2.weight",
                  p + "mlp.gate.weight", p + "mlp.up.weight", p + "mlp.down.weight"]
    return names + ["norm_f.weight", "lm_head.weight"]


def test_config_geometry_and_rules():
    c = ModelConfig(vocab_size=50304, depth=24, dim=1536, num_heads=64, dim_ff=6144)
    assert (c.d_qk, c.d_v, c.dim_ff, c.vocab_size) == (24, 24, 6144, 50304)
    c = ModelConfig(vocab_size=1000, depth=1, dim=96, num_heads=4)
    assert (c.d_qk, c.dim_ff, c.vocab_size) == (24, 256, 1024)     # 8*96/3 = 256, pad 128
    with pytest.raises(ValueError, match="d_qk"):
        ModelConfig(vocab_size=10, depth=1, dim=128, num_heads=1)  # d_qk 128 > 64
    with pytest.raises(ValueError, match="divisible"):
        ModelConfig(vocab_size=10, depth=1, dim=100, num_heads=3)
    with pytest.raises(ValueError, match="attn"):
        ModelConfig(vocab_size=10, depth=1, dim=64, num_heads=2, attn="softmax")


def test_parameter_names_shapes_and_init():
    cfg = ModelConfig(vocab_size=300, depth=3, dim=64, num_heads=4, d_qk=8, d_v=16)
    torch.manual_seed(0)
    m = Transformer(cfg)
    sd = m.state_dict()
    assert list(sd) == reference_param_names(3)
    assert sd["blocks.0.attn.q_proj.weight"].shape == (4 * 8, 64)
    assert sd["blocks.0.attn.o_proj.weight"].shape == (64, 4 * 16)
    assert sd["lm_head.weight"].shape == (384, 64)
    # std 1/sqrt(fan_in), residual outputs scaled by 1/sqrt(2 depth), embedding 1/sqrt(dim)
    big = ModelConfig(vocab_size=4096, depth=2, dim=256, num_heads=8, dim_ff=1024)
    torch.manual_seed(1)
    b = Transformer(big).state_dict()
    def near(t, want):
        assert abs(t.float().std().item() / want - 1) < 0.05, (t.float().std().item(), want)
    near(b["tok_emb.weight"], 1 / math.sqrt(256))
    near(b["blocks.0.attn.q_proj.weight"], 1 / math.sqrt(256))
    near(b["blocks.1.mlp.up.weight"], 1 / math.sqrt(256))
    near(b["blocks.0.attn.o_proj.weight"], 1 / math.sqrt(256) / math.sqrt(4))
    near(b["blocks.1.mlp.down.weight"], 1 / math.sqrt(1024) / math.sqrt(4))
    assert torch.equal(b["norm_f.weight"], torch.ones(256))
    # the same seed gives the same weights
    torch.manual_seed(1)
    again = Transformer(big).state_dict()
    assert all(torch.equal(b[k], again[k]) for k in b)


def test_forward_refuses_cpu_and_soft_mode():
    cfg = ModelConfig(vocab_size=128, depth=1, dim=32, num_heads=2)
    m = Transformer(cfg)
    with pytest.raises(NotImplementedError, match="hard"):
        m(torch.zeros(1, 4, dtype=torch.long))
    m.set_hard(True)
    with pytest.raises(TypeError):
        m(torch.zeros(1, 4, dtype=torch.long))        # the exact op is device-only
    with pytest.raises(ValueError, match="host RAM"):
        m.new_cache("disk")


def test_model_oracle_exact_op_is_the_dict_rule():
    rng = np.random.default_rng(0)
    zq = torch.from_numpy(rng.standard_normal((2, 3, 200, 3)))
    zk = torch.from_numpy(rng.standard_normal((2, 3, 200, 3)))
    v = torch.from_numpy(rng.standard_normal((2, 3, 200, 5)))
    y, src = torch_model.lema_exact(zq, zk, v)
    qc = torch_model.pack(zq).reshape(6, 200).numpy()
    kc = torch_model.pack(zk).reshape(6, 200).numpy()
    want = np.stack([oracle.dict_rule(qc[r], kc[r]) for r in range(6)]).reshape(2, 3, 200)
    assert np.array_equal(src.numpy(), want)
    assert (src >= 0).float().mean() > 0.5                    # 8 codes: mostly hits
    hit = torch.from_numpy(want >= 0).unsqueeze(-1)
    g = torch.gather(v, 2, torch.from_numpy(want).clamp_min(0).unsqueeze(-1).expand_as(v))
    assert torch.equal(y, torch.where(hit, g, torch.zeros_like(g)))


def test_model_oracle_zero_qk_is_previous_token_copy():
    """With zero q/k projections every code is all ones (z = 0 >= 0), so every query's
    latest match is the previous position: attention copies v one position back (position 0
    reads zeros). The oracle's forward must equal that closed form."""
    cfg = ModelConfig(vocab_size=128, depth=2, dim=32, num_heads=2, dim_ff=64)
    torch.manual_seed(0)
    sd = {k: v.double() for k, v in Transformer(cfg).state_dict().items()}
    for i in range(cfg.depth):
        sd[f"blocks.{i}.attn.q_proj.weight"].zero_()
        sd[f"blocks.{i}.attn.k_proj.weight"].zero_()
    idx = torch.randint(0, 128, (2, 40))
    got = torch_model.forward_hidden(sd, cfg, idx)

    F = torch.nn.functional
    x = F.embedding(idx, sd["tok_emb.weight"])
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        h = F.rms_norm(x, (32,), sd[p + "norm1.weight"], cfg.norm_eps)
        v = h @ sd[p + "attn.v_proj.weight"].T                   # [B, T, H * d_v]
        shifted = torch.cat([torch.zeros_like(v[:, :1]), v[:, :-1]], dim=1)
        x = x + shifted @ sd[p + "attn.o_proj.weight"].T
        h = F.rms_norm(x, (32,), sd[p + "norm2.weight"], cfg.norm_eps)
        x = x + (F.silu(h @ sd[p + "mlp.gate.weight"].T) * (h @ sd[p + "mlp.up.weight"].T)) \
            @ sd[p + "mlp.down.weight"].T
    want = F.rms_norm(x, (32,), sd["norm_f.weight"], cfg.norm_eps)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


def _aten_ops(fn):
    from torch.profiler import ProfilerActivity, profile
    with profile(activities=[ProfilerActivity.CPU]) as p:
        fn()
    return {e.key for e in p.key_averages()}


def test_losses_run_the_head_as_plain_gemms():
    """The chunked head must see 2-D contiguous blocks: a strided 3-D slice would make matmul
    expand the transposed weight into a batched bf16 product (aten::bmm), a form that is
    not used anywhere on this path."""
    from latest_exact_match_attention_amd import model as M
    cfg = ModelConfig(vocab_size=256, depth=1, dim=64, num_heads=2)
    torch.manual_seed(0)
    m = Transformer(cfg).to(torch.bfloat16)
    x = torch.randint(0, 256, (2, 96))
    y = torch.randint(0, 256, (2, 96))
    h = torch.randn(2, 96, 64, dtype=torch.bfloat16)
    m.hidden = lambda idx: h                      # the head and the loss alone
    ops = _aten_ops(lambda: M.lm_loss(m, x, y, chunk=32))
    assert "aten::mm" in ops and "aten::bmm" not in ops
    sd = {k: v.float() for k, v in Transformer(cfg).state_dict().items()}
    ops = _aten_ops(lambda: torch_model.loss(sd, cfg, x, y, chunk=32))
    assert "aten::bmm" not in ops


def test_fused_decode_segments_decline_what_they_cannot_take():
    """The MLP-with-pre-norm launch, the embedding gather and the argmax are device bf16 paths:
    on CPU tensors forward_normed declines (the caller then runs rms_norm and the MLP), and the
    embedding and argmax fall back to the torch ops they mirror."""
    from latest_exact_match_attention_amd.model import SwiGLU, argmax_into, embed
    mlp = SwiGLU(64, 128).to(torch.bfloat16)
    norm = torch.nn.RMSNorm(64, eps=1e-5).to(torch.bfloat16)
    x = torch.randn(2, 1, 64).to(torch.bfloat16)
    assert mlp.forward_normed(x, x.clone(), norm) is None
    emb = torch.nn.Embedding(10, 8)
    ids = torch.tensor([[3], [9]])
    assert torch.equal(embed(emb, ids), emb(ids))
    logits = torch.tensor([[[0.5, 2.0, 2.0, -1.0]], [[float("nan"), 1.0, 3.0, 0.0]]])
    tok = torch.zeros(2, 1, dtype=torch.long)
    argmax_into(logits, tok)
    assert tok.view(-1).tolist() == [1, 0]


class _HostStoreView:
    """A stand-in for a layer's store view on the CPU: the exchange returns zeros like v (the
    op trace, not the values, is what the test looks at)."""

    def exchange(self, qc, kc, v, check=True):
        return torch.zeros(v.shape, dtype=v.dtype)


class _HostCache:
    def __init__(self, depth):
        self.t, self._v = 0, [_HostStoreView() for _ in range(depth)]

    def layer(self, i):
        return self._v[i]


def test_forward_and_decode_step_issue_no_batched_products(monkeypatch):
    """Transformer.forward (dense and through a cache) and one decode step's work -- the
    cached forward of one token per stream, then the greedy pick -- in bf16 on the CPU with
    the device-only exact op stubbed by the oracle's: no aten::bmm anywhere (every product is
    a plain 2-D GEMM), the form a bf16 batched product with a transposed operand takes."""
    from latest_exact_match_attention_amd import model as M
    monkeypatch.setattr(M, "lema_hard", lambda q, k, v: torch_model.lema_exact(q, k, v)[0])
    monkeypatch.setattr(M, "pack_codes", lambda z, dt=torch.int64: torch_model.pack(z).to(dt))
    cfg = ModelConfig(vocab_size=256, depth=2, dim=64, num_heads=4, d_qk=16, d_v=16)
    torch.manual_seed(0)
    m = Transformer(cfg).to(torch.bfloat16).eval().requires_grad_(False)
    m.set_hard(True)
    x = torch.randint(0, 256, (2, 48))
    with torch.no_grad():
        ops = _aten_ops(lambda: m(x))
        assert "aten::mm" in ops and "aten::bmm" not in ops, sorted(ops)
        cache = _HostCache(cfg.depth)
        ops = _aten_ops(lambda: m(x, cache=cache))
        assert "aten::bmm" not in ops, sorted(ops)
        tok = torch.zeros(2, 1, dtype=torch.long)

        def step():
            logits = m(tok, cache=cache)
            M.argmax_into(logits, tok)
        ops = _aten_ops(step)
        assert "aten::bmm" not in ops, sorted(ops)
        assert cache.t == 48 + 1


def test_load_trained_reads_a_run_directory(tmp_path):
    """load_trained (code/lema/model.py:420-436): a run directory's model.pt with the config
    as a plain dict (reference-only fields among them) and a state dict holding one entry this
    model does not have; the model comes back with those weights, in hard mode."""
    import dataclasses
    from latest_exact_match_attention_amd.model import load_trained
    cfg = ModelConfig(vocab_size=300, depth=2, dim=64, num_heads=4, d_qk=8, d_v=16)
    torch.manual_seed(3)
    src = Transformer(cfg)
    conf = dataclasses.asdict(cfg) | {"rope_base": 10000.0, "gdn_expand_v": 2}
    sd = dict(src.state_dict()) | {"blocks.0.attn.inner.extra": torch.zeros(3)}
    torch.save({"config": conf, "state_dict": sd, "step": 7}, tmp_path / "model.pt")
    torch.manual_seed(4)                      # a different draw: the weights must come from disk
    m, c = load_trained(tmp_path, device="cpu")
    assert c == cfg and not m.training and all(a.hard for a in m.lema_layers())
    for k, v in src.state_dict().items():
        assert torch.equal(m.state_dict()[k], v), k
    # a checkpoint that needs an arbitrary object to load is refused, not executed
    import fractions
    torch.save({"config": conf, "state_dict": sd, "obj": fractions.Fraction(1, 3)},
               tmp_path / "bad.pt")
    with pytest.raises(Exception, match="[Ww]eights only"):
        load_trained(tmp_path / "bad.pt", device="cpu")
