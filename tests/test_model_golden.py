"""The model against vectors the reference's own LEMA model wrote (tests/golden/model.npz,
made by tests/golden/make_model_golden.py from code/lema/model.py): the same seed draws the
same parameters bit for bit, and the functional oracle model reproduces the reference's
codes, match indices, logits and loss. CPU only; the GPU half is in test_gpu_model.py."""
import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import torch_model
from latest_exact_match_attention_amd.model import ModelConfig, Transformer

GOLDEN = Path(__file__).resolve().parent / "golden" / "model.npz"
NAMES = ("d16", "d40")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN)


def config(g, name):
    vocab, depth, dim, heads, d_qk, d_v, dim_ff, seed = g[f"{name}/config"].tolist()
    return ModelConfig(vocab_size=vocab, depth=depth, dim=dim, num_heads=heads, d_qk=d_qk,
                       d_v=d_v, dim_ff=dim_ff), seed


def build(g, name):
    """The repository's Transformer at the fixture's geometry and seed, on the CPU."""
    cfg, seed = config(g, name)
    torch.manual_seed(seed)
    return Transformer(cfg), cfg


def tie_k_to_q(sd):
    """The fixture's forward runs with every block's k_proj set to its q_proj."""
    sd = dict(sd)
    for key in list(sd):
        if key.endswith("attn.k_proj.weight"):
            sd[key] = sd[key.replace("k_proj", "q_proj")].clone()
    return sd


def digest(t):
    return hashlib.sha256(t.detach().float().contiguous().numpy().tobytes()).hexdigest()


@pytest.mark.parametrize("name", NAMES)
def test_same_seed_draws_the_reference_parameters(g, name):
    """Names, module order, shapes and every float32 bit of the initial parameters equal
    the reference's Transformer(cfg) after torch.manual_seed(seed)
    (code/lema/model.py:258-281)."""
    m, _ = build(g, name)
    sd = m.state_dict()
    assert list(sd) == g[f"{name}/param_names"].tolist()
    shapes = [list(t.shape) + [0] * (2 - t.dim()) for t in sd.values()]
    assert shapes == g[f"{name}/param_shapes"].tolist()
    assert [digest(t) for t in sd.values()] == g[f"{name}/param_sha256"].tolist()


def run_oracle(g, name, sd=None):
    m, cfg = build(g, name)
    sd = tie_k_to_q(m.state_dict() if sd is None else sd)
    tok = torch.from_numpy(g[f"{name}/tokens"])
    x, y = tok[:, :-1], tok[:, 1:]
    rec = []
    with torch.no_grad():
        h = torch_model.forward_hidden(sd, cfg, x, record=rec)
        logits = torch.nn.functional.linear(h, sd["lm_head.weight"])
        loss = torch_model.loss(sd, cfg, x, y, chunk=16).item()
    return m, cfg, sd, rec, logits, loss


@pytest.mark.parametrize("name", NAMES)
def test_oracle_model_reproduces_the_reference_forward(g, name):
    """The functional oracle model (oracle/torch_model.py) on the fixture's weights and
    tokens: every layer's match indices equal the reference's, the layer-0 codes equal its
    pack_codes, the logits agree to fp32 rounding and the loss within 1e-6 relative."""
    torch.set_num_threads(1)
    m, cfg, sd, rec, logits, loss = run_oracle(g, name)
    src = g[f"{name}/src"]
    assert len(rec) == cfg.depth
    for i, s in enumerate(rec):
        assert np.array_equal(s.numpy(), src[i]), f"layer {i} indices"
    assert (src >= 0).mean() > 0.2          # the fixture exercises matches, not only misses
    x = torch.from_numpy(g[f"{name}/tokens"])[:, :-1]
    B, T = x.shape
    h0 = torch.nn.functional.rms_norm(torch.nn.functional.embedding(x, sd["tok_emb.weight"]),
                                      (cfg.dim,), sd["blocks.0.norm1.weight"], cfg.norm_eps)
    zq = torch.nn.functional.linear(h0, sd["blocks.0.attn.q_proj.weight"])
    qc0 = torch_model.pack(zq.view(B, T, cfg.num_heads, cfg.d_qk).transpose(1, 2))
    assert np.array_equal(qc0.numpy(), g[f"{name}/qc"][0])
    assert np.array_equal(g[f"{name}/qc"][0], g[f"{name}/kc"][0])   # k tied to q
    want = g[f"{name}/logits"]
    assert np.abs(logits.numpy() - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    ref = float(g[f"{name}/loss"])
    assert abs(loss - ref) <= 1e-6 * abs(ref), (loss, ref)


@pytest.mark.parametrize("mistake", ["gate_up_swapped", "o_proj_unscaled", "norm2_weight_doubled"])
def test_fixture_catches_planted_oracle_mistakes(g, mistake):
    """A plausible slip in the model restatement moves the loss far past the 1e-6 bar
    (planted in the oracle's inputs on the CPU): the fixture discriminates."""
    m, cfg = build(g, "d16")
    sd = dict(m.state_dict())
    if mistake == "gate_up_swapped":
        for i in range(cfg.depth):
            p = f"blocks.{i}.mlp."
            sd[p + "gate.weight"], sd[p + "up.weight"] = sd[p + "up.weight"], sd[p + "gate.weight"]
    elif mistake == "o_proj_unscaled":
        for i in range(cfg.depth):
            k = f"blocks.{i}.attn.o_proj.weight"
            sd[k] = sd[k] * (2 * cfg.depth) ** 0.5
    else:
        for i in range(cfg.depth):
            sd[f"blocks.{i}.norm2.weight"] = torch.full_like(sd[f"blocks.{i}.norm2.weight"], 2.0)
    _, _, _, _, _, loss = run_oracle(g, "d16", sd)
    ref = float(g["d16/loss"])
    assert abs(loss - ref) > 1e-4 * abs(ref), (mistake, loss, ref)
