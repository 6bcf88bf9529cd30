"""The analysis consumers on the GPU: trace records against the oracle (pack and the
reference's sort-based latest match), the distinct-code census against its definition, and the
generation state against the dense forward."""
import numpy as np
import pytest
import torch

from oracle import torch_model
from oracle.torch_port import latest_prev_match_sorted
from latest_exact_match_attention_amd.analysis import LemaState, census, prefix_distinct, trace
from latest_exact_match_attention_amd.model import ModelConfig, Transformer

pytestmark = pytest.mark.gpu


def make(dev, dtype=torch.float32, **geo):
    torch.manual_seed(0)
    with torch.device(dev):
        m = Transformer(ModelConfig(**geo))
    m = m.to(dtype).eval().requires_grad_(False)
    m.set_hard(True)
    return m


GEO = dict(vocab_size=64, depth=2, dim=128, num_heads=4, d_qk=5, d_v=32)


def test_trace_records_match_the_oracle(dev):
    m = make(dev, **GEO)
    x = torch.randint(0, 64, (2, 300), device=dev)
    with torch.no_grad():
        logits, recs = trace(m, x)
        assert torch.equal(logits, m(x))
        h = m.tok_emb(x)
        for li, blk in enumerate(m.blocks):
            zq, zk, _ = blk.attn.project(blk.norm1(h))
            qc, kc = torch_model.pack(zq), torch_model.pack(zk)
            assert torch.equal(recs[li]["qc"], qc) and torch.equal(recs[li]["kc"], kc)
            want = latest_prev_match_sorted(qc.reshape(-1, 300), kc.reshape(-1, 300))
            assert torch.equal(recs[li]["src"].reshape(-1, 300), want), li
            assert (recs[li]["src"] >= 0).float().mean() > 0.3
            h = blk(h)


def test_prefix_distinct_is_the_distinct_count(dev):
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 400, size=(5, 3000)).astype(np.int64)
    codes[1] = 7                                   # one code only
    codes[2] = np.arange(3000)                     # all distinct
    got = prefix_distinct(torch.from_numpy(codes).to(dev)).cpu().numpy()
    for h in range(5):
        seen, want = set(), []
        for c in codes[h]:
            seen.add(int(c))
            want.append(len(seen))
        assert np.array_equal(got[h], want), h


def test_census_counts_every_layer(dev):
    m = make(dev, **GEO)
    x = torch.randint(0, 64, (1, 500), device=dev)
    c = census(m, x)
    _, recs = trace(m, x)
    assert c.shape == (2, 4, 500)
    for li in range(2):
        assert torch.equal(c[li], prefix_distinct(recs[li]["kc"][0]))
    assert (c[:, :, 1:] >= c[:, :, :-1]).all() and (c <= 32).all()   # 5-bit codes


def test_lema_state_steps_equal_the_dense_forward(dev):
    """Prefill 40 tokens, then 24 single-token steps: every returned hidden state equals the
    dense forward's at that position (fp32)."""
    m = make(dev, **GEO)
    x = torch.randint(0, 64, (3, 64), device=dev)
    with torch.no_grad():
        dense = m.hidden(x)
        st = LemaState(m, B=3, maxlen=64, device=dev)
        outs = [st.prefill(x[:, :40])]
        for t in range(40, 64):
            outs.append(st.step(x[:, t:t + 1]))
    got = torch.cat(outs, dim=1)
    want = dense[:, 39:]
    assert (got - want).abs().max() <= 1e-4 * want.abs().max()
    assert st.n == 64 and st.cache.entries() > 0
