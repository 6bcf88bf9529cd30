"""The prefill's query and key projections straight to codes (lema_qk_pack_bf16: a persistent
MFMA GEMM whose epilogue packs the signs) against torch's bf16 product packed by the oracle's
pack_codes restatement (code/lema/attention.py:82-97), through the C ABI, and inside the model
with FUSED_QK_PACK set (it is off by default): Attention.forward and a cached prefill in chunks
of 2048 rows give the unfused path's output.

The two products sum in the same order, so the codes are expected to be identical; the stated
binarization tolerance still bounds what may differ: a bit only where its fp32 pre-activation
is within 1e-3 of zero."""
import pytest
import torch

from oracle import torch_model
from latest_exact_match_attention_amd import _lib, code_dtype_for, lema_hard
from latest_exact_match_attention_amd.model import ModelConfig, Transformer

pytestmark = pytest.mark.gpu


def fused_codes(x, wq, wk, d, T):
    M, K = x.shape
    N = wq.shape[0]
    ct = code_dtype_for(d)
    qc = torch.full((M // T, N // d, T), -1, dtype=ct, device=x.device)
    kc = torch.full_like(qc, -1)
    _lib.check(_lib.lib().lema_qk_pack_bf16(
        x.data_ptr(), K, wq.data_ptr(), wk.data_ptr(), K, M, N, K, d, T, qc.data_ptr(),
        kc.data_ptr(), qc.element_size(), _lib.stream_of(x)))
    return qc, kc


def check_against_product(got, x, w, d, T):
    M, _ = x.shape
    N = w.shape[0]
    z = torch.matmul(x, w.T).view(M // T, T, N // d, d).transpose(1, 2)
    want = torch_model.pack(z)                                    # int64, bits [0, d)
    mask = (1 << d) - 1 if d < 64 else -1
    g = got.long() & (0xFFFFFFFF if got.element_size() == 4 else -1)
    if d < 64:
        assert bool(((g >> d) == 0).all()), "bits above d are set"
    diff = (g ^ want) & mask
    if bool((diff != 0).any()):
        zf = (x.float() @ w.float().T).view(M // T, T, N // d, d).transpose(1, 2)
        bits = ((diff.unsqueeze(-1) >> torch.arange(d, device=x.device)) & 1).bool()
        assert (zf.abs()[bits] < 1e-3).all(), zf.abs()[bits].max()


@pytest.mark.parametrize("M,T,K,N,d", [(2048, 2048, 64, 256, 8), (4096, 1024, 128, 512, 32),
                                       (2048, 256, 192, 768, 24), (2048, 512, 128, 256, 64),
                                       (4096, 4096, 64, 1280, 40), (8192, 2048, 1536, 1536, 24),
                                       (2048, 128, 64, 512, 16)])   # streams shorter than a tile
def test_codes_equal_the_packed_product(dev, M, T, K, N, d):
    g = torch.Generator(device=dev).manual_seed(M + N + d)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    x[3].zero_()                                    # z = +0: bit 1
    x[5, 0] = float("nan")                          # NaN: bit 0
    x[7, 1] = float("inf")                          # +-inf, or NaN where a weight is 0
    wq = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    wk = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    wk[0].zero_()
    qc, kc = fused_codes(x, wq, wk, d, T)
    check_against_product(qc, x, wq, d, T)
    check_against_product(kc, x, wk, d, T)
    # rows of x are streams of T positions: row m is (m // T, m % T)
    assert torch.equal(qc[M // T - 1, 0, T - 1].long() & ((1 << d) - 1 if d < 64 else -1),
                       torch_model.pack(torch.matmul(x[-1:], wq[:d].T)).view(()))


def test_shapes_outside_the_tiles_are_refused(dev):
    L = _lib.lib()
    x = torch.zeros(2048, 128, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(256, 128, dtype=torch.bfloat16, device=dev)
    c = torch.zeros(1, 32, 2048, dtype=torch.int32, device=dev)
    s = _lib.stream_of(x)
    ok = L.lema_qk_pack_bf16(x.data_ptr(), 128, w.data_ptr(), w.data_ptr(), 128, 2048, 256, 128,
                             8, 2048, c.data_ptr(), c.data_ptr(), 4, s)
    assert ok == _lib.OK
    for args in ((1024, 256, 128, 8, 1024, 4), (2048, 128, 128, 8, 2048, 4),
                 (2048, 65536 + 256, 128, 8, 2048, 4),
                 (2048, 256, 96, 8, 2048, 4), (2048, 256, 128, 12, 2048, 4),
                 (2048, 256, 128, 40, 2048, 4), (2048, 256, 128, 8, 1000, 4)):
        M, N, K, d, T, cb = args
        rc = L.lema_qk_pack_bf16(x.data_ptr(), 128, w.data_ptr(), w.data_ptr(), 128, M, N, K, d,
                                 T, c.data_ptr(), c.data_ptr(), cb, s)
        assert rc == _lib.BAD_ARG, args


def _model(dev, T):
    cfg = ModelConfig(vocab_size=512, depth=2, dim=256, num_heads=8, dim_ff=512)   # d_qk 32
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            m = Transformer(cfg)
    finally:
        torch.set_default_dtype(prev)
    m.eval().requires_grad_(False)
    m.set_hard(True)
    return m, cfg


def test_attention_forward_equals_the_unfused_path(dev, monkeypatch):
    """Attention.forward on a 2 x 2048-token prefill with FUSED_QK_PACK set takes the fused
    codes; its output equals project + lema_hard + merge bit for bit."""
    import latest_exact_match_attention_amd.model as model_mod
    monkeypatch.setattr(model_mod, "FUSED_QK_PACK", True)
    m, cfg = _model(dev, 2048)
    at = m.blocks[0].attn
    with torch.no_grad():
        x = m.blocks[0].pre_attn(m.tok_emb(torch.randint(0, 512, (2, 2048), device=dev)))
        got = at(x)
        zq, zk, v = at.project(x)
        want = at.merge(lema_hard(zq, zk, v))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_cached_prefill_in_2048_row_chunks(dev, monkeypatch):
    """A cached forward fed 2 x 4096 tokens in chunks of 1024 positions (2048 rows each: with
    FUSED_QK_PACK set, the fused codes in Block.gpu_pre) gives bit for bit the logits and the
    table of the same cached forward with the codes from project + pack_codes; and the dense
    forward's logits within bf16 rounding."""
    import latest_exact_match_attention_amd.model as model_mod
    monkeypatch.setattr(model_mod, "FUSED_QK_PACK", True)
    m, cfg = _model(dev, 4096)
    x = torch.randint(0, 512, (2, 4096), device=dev)

    def cached():
        cache = m.new_cache("hbm", max_cache_len=4096, batch=2)
        parts = [m(x[:, s:s + 1024], cache=cache) for s in range(0, 4096, 1024)]
        return torch.cat(parts, dim=1), cache

    with torch.no_grad():
        dense = m(x)
        fused, c1 = cached()
        monkeypatch.setattr(model_mod, "FUSED_QK_PACK", False)      # no fused codes
        plain, c2 = cached()
    assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(c1.counts(), c2.counts()) and c1.entries() == c2.entries() > 0
    assert (dense.argmax(-1) == fused.argmax(-1)).float().mean() > 0.99
    assert (dense.float() - fused.float()).abs().max() <= 5e-2 * dense.float().abs().max()
