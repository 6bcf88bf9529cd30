"""The skinny MFMA products of decode steps against plain PyTorch fp32 references: y within
one bf16 rounding of the fp32 product, and codes equal to the signs of the rounded product
except where the pre-activation is below 1e-3 in magnitude."""
import pytest
import torch

from oracle import torch_model
from latest_exact_match_attention_amd import _lib

pytestmark = pytest.mark.gpu


def skinny(x, w):
    M, K = x.shape
    N = w.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.lib().lema_skinny_gemm_bf16(x.data_ptr(), K, w.data_ptr(), K, y.data_ptr(),
                                                 N, M, N, K, _lib.stream_of(x)))
    return y


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("N,K", [(1536, 1536), (4608, 1536), (1536, 6144), (50304, 1536), (40, 64)])
def test_skinny_gemm_matches_fp32(dev, M, N, K):
    g = torch.Generator(device=dev).manual_seed(M * 7 + N)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    got = skinny(x, w).float()
    ref = x.float() @ w.float().T
    err = (got - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 1e-5).all(), (err / ref.abs().clamp_min(1e-6)).max()


@pytest.mark.parametrize("d", [24, 16, 32, 8, 64, 40, 48])
@pytest.mark.parametrize("B,T", [(16, 1), (4, 3), (1, 32)])
def test_skinny_pack_codes(dev, d, B, T):
    """Codes of d-bit heads, heads split over 16-column blocks when d is a multiple of 8 (each
    block writes its bytes of the code): the bits match the packed bf16 projection, and the
    bits above d are zero although the buffer starts as all ones."""
    H, K = 64, 1536
    g = torch.Generator(device=dev).manual_seed(d + B)
    x = torch.randn(B, T, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(H * d, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    ct = torch.int32 if d <= 32 else torch.int64
    codes = torch.full((B, H, T), -1, dtype=ct, device=dev)
    _lib.check(_lib.lib().lema_skinny_pack_bf16(x.data_ptr(), K, w.data_ptr(), K, B * T, H * d, K,
                                                d, T, codes.data_ptr(), codes.element_size(),
                                                _lib.stream_of(x)))
    z = (x.float().reshape(B * T, K) @ w.float().T).view(B, T, H, d).transpose(1, 2)
    want = torch_model.pack(z.to(torch.bfloat16))
    raw = codes.long() & 0xFFFFFFFF if ct == torch.int32 else codes.long()
    if d < codes.element_size() * 8:
        assert (raw >> d == 0).all(), "bits above d are set"
    got = raw
    diff = got ^ want
    if diff.any():                                   # only near-zero pre-activations may flip
        bits = ((diff.unsqueeze(-1) >> torch.arange(d, device=dev)) & 1).bool()
        assert (z.abs()[bits] < 1e-3).all()
    assert (diff != 0).float().mean() < 0.01


def pack(x, w, d, T, ct):
    M, K = x.shape
    H = w.shape[0] // d
    codes = torch.empty((M // T, H, T), dtype=ct, device=x.device)
    _lib.check(_lib.lib().lema_skinny_pack_bf16(x.data_ptr(), K, w.data_ptr(), K, M, H * d, K, d,
                                                T, codes.data_ptr(), codes.element_size(),
                                                _lib.stream_of(x)))
    return codes


@pytest.mark.parametrize("d,Nv", [(24, 1536), (16, 1024), (32, 2048), (8, 40), (64, 1536),
                                  (40, 1536), (56, 1536)])
@pytest.mark.parametrize("B,T", [(16, 1), (4, 3), (1, 1)])
def test_skinny_qkv_equals_separate_launches(dev, d, Nv, B, T):
    """The one-launch q/k/v projection gives bit for bit what three launches give (each column
    is summed in the same order whatever the block's width)."""
    H, K = 64, 1536
    g = torch.Generator(device=dev).manual_seed(d * 3 + B)
    x = torch.randn(B * T, K, device=dev, generator=g).to(torch.bfloat16)
    wq, wk = ((torch.randn(H * d, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
              for _ in range(2))
    wv = (torch.randn(Nv, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    ct = torch.int32 if d <= 32 else torch.int64
    qc = torch.full((B, H, T), -1, dtype=ct, device=dev)
    kc = torch.full_like(qc, -1)
    v = torch.empty((B * T, Nv), dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.lib().lema_skinny_qkv_bf16(
        x.data_ptr(), K, wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), K, B * T, H * d, Nv, K, d,
        T, qc.data_ptr(), kc.data_ptr(), qc.element_size(), v.data_ptr(), _lib.stream_of(x)))
    assert torch.equal(qc, pack(x, wq, d, T, ct))
    assert torch.equal(kc, pack(x, wk, d, T, ct))
    assert torch.equal(v.view(torch.int16), skinny(x, wv).view(torch.int16))


@pytest.mark.parametrize("M", [1, 16, 17, 32])
@pytest.mark.parametrize("N,K", [(6144, 1536), (40, 64), (4096, 1024)])
def test_skinny_swiglu_equals_unfused(dev, M, N, K):
    """gate, up and the SwiGLU product in one launch against the two products and the
    elementwise kernel (bit for bit), and against fp32 within bf16 roundings."""
    from latest_exact_match_attention_amd.model import swiglu
    g = torch.Generator(device=dev).manual_seed(M + N)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    wg, wu = ((torch.randn(N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
              for _ in range(2))
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.lib().lema_skinny_swiglu_bf16(x.data_ptr(), K, wg.data_ptr(), wu.data_ptr(),
                                                  K, M, N, K, out.data_ptr(), _lib.stream_of(x)))
    want = swiglu(skinny(x, wg), skinny(x, wu))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    zg, zu = x.float() @ wg.float().T, x.float() @ wu.float().T
    ref = torch.nn.functional.silu(zg) * zu
    assert ((out.float() - ref).abs() <= 2 ** -6 * ref.abs() + 1e-3).all()


@pytest.mark.parametrize("M", [1, 16, 32])
@pytest.mark.parametrize("N,K", [(1536, 6144), (40, 64)])
def test_skinny_gemm_add_residual(dev, M, N, K):
    """y = r + x . w^T with the product rounded to bf16 first, as `x + mlp(h)` in bf16; also
    in place (y aliasing r)."""
    g = torch.Generator(device=dev).manual_seed(M * 5 + N)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    r = torch.randn(M, N, device=dev, generator=g).to(torch.bfloat16)
    want = r + skinny(x, w)
    y = torch.empty_like(r)
    fn = _lib.lib().lema_skinny_gemm_add_bf16
    _lib.check(fn(x.data_ptr(), K, w.data_ptr(), K, r.data_ptr(), y.data_ptr(), N, M, N, K,
                  _lib.stream_of(x)))
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    _lib.check(fn(x.data_ptr(), K, w.data_ptr(), K, r.data_ptr(), r.data_ptr(), N, M, N, K,
                  _lib.stream_of(x)))
    assert torch.equal(r.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("with_d", [True, False])
@pytest.mark.parametrize("M", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("N,K", [(6144, 1536), (40, 64), (1024, 2048)])
def test_skinny_norm_swiglu_equals_unfused(dev, M, N, K, with_d):
    """The MLP's pre-norm inside the gate/up launch against the norm kernel followed by the
    unfused launch, bit for bit (the normalised rows and x + d round alike). Rows that do not
    fit a workgroup's LDS (32 of 2048) are refused on the host."""
    from latest_exact_match_attention_amd.model import rms_norm
    g = torch.Generator(device=dev).manual_seed(M * 3 + N + K)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    d = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16) if with_d else None
    norm = torch.nn.RMSNorm(K, eps=1e-5).to(dev, torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(K, device=dev, generator=g))
    wg, wu = ((torch.randn(N, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
              for _ in range(2))
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    xo = torch.full_like(x, 7.0)
    args = (x.data_ptr(), d.data_ptr() if d is not None else None, norm.weight.data_ptr(), 1e-5,
            xo.data_ptr(), wg.data_ptr(), wu.data_ptr(), K, M, N, K, out.data_ptr(),
            _lib.stream_of(x))
    if M * (K + 8) * 2 + 8 * (16 if M <= 16 else 32) * 33 * 4 > 160 * 1024:
        with pytest.raises(Exception, match="LDS"):
            _lib.check(_lib.lib().lema_skinny_norm_swiglu_bf16(*args))
        return
    _lib.check(_lib.lib().lema_skinny_norm_swiglu_bf16(*args))
    with torch.no_grad():
        h, s = rms_norm(x, norm, d)
    want = torch.empty_like(out)
    _lib.check(_lib.lib().lema_skinny_swiglu_bf16(h.data_ptr(), K, wg.data_ptr(), wu.data_ptr(),
                                                  K, M, N, K, want.data_ptr(), _lib.stream_of(x)))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    if with_d:
        assert torch.equal(xo.view(torch.int16), s.view(torch.int16))
    else:
        assert (xo == 7.0).all()                      # no addend: x_out is left alone


@pytest.mark.parametrize("B", [1, 16])
def test_block_mlp_half_fused_equals_unfused(dev, B):
    """Block.forward's MLP half on a decode step: SwiGLU.forward_normed (norm inside the
    gate/up launch) returns what rms_norm followed by SwiGLU.forward returns, bit for bit."""
    from latest_exact_match_attention_amd.model import SwiGLU, rms_norm
    torch.manual_seed(B)
    mlp = SwiGLU(1536, 4096).to(dev, torch.bfloat16)
    norm = torch.nn.RMSNorm(1536, eps=1e-5).to(dev, torch.bfloat16)
    x = torch.randn(B, 1, 1536, device=dev).to(torch.bfloat16)
    d = torch.randn(B, 1, 1536, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(1536, device=dev))
        got = mlp.forward_normed(x, d, norm)
        h, s = rms_norm(x, norm, d)
        want = mlp(h, residual=s)
    assert got is not None
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("K,d,H", [(1536, 24, 64), (256, 16, 8), (2048, 64, 16), (2048, 12, 8),
                                   (64, 40, 2)])
def test_skinny_norm_qkv_equals_unfused(dev, M, K, d, H):
    """The attention's pre-norm inside the q/k/v launch against the norm kernel followed by the
    q/k/v launch, codes and v bit for bit. Rows that do not fit a workgroup's LDS beside the
    partial sums (32 rows of 2048 with 48-column blocks) are refused on the host."""
    from latest_exact_match_attention_amd.model import rms_norm
    g = torch.Generator(device=dev).manual_seed(M * 5 + K + d)
    T = 1 if M % 2 else 2
    B = M // T
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    norm = torch.nn.RMSNorm(K, eps=1e-5).to(dev, torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(K, device=dev, generator=g))
    wq, wk = ((torch.randn(H * d, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
              for _ in range(2))
    Nv = H * 24
    wv = (torch.randn(Nv, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    ct = torch.int32 if d <= 32 else torch.int64
    qc = torch.full((B, H, T), -1, dtype=ct, device=dev)
    kc = torch.full_like(qc, -1)
    v = torch.empty((M, Nv), dtype=torch.bfloat16, device=dev)
    args = (x.data_ptr(), norm.weight.data_ptr(), 1e-5, wq.data_ptr(), wk.data_ptr(),
            wv.data_ptr(), K, M, H * d, Nv, K, d, T, qc.data_ptr(), kc.data_ptr(),
            qc.element_size(), v.data_ptr(), _lib.stream_of(x))
    blocks = 1 if d % 8 == 0 else next(c for c in (1, 2, 3, 4) if (16 * c) % d == 0)
    if M * (K + 8) * 2 + 8 * (16 if M <= 16 else 32) * (16 * blocks + 1) * 4 > 160 * 1024:
        with pytest.raises(Exception, match="LDS"):
            _lib.check(_lib.lib().lema_skinny_norm_qkv_bf16(*args))
        return
    _lib.check(_lib.lib().lema_skinny_norm_qkv_bf16(*args))
    with torch.no_grad():
        h, _ = rms_norm(x, norm)
    wq_, wk_ = torch.full_like(qc, -1), torch.full_like(kc, -1)
    wv_ = torch.empty_like(v)
    _lib.check(_lib.lib().lema_skinny_qkv_bf16(
        h.data_ptr(), K, wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), K, M, H * d, Nv, K, d, T,
        wq_.data_ptr(), wk_.data_ptr(), wq_.element_size(), wv_.data_ptr(), _lib.stream_of(x)))
    assert torch.equal(qc, wq_) and torch.equal(kc, wk_)
    assert torch.equal(v.view(torch.int16), wv_.view(torch.int16))


@pytest.mark.parametrize("B", [1, 16])
def test_block_attention_input_fused_equals_unfused(dev, B):
    """Block.gpu_pre on a decode step (norm1 inside the q/k/v launch) returns the codes and v
    that rms_norm followed by the q/k/v launch returns, bit for bit."""
    from latest_exact_match_attention_amd.model import Block, ModelConfig, project_qkv
    from latest_exact_match_attention_amd.attention import code_dtype_for
    torch.manual_seed(B)
    cfg = ModelConfig(vocab_size=256, depth=1, dim=1536, num_heads=64)
    blk = Block(cfg).to(dev, torch.bfloat16)
    with torch.no_grad():
        blk.norm1.weight.copy_(1 + 0.1 * torch.randn(1536, device=dev))
    x = torch.randn(B, 1, 1536, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        qc, kc, v = blk.gpu_pre(x)
        want = project_qkv(blk.pre_attn(x), blk.attn, code_dtype_for(cfg.d_qk))
    assert want is not None
    assert torch.equal(qc, want[0]) and torch.equal(kc, want[1])
    assert torch.equal(v.view(torch.int16), want[2].view(torch.int16))
