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


@pytest.mark.parametrize("d", [24, 16, 32, 8])
@pytest.mark.parametrize("B,T", [(16, 1), (4, 3), (1, 32)])
def test_skinny_pack_codes(dev, d, B, T):
    H, K = 64, 1536
    g = torch.Generator(device=dev).manual_seed(d + B)
    x = torch.randn(B, T, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(H * d, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    ct = torch.int32 if d <= 32 else torch.int64
    codes = torch.empty((B, H, T), dtype=ct, device=dev)
    _lib.check(_lib.lib().lema_skinny_pack_bf16(x.data_ptr(), K, w.data_ptr(), K, B * T, H * d, K,
                                                d, T, codes.data_ptr(), codes.element_size(),
                                                _lib.stream_of(x)))
    z = (x.float().reshape(B * T, K) @ w.float().T).view(B, T, H, d).transpose(1, 2)
    want = torch_model.pack(z.to(torch.bfloat16))
    got = codes.long() & ((1 << d) - 1)
    diff = got ^ want
    if diff.any():                                   # only near-zero pre-activations may flip
        bits = ((diff.unsqueeze(-1) >> torch.arange(d, device=dev)) & 1).bool()
        assert (z.abs()[bits] < 1e-3).all()
    assert (diff != 0).float().mean() < 0.01
