"""The fused bf16 model segments against the torch ops they replace (plain PyTorch
references: F.silu(g) * u, nn.RMSNorm after a bf16 add, F.cross_entropy on fp32 logits), and
the device copy the benchmark's roofline compares against."""
import pytest
import torch
import torch.nn.functional as F

from latest_exact_match_attention_amd.model import cross_entropy_sum, rms_norm, swiglu

pytestmark = pytest.mark.gpu


def ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units in the last place (same-sign finite values)."""
    ia, ib = a.view(torch.int16).int(), b.view(torch.int16).int()
    return (ia - ib).abs()


def test_swiglu_matches_silu_times_up(dev):
    g = (torch.randn(4096, 6144, device=dev) * 3).to(torch.bfloat16)
    u = torch.randn(4096, 6144, device=dev).to(torch.bfloat16)
    g[0, :6] = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 88.0, -88.0])
    got = swiglu(g, u)
    want = F.silu(g) * u
    fin = torch.isfinite(want)
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    d = ulps(got[fin], want[fin])
    assert (d == 0).float().mean() > 0.999 and d.max() <= 1, (d.max(), (d == 0).float().mean())


@pytest.mark.parametrize("residual", [False, True])
def test_rmsnorm_matches_torch(dev, residual):
    D = 1536
    norm = torch.nn.RMSNorm(D, eps=1e-5).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(D, device=dev))
    x = torch.randn(3000, D, device=dev).to(torch.bfloat16)
    d = torch.randn(3000, D, device=dev).to(torch.bfloat16) if residual else None
    with torch.no_grad():
        h, xo = rms_norm(x, norm, d)
        xr = x + d if residual else x
        assert torch.equal(xo, xr)                       # the bf16 add, exactly
        want = norm(xr)
    # torch rounds x * rsqrt(mean(x^2) + eps) * w to bf16 once, from fp32, as the kernel does;
    # only the order of the mean's fp32 sum differs, which can move a rare element by one ulp
    rel = ((h.float() - want.float()).abs() / want.float().abs().clamp_min(1e-2)).max()
    assert rel <= 2 ** -7, rel                            # within one bf16 rounding
    assert (h == want).float().mean() > 0.9999


def test_cross_entropy_from_bf16_logits(dev):
    V = 50304
    logits = (torch.randn(1000, V, device=dev) * 4).to(torch.bfloat16)
    y = torch.randint(0, V, (1000,), device=dev)
    got = cross_entropy_sum(logits, y)
    want = F.cross_entropy(logits.float(), y, reduction="sum")
    assert abs(got.item() - want.item()) <= 1e-5 * abs(want.item())


@pytest.mark.parametrize("V,scale", [(8, 4.0), (2056, 1.0), (8200, 30.0), (50304, 4.0)])
def test_cross_entropy_rows(dev, V, scale):
    """Every row's loss within 1e-6 of an fp32 cross-entropy, relative to the loss or to 1
    where the loss is smaller (float32 rounding of log S + M - x_t): vocabularies that end
    inside a thread's first or second piece, logits spread from 1 to 30 standard deviations,
    and -inf logits (a masked entry adds nothing, also where a thread's first pieces are
    wholly masked)."""
    from latest_exact_match_attention_amd import _lib
    g = torch.Generator(device=dev).manual_seed(V)
    rows = 37
    logits = (torch.randn(rows, V, device=dev, generator=g) * scale).to(torch.bfloat16)
    y = torch.randint(0, V, (rows,), device=dev, generator=g)
    logits[1, (y[1] + 1) % V] = -float("inf")
    logits[2, :: 3] = -float("inf")
    logits[2, y[2]] = 0.5
    # a contiguous masked block: every logit of some threads' first trips (and, past 4096,
    # whole trips) is -inf
    logits[3, : min(V - 1, 4096 + 8)] = -float("inf")
    logits[3, y[3]] = 1.25
    loss = torch.empty(rows, device=dev, dtype=torch.float32)
    _lib.check(_lib.lib().lema_cross_entropy_bf16(logits.data_ptr(), rows, V, V, y.data_ptr(),
                                                  loss.data_ptr(), _lib.stream_of(logits)))
    want = F.cross_entropy(logits.float(), y, reduction="none")
    rel = ((loss.double() - want.double()).abs() / want.double().abs().clamp_min(1.0)).max()
    assert rel <= 1e-6, rel


@pytest.mark.parametrize("rows", [1, 16, 33])
@pytest.mark.parametrize("V", [50304, 8, 64, 8200])
def test_argmax_equals_torch(dev, rows, V):
    """The decode step's greedy pick against torch.argmax on bf16 logits: planted ties (the
    first index wins), NaNs (above every number, the first one wins) and all -inf rows."""
    from latest_exact_match_attention_amd.model import argmax_into
    g = torch.Generator(device=dev).manual_seed(rows * 7 + V)
    x = torch.randn(rows, V, device=dev, generator=g).to(torch.bfloat16)
    if V >= 64:
        x[0, V // 3] = x[0, V - 5] = 9.0                      # a tie: the lower index
        if rows > 1:
            x[1, V - 1] = float("nan")                          # NaN wins
            x[1, 5] = 100.0
        if rows > 2:
            x[2].fill_(float("-inf"))                           # all -inf: index 0
            x[3 % rows, 7] = x[3 % rows, 3] = float("nan")      # the first NaN
    out = torch.full((rows, 1), -9, dtype=torch.long, device=dev)
    argmax_into(x.view(rows, 1, V), out)
    assert torch.equal(out.view(-1), x.argmax(-1))


def test_embedding_equals_torch(dev):
    """Decode-step embedding rows against nn.Embedding bit for bit; ids outside the table give
    zero rows (where nn.Embedding raises)."""
    from latest_exact_match_attention_amd.model import embed
    emb = torch.nn.Embedding(50304, 1536).to(dev, torch.bfloat16)
    ids = torch.tensor([[0], [50303], [17], [17], [31000]], device=dev)
    got = embed(emb, ids)
    assert torch.equal(got.view(torch.int16), emb(ids).view(torch.int16))
    bad = torch.tensor([[-1], [50304], [3]], device=dev)
    got = embed(emb, bad)
    assert (got[:2] == 0).all() and torch.equal(got[2], emb.weight[3].view(1, -1))


def test_device_copy(dev):
    """lema_device_copy (the roofline's reference copy) copies every byte, also where the last
    32 KB region is partial, and refuses sizes that are not whole 16-byte pieces."""
    from latest_exact_match_attention_amd import _lib
    st = torch.cuda.current_stream(dev).cuda_stream
    for n16 in (1, 2047, 2048, 2049, 70001):
        src = torch.randint(-2**31, 2**31 - 1, (4 * n16,), dtype=torch.int32, device=dev)
        dst = torch.zeros(4 * n16 + 8, dtype=torch.int32, device=dev)
        _lib.check(_lib.lib().lema_device_copy(src.data_ptr(), dst.data_ptr(), 16 * n16, st))
        torch.cuda.synchronize()
        assert torch.equal(dst[:4 * n16], src), n16
        assert not dst[4 * n16:].any(), n16           # nothing written past the end
    with pytest.raises(ValueError):
        _lib.check(_lib.lib().lema_device_copy(src.data_ptr(), dst.data_ptr(), 24, st))
