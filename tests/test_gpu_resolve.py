"""Parity of the prefill path on the GPU: pack_codes, latest_prev_match, the fused
resolve+gather and the standalone gather, against the CPU oracle and the golden fixtures.
Integer results (codes, indices) and gathered value bits must be identical; NaN payloads
are compared as NaN (the reference multiplies by the 0/1 mask, which may requiet a NaN).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from latest_exact_match_attention_amd import (gather_values, latest_prev_match, lema_from_codes,
                                              lema_hard, pack_codes)
from latest_exact_match_attention_amd.workloads import dense_plumbing, zipf_prefill

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_bf16(a: np.ndarray, dev) -> torch.Tensor:
    """float32 numpy -> bf16 device tensor (round to nearest even, torch's rule)."""
    return torch.from_numpy(a).to(dev).to(torch.bfloat16)


def same_values(got: np.ndarray, want: np.ndarray, dtype: str) -> bool:
    """Bitwise equality, except that any NaN equals any NaN."""
    if dtype == "f32":
        g, w = got.view(np.uint32), want.view(np.uint32)
        gn = np.isnan(got.view(np.float32))
        wn = np.isnan(want.view(np.float32))
    else:
        g, w = got.view(np.uint16), want.view(np.uint16)
        e, m = (0x7F80, 0x7F) if dtype == "bf16" else (0x7C00, 0x3FF)
        gn = ((g & e) == e) & ((g & m) != 0)
        wn = ((w & e) == e) & ((w & m) != 0)
    return bool(np.array_equal(gn, wn) and np.array_equal(g[~gn], w[~wn]))


# ------------------------------------------------------------------------ pack codes
def test_pack_golden(dev):
    g = np.load(GOLDEN / "pack.npz")
    for D in (24, 64):
        z = torch.from_numpy(g[f"z_f32_d{D}"]).to(dev)
        got = pack_codes(z).cpu().numpy().view(np.uint64)
        assert np.array_equal(got, g[f"codes_f32_d{D}"]), D
        for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
            z = torch.from_numpy(g[f"z_{name}_d{D}"].view(np.int16)).to(dev).view(dt)
            got = pack_codes(z).cpu().numpy().view(np.uint64)
            assert np.array_equal(got, g[f"codes_{name}_d{D}"]), (name, D)
            if D <= 32:
                got32 = pack_codes(z, torch.int32).cpu().numpy().view(np.uint32)
                assert np.array_equal(got32.astype(np.uint64), g[f"codes_{name}_d{D}"])


@pytest.mark.parametrize("D", [1, 8, 24, 32, 33, 63, 64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["contiguous", "projection", "sliced"])
@pytest.mark.parametrize("H", [3, 64])
def test_pack_layouts(dev, D, dtype, layout, H):
    """64 heads in the projection layout take the tiled kernel (codes staged per workgroup,
    77 positions: tiles cross the batch boundary and the last one is partial)."""
    B, T = 2, 77
    gen = torch.Generator(device="cpu").manual_seed(D * 7 + H)
    specials = torch.tensor([0.0, -0.0, float("nan"), float("inf"), -float("inf")]).to(dtype)
    if layout == "contiguous":
        base = torch.randn(B, H, T, D, generator=gen).to(dtype)
        base.view(-1)[:5] = specials
        z = base
    elif layout == "projection":          # [B, T, H*D] viewed as [B, H, T, D]
        base = torch.randn(B, T, H * D, generator=gen).to(dtype)
        base.view(-1)[:5] = specials
        z = base.view(B, T, H, D).transpose(1, 2)
    else:                                 # every other position: not one packed array
        base = torch.randn(B, H, 2 * T, D, generator=gen).to(dtype)
        base.view(-1)[:5] = specials
        z = base[:, :, ::2]
    zd = base.to(dev)
    zd = zd if layout == "contiguous" else (
        zd.view(B, T, H, D).transpose(1, 2) if layout == "projection" else zd[:, :, ::2])
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    zc = z.contiguous()
    carrier = zc.numpy() if dtype == torch.float32 else zc.view(torch.int16).numpy().view(np.uint16)
    want = oracle.pack_codes(carrier, name)
    got = pack_codes(zd).cpu().numpy().view(np.uint64)
    assert np.array_equal(got, want)
    if D <= 32:
        got32 = pack_codes(zd, torch.int32).cpu().numpy().view(np.uint32)
        assert np.array_equal(got32.astype(np.uint64), want)


@pytest.mark.parametrize("D,code_dtype", [(24, torch.int32), (64, torch.int64)])
def test_pack_projection_large(dev, D, code_dtype):
    """The tiled kernel's larger tiles (inputs of 2^21 rows or more): B1 H64 T32845 in the
    projection layout, the last tile partial."""
    B, H, T = 1, 64, 32845
    assert B * H * T >= 1 << 21
    gen = torch.Generator(device="cpu").manual_seed(D)
    base = torch.randn(B, T, H * D, generator=gen).to(torch.bfloat16)
    base.view(-1)[:5] = torch.tensor([0.0, -0.0, float("nan"), float("inf"), -float("inf")]).to(torch.bfloat16)
    zd = base.to(dev).view(B, T, H, D).transpose(1, 2)
    carrier = base.view(B, T, H, D).transpose(1, 2).contiguous().view(torch.int16).numpy().view(np.uint16)
    want = oracle.pack_codes(carrier, "bf16")
    got = pack_codes(zd, code_dtype).cpu().numpy()
    got = got.view(np.uint32).astype(np.uint64) if code_dtype == torch.int32 else got.view(np.uint64)
    assert np.array_equal(got, want)


def test_pack_generic_shape(dev):
    z = torch.randn(5, 7, 3, 9, 12)
    got = pack_codes(z.to(dev)).cpu().numpy().view(np.uint64)
    assert got.shape == (5, 7, 3, 9)
    assert np.array_equal(got, oracle.pack_codes(z.numpy(), "f32"))


# ------------------------------------------------------------------ latest prev match
def test_latest_match_golden(dev):
    g = np.load(GOLDEN / "latest_match.npz")
    qc, kc = torch.from_numpy(g["qc"]).to(dev), torch.from_numpy(g["kc"]).to(dev)
    assert np.array_equal(latest_prev_match(qc, kc).cpu().numpy(), g["src"])
    got32 = latest_prev_match(qc, kc, out_dtype=torch.int32).cpu().numpy()
    assert np.array_equal(got32.astype(np.int64), g["src"])


@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 1023, 1024, 1025, 2049, 5000])
@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_latest_match_random(dev, T, code_dtype):
    rng = np.random.default_rng(T)
    for N, alpha in ((1, 3), (3, 50), (9, 5000)):
        qc = rng.integers(0, alpha, (N, T))
        kc = rng.integers(0, alpha, (N, T))
        want = oracle.latest_prev_match(qc, kc)
        got = latest_prev_match(torch.from_numpy(qc).to(dev).to(code_dtype),
                                torch.from_numpy(kc).to(dev).to(code_dtype))
        assert np.array_equal(got.cpu().numpy(), want), (N, alpha)


@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_latest_match_all_ones_code(dev, code_dtype):
    """The all-ones pattern is the kernel's empty-slot marker; as a code it must still
    behave like any other (chunks of 1024 positions, so T = 3000 crosses two boundaries)."""
    rng = np.random.default_rng(1)
    T = 3000
    qc = rng.choice([-1, 0, 1, 7], size=(4, T))
    kc = rng.choice([-1, 0, 1, 9], size=(4, T))
    qc[1] = -1
    kc[1, :] = 5
    kc[1, 1500] = -1
    want = oracle.latest_prev_match(qc, kc)
    got = latest_prev_match(torch.from_numpy(qc).to(dev).to(code_dtype),
                            torch.from_numpy(kc).to(dev).to(code_dtype)).cpu().numpy()
    assert np.array_equal(got, want)
    assert (got[1, 1501:] == 1500).all() and (got[1, :1501] == -1).all()


def test_latest_match_mixed_widths_zero_extend(dev):
    """An int32 code is its 32-bit pattern: mixed with int64 codes it must match the int64
    code below 2^32 with the same bits, also when bit 31 is set (half of all 32-bit codes),
    never the sign-extended negative int64."""
    rng = np.random.default_rng(31)
    T = 3000
    pats = (np.arange(40, dtype=np.int64) * 0x9E3779B1) & 0xFFFFFFFF
    assert (pats >= 1 << 31).any() and (pats < 1 << 31).any()
    qc = rng.choice(pats, size=(3, T))
    kc = rng.choice(pats, size=(3, T))
    kc[2, ::5] -= 1 << 32          # sign-extended twins: these keys must NOT match
    want = oracle.latest_prev_match(qc, kc)
    q32 = torch.from_numpy(qc.astype(np.uint32).view(np.int32)).to(dev)
    k64 = torch.from_numpy(kc).to(dev)
    got = latest_prev_match(q32, k64).cpu().numpy()
    assert np.array_equal(got, want)
    assert (got >= 0).mean() > 0.5
    got = latest_prev_match(torch.from_numpy(kc).to(dev), q32).cpu().numpy()
    assert np.array_equal(got, oracle.latest_prev_match(kc, qc))


def test_latest_match_structured_rows(dev):
    T = 4100
    i = np.arange(T)
    qc = np.stack([np.full(T, 3), i, i - 3, i // 700, (i * 2654435761) % 4096])
    kc = np.stack([np.full(T, 3), i, i, i // 700, (i * 2246822519) % 4096])
    want = oracle.latest_prev_match(qc, kc)
    got = latest_prev_match(torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev))
    assert np.array_equal(got.cpu().numpy(), want)
    assert (want[0] == i - 1).all() and (want[1] == -1).all()


def test_empty_and_tiny(dev):
    e = torch.empty((3, 0), dtype=torch.int64, device=dev)
    assert latest_prev_match(e, e).shape == (3, 0)
    one = torch.tensor([[5]], device=dev)
    assert latest_prev_match(one, one).item() == -1
    v = torch.randn(1, 1, 1, 8, device=dev)
    y = lema_from_codes(one.view(1, 1, 1), one.view(1, 1, 1), v)
    assert (y == 0).all()


# ------------------------------------------------------------------- fused + gather
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("miss", ["dense", "zero"])
def test_gather_golden(dev, dtype, miss):
    g = np.load(GOLDEN / "gather.npz")
    src = torch.from_numpy(g["src"]).to(dev)
    N, T, dv = g["v_f32"].shape
    if dtype == "f32":
        v = torch.from_numpy(g["v_f32"]).to(dev)
    else:
        v = torch.from_numpy(g["v_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
    y = gather_values(v.view(1, N, T, dv), src.view(1, N, T), miss=miss)
    got = y.cpu().numpy() if dtype == "f32" else bits16(y)
    want = g[f"y_{dtype}_{miss}"]
    assert same_values(got.reshape(want.shape), want, dtype)
    y32 = gather_values(v.view(1, N, T, dv), src.view(1, N, T).to(torch.int32), miss=miss)
    assert torch.equal(y32.view(torch.uint8), y.view(torch.uint8))


@pytest.mark.parametrize("dv,dtype", [(1, "bf16"), (3, "bf16"), (5, "f32"), (40, "bf16"),
                                      (100, "f32"), (1100, "f32"), (2100, "bf16")])
def test_value_row_shapes(dev, dv, dtype):
    """Value rows of 2 B to 4.4 KB through the fused path and the standalone gather: pieces of
    2, 4, 8 and 16 bytes, piece counts that leave threads of the workgroup idle (3, 5, 25),
    and rows of more than 256 pieces (275 and 525: the strided copy). Row 0 holds -0, NaN and
    -inf, the dense miss fill's source."""
    B, H, T = 1, 3, 1500
    rng = np.random.default_rng(dv)
    qc = rng.integers(0, 1000, size=(B, H, T)).astype(np.int32)
    kc = rng.integers(0, 1000, size=(B, H, T)).astype(np.int32)
    v32 = rng.standard_normal((B, H, T, dv)).astype(np.float32)
    v32[:, :, 0, 0] = -0.0
    if dv > 1:
        v32[:, :, 0, 1] = np.nan
    if dv > 2:
        v32[:, :, 0, 2] = -np.inf
    v = torch.from_numpy(v32).to(dev)
    if dtype == "bf16":
        v = v.to(torch.bfloat16)

    def carrier(t):
        t = t.contiguous().cpu()
        return t.numpy() if dtype == "f32" else t.view(torch.int16).numpy().view(np.uint16)

    q, k = torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)
    y, src = lema_from_codes(q, k, v, return_src=True)
    want_src = oracle.latest_prev_match(qc.reshape(B * H, T), kc.reshape(B * H, T))
    assert np.array_equal(src.cpu().numpy().reshape(B * H, T), want_src)
    vc = carrier(v).reshape(B * H, T, dv)
    want = oracle.gather(vc, dtype, want_src, 0)
    assert same_values(carrier(y).reshape(want.shape), want, dtype)
    assert 0.2 < (want_src < 0).mean() < 0.8  # both copies and misses
    for miss, mode in (("dense", 0), ("zero", 1)):
        yg = gather_values(v, src, miss=miss)
        want = oracle.gather(vc, dtype, want_src, mode)
        assert same_values(carrier(yg).reshape(want.shape), want, dtype), miss


@pytest.mark.parametrize("N,T,code_dtype,dv", [
    (72, 27000, torch.int32, 24),    # 1944 items on 976 workgroups: some take 2, some 1
    (64, 29500, torch.int32, 64),    # grouped order, a partial last chunk
    (100, 29000, torch.int32, 64),   # 2900 items, 3 per workgroup, 128-byte value rows
    (128, 12000, torch.int64, 32),   # 8-byte codes: 3 workgroups per CU
    (16, 131072, torch.int32, 8),    # 128 chunks per row: the chunk summaries
])
def test_persistent_copy_shapes(dev, N, T, code_dtype, dv):
    """Shapes with more chunks than the GPU holds workgroups at once, where one workgroup
    resolves and copies several chunks (half of them copying each chunk one item late):
    indices and values against the oracle."""
    rng = np.random.default_rng(N + T)
    alpha = T // 2  # about 43% misses
    qc = rng.integers(0, alpha, size=(1, N, T))
    kc = rng.integers(0, alpha, size=(1, N, T))
    v = torch.from_numpy(rng.standard_normal((1, N, T, dv)).astype(np.float32)).to(dev)
    v = v.to(torch.bfloat16)
    q = torch.from_numpy(qc).to(dev).to(code_dtype)
    k = torch.from_numpy(kc).to(dev).to(code_dtype)
    y, src = lema_from_codes(q, k, v, return_src=True)
    want_src = oracle.latest_prev_match(qc.reshape(N, T), kc.reshape(N, T))
    assert np.array_equal(src.cpu().numpy().reshape(N, T), want_src)
    vc = bits16(v).reshape(N, T, dv)
    want = oracle.gather(vc, "bf16", want_src, 0)
    assert same_values(bits16(y).reshape(want.shape), want, "bf16")
    assert 0.05 < (want_src < 0).mean() < 0.95


def test_persistent_copy_in_a_graph(dev):
    """The fused op captured in a HIP graph on a shape that takes the persistent kernel (1944
    items): every replay, with eager work between them, equals the eager result."""
    N, T, dv = 72, 27000, 24
    rng = np.random.default_rng(5)
    q = torch.from_numpy(rng.integers(0, T // 2, size=(1, N, T))).to(dev).to(torch.int32)
    k = torch.from_numpy(rng.integers(0, T // 2, size=(1, N, T))).to(dev).to(torch.int32)
    v = torch.randn(1, N, T, dv, device=dev).to(torch.bfloat16)
    want, want_src = lema_from_codes(q, k, v, return_src=True)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up on the capturing stream
        lema_from_codes(q, k, v, return_src=True)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y, src = lema_from_codes(q, k, v, return_src=True)
    for rep in range(3):
        y.zero_()
        src.fill_(-7)
        noise = torch.randn(1 << 20, device=dev).sum()  # eager work between the replays
        g.replay()
        torch.cuda.synchronize(dev)
        assert torch.isfinite(noise)
        assert torch.equal(src, want_src), rep
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), rep


def test_dense_plumbing_workload(dev):
    """B1 H8 T4096, 16-bit codes, fp32 values: indices and outputs bit-exact."""
    qc, kc, v = dense_plumbing(0)
    want_src = oracle.latest_prev_match(qc.reshape(8, -1), kc.reshape(8, -1))
    want_y = oracle.gather(v.reshape(8, 4096, 64), "f32", want_src, 0)
    for ct in (torch.int64, torch.int32):
        y, src = lema_from_codes(torch.from_numpy(qc).to(dev).to(ct),
                                 torch.from_numpy(kc).to(dev).to(ct),
                                 torch.from_numpy(v).to(dev), return_src=True)
        assert np.array_equal(src.cpu().numpy().reshape(8, -1), want_src)
        assert same_values(y.cpu().numpy().reshape(8, 4096, 64), want_y, "f32")
    assert (want_src >= 0).sum() > 100          # the workload does produce matches


def test_zipf_prefill_full_size(dev):
    """B8 H16 T16384, Zipf 24-bit codes, d_v 64 bf16 -- the benchmark workload at its real
    size: every index and every output bit against the oracle."""
    qc, kc, v = zipf_prefill(0)
    N, T = 128, 16384
    want_src = oracle.latest_prev_match(qc.reshape(N, T), kc.reshape(N, T))
    vb = to_bf16(v, dev)
    y, src = lema_from_codes(torch.from_numpy(qc).to(dev).to(torch.int32),
                             torch.from_numpy(kc).to(dev).to(torch.int32), vb,
                             return_src=True)
    assert np.array_equal(src.cpu().numpy().reshape(N, T), want_src)
    want_y = oracle.gather(bits16(vb).reshape(N, T, 64), "bf16", want_src, 0)
    assert same_values(bits16(y).reshape(N, T, 64), want_y, "bf16")
    hit = (want_src >= 0).mean()
    assert 0.8 < hit < 0.95          # Zipf(1.1) over 4096 codes: 86.6% of queries match


@pytest.mark.parametrize("D", [24, 40])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_lema_hard_end_to_end(dev, D, dtype):
    """pack -> resolve -> gather from pre-activations laid out like the projections
    ([B, T, H*D] viewed as [B, H, T, D]); few distinct codes so matches are common."""
    B, H, T, dv = 2, 4, 1500, 24
    gen = torch.Generator().manual_seed(D)
    base = torch.randn(B, T, H, 3, generator=gen)
    # only 3 free signs per row: ~8 distinct codes per head, many matches
    zq = base.repeat_interleave(-(-D // 3), dim=-1)[..., :D].reshape(B, T, H * D)
    zk = torch.roll(base, 5, dims=1).repeat_interleave(-(-D // 3), dim=-1)[..., :D]
    zk = zk.reshape(B, T, H * D)
    v = torch.randn(B, T, H * dv, generator=gen)
    q4 = zq.to(dtype).view(B, T, H, D).transpose(1, 2)
    k4 = zk.to(dtype).view(B, T, H, D).transpose(1, 2)
    v4 = v.to(dtype).view(B, T, H, dv).transpose(1, 2)
    y = lema_hard(q4.to(dev), k4.to(dev), v4.to(dev))
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]

    def carrier(t):
        t = t.contiguous()
        return t.numpy() if dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)

    qc = oracle.pack_codes(carrier(q4), name).reshape(B * H, T)
    kc = oracle.pack_codes(carrier(k4), name).reshape(B * H, T)
    src = oracle.latest_prev_match(qc, kc)
    want = oracle.gather(carrier(v4).reshape(B * H, T, dv), name, src, 0)
    got = carrier(y.cpu())
    assert same_values(got.reshape(want.shape), want, name)
    assert (src >= 0).mean() > 0.5


def test_lema_hard_value_gradient(dev):
    """d/dv of sum(y * w): each source row collects the weights of the queries it serves."""
    B, H, T, D, dv = 1, 2, 300, 8, 4
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, T, D, generator=gen).sign()
    q[..., 2:] = 1.0
    k = torch.roll(q, 1, dims=2)
    v = torch.randn(B, H, T, dv, generator=gen)
    w = torch.randn(B, H, T, dv, generator=gen)
    vd = v.to(dev).requires_grad_(True)
    y = lema_hard(q.to(dev), k.to(dev), vd)
    (y * w.to(dev)).sum().backward()
    qc = oracle.pack_codes(q.numpy(), "f32").reshape(B * H, T)
    kc = oracle.pack_codes(k.numpy(), "f32").reshape(B * H, T)
    src = oracle.latest_prev_match(qc, kc)
    want = np.zeros((B * H, T, dv), dtype=np.float64)
    for n in range(B * H):
        for i in range(T):
            if src[n, i] >= 0:
                want[n, src[n, i]] += w.numpy().reshape(B * H, T, dv)[n, i]
    np.testing.assert_allclose(vd.grad.cpu().numpy().reshape(B * H, T, dv), want,
                               rtol=1e-5, atol=1e-5)


def test_runs_on_current_stream(dev):
    qc, kc, v = dense_plumbing(3, T=2048)
    s = torch.cuda.Stream()
    a, b, vv = (torch.from_numpy(x).to(dev) for x in (qc, kc, v))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        y, src = lema_from_codes(a, b, vv, return_src=True)
    s.synchronize()
    want = oracle.latest_prev_match(qc.reshape(8, -1), kc.reshape(8, -1))
    assert np.array_equal(src.cpu().numpy().reshape(8, -1), want)


# --------------------------------------------------- chunk-summary path (workspace entries)
def resolve_c(qc: torch.Tensor, kc: torch.Tensor, ws: bool) -> np.ndarray:
    """latest_prev_match through the C ABI: the backward scan (no workspace) or the chunk
    summaries (lema_latest_prev_match_ws)."""
    from latest_exact_match_attention_amd import _lib
    N, T = qc.shape
    src = torch.empty((N, T), dtype=torch.int64, device=qc.device)
    L, st = _lib.lib(), _lib.stream_of(qc)
    if ws:
        n = L.lema_resolve_workspace_bytes(N, T)
        w = torch.empty(max(n, 1), dtype=torch.uint8, device=qc.device)
        _lib.check(L.lema_latest_prev_match_ws(qc.data_ptr(), kc.data_ptr(), qc.element_size(), N,
                                               T, src.data_ptr(), 8, w.data_ptr() if n else None,
                                               n, st))
    else:
        _lib.check(L.lema_latest_prev_match(qc.data_ptr(), kc.data_ptr(), qc.element_size(), N, T,
                                            src.data_ptr(), 8, st))
    return src.cpu().numpy()


def both_paths(qc: np.ndarray, kc: np.ndarray, dev, code_dtype) -> np.ndarray:
    q = torch.from_numpy(qc).to(dev).to(code_dtype)
    k = torch.from_numpy(kc).to(dev).to(code_dtype)
    want = oracle.latest_prev_match(qc, kc)
    assert np.array_equal(resolve_c(q, k, ws=False), want)
    assert np.array_equal(resolve_c(q, k, ws=True), want)
    return want


LONG = 64 * 1024 + 464          # rows of 65 chunks (ragged last chunk) take the summaries


@pytest.mark.parametrize("T", [64 * 1024 - 1024, 64 * 1024 - 1023, LONG])
@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_summary_path_equals_scan(dev, T, code_dtype):
    """Rows at the summaries' threshold (64 chunks) and past it, ragged last chunk included:
    both paths equal the oracle, on few-code rows (matches within a chunk), many-code rows
    (matches across chunks; past the threshold these chunks scan through the queue), far
    copies (matches many chunks back) and rows of ~690 distinct codes per chunk (the filter's
    chunks that still read the summaries)."""
    from latest_exact_match_attention_amd import _lib
    assert (_lib.lib().lema_resolve_workspace_bytes(5, T) > 0) == (T > 63 * 1024)
    rng = np.random.default_rng(T)
    rows = [rng.integers(0, 7, T), rng.integers(0, 30000, T), rng.integers(-2, 2, T)]
    far = rng.integers(0, 1 << 31, T)
    far[T // 2:] = far[:T - T // 2]          # every key of the second half repeats one
    rows.append(far)
    rows.append(rng.integers(0, 1200, T))
    kc = np.stack(rows)
    i = np.arange(T)
    # row 3: query i >= T/2 asks for the key of i - T/2 (its copy at i itself is not < i)
    q3 = np.where(i >= T // 2, far[np.maximum(i - T // 2, 0)], rng.integers(0, 1 << 31, T))
    qc = np.stack([rng.integers(0, 7, T), rng.integers(0, 30000, T), rng.integers(-2, 2, T), q3,
                   rng.integers(0, 1200, T)])
    want = both_paths(qc, kc, dev, code_dtype)
    assert (want[3] >= 0).mean() > 0.4


def test_summary_fold_collisions(dev):
    """64-bit codes x and x ^ (m << 32 | m) fold to the same 32 bits, so they share the
    summary bucket and fingerprint: only the check against the key code tells them apart."""
    T, m, late = LONG, 0x5A5A5A5A, 40 * 1024
    rng = np.random.default_rng(3)
    base = rng.integers(1, 1 << 62, 40)
    twin = base ^ ((m << 32) | m)
    pool = np.concatenate([base, twin])
    kc = pool[rng.integers(0, 80, (3, T))]
    qc = pool[rng.integers(0, 80, (3, T))]
    kc[2, late:] = twin[0]                    # row 2: late keys are all the twin of base[0]
    qc[2, late:] = base[0]                    # so base[0] is found before chunk 40 only
    want = both_paths(qc, kc, dev, torch.int64)
    assert (want[2, late + 1:] < late).all() and (want[2, late + 1:] >= 0).all()


def _fib_bucket(x):
    return ((x * 0x9E3779B1) & 0xFFFFFFFF) * 512 >> 32


def _fingerprint(h):
    h = h ^ (h >> 16)
    h = (h * 0x85EBCA6B) & 0xFFFFFFFF
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & 0xFFFFFFFF
    h ^= h >> 16
    f = h >> 10
    return np.where(f == 0x3FFFFF, 0x3FFFFE, f)


def test_summary_fingerprint_collisions(dev):
    """32-bit codes with the same summary bucket and fingerprint (found by brute force): a
    chunk holding one of them must not answer for the other."""
    rng = np.random.default_rng(5)
    x = np.unique(rng.integers(0, 1 << 32, 1 << 21, dtype=np.uint64))
    key = (_fib_bucket(x) << 22) | _fingerprint(x)
    order = np.argsort(key, kind="stable")
    ks = key[order]
    dup = np.nonzero(ks[1:] == ks[:-1])[0]
    pairs = [(int(x[order[i]]), int(x[order[i + 1]])) for i in dup]
    pairs = [(a, b) for a, b in pairs if min(a, b) >= 1 << 20][:6]   # apart from the filler
    assert len(pairs) == 6
    T = LONG
    kc = np.zeros((len(pairs), T), dtype=np.int64)
    qc = np.zeros((len(pairs), T), dtype=np.int64)
    for r, (a, b) in enumerate(pairs):
        kc[r] = rng.integers(0, 1 << 20, T)
        kc[r, 100] = a                         # a early (chunk 0), b in every later chunk
        kc[r, 1024::512] = b
        qc[r] = rng.integers(0, 1 << 20, T)
        qc[r, 2048::7] = a
    want = both_paths(qc.astype(np.uint32).view(np.int32).astype(np.int64),
                      kc.astype(np.uint32).view(np.int32).astype(np.int64), dev, torch.int32)
    assert (want[:, 2048::7] == 100).all()


def test_summary_full_buckets(dev):
    """Chunks of 1024 distinct uniform 32-bit keys (summary tables at load 1/2, so some
    buckets are full and probes continue), queries copying keys from any earlier chunk."""
    rng = np.random.default_rng(9)
    T = LONG
    kc = rng.integers(0, 1 << 32, (3, T), dtype=np.uint64).astype(np.uint32).view(np.int32)
    back = rng.integers(1, T, (3, T))
    i = np.arange(T)
    qc = np.where(i - back >= 0, np.take_along_axis(kc, np.maximum(i - back, 0), 1), 12345)
    qc = qc.astype(np.int32)
    want = both_paths(qc.astype(np.int64), kc.astype(np.int64), dev, torch.int32)
    assert (want >= 0).mean() > 0.45


@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_summary_all_ones_code(dev, code_dtype):
    """The all-ones code is the summary tables' empty marker and is kept apart; as a code it
    is found across chunks like any other."""
    T = LONG
    rng = np.random.default_rng(2)
    kc = rng.choice([-1, 0, 1, 9], size=(3, T))
    qc = rng.choice([-1, 0, 1, 7], size=(3, T))
    kc[1] = 5
    kc[1, 1500] = -1                           # the only all-ones key of row 1, in chunk 1
    qc[1] = -1
    kc[2] = 5
    kc[2, 65000] = -1
    qc[2, :] = -1
    want = both_paths(qc, kc, dev, code_dtype)
    assert (want[1, 1501:] == 1500).all()
    assert (want[2, 65001:] == 65000).all() and (want[2, :65001] == -1).all()


def test_hard_ws_equals_hard(dev):
    """lema_hard_ws (summaries + fused gather) writes the same y and src bytes as lema_hard."""
    from latest_exact_match_attention_amd import _lib
    from latest_exact_match_attention_amd.attention import resolve_workspace
    B, H, T, dv = 1, 3, LONG, 24
    rng = np.random.default_rng(4)
    qc = torch.from_numpy(rng.integers(0, 900, (B * H, T))).to(dev).to(torch.int32)
    kc = torch.from_numpy(rng.integers(0, 900, (B * H, T))).to(dev).to(torch.int32)
    v = torch.randn(B, H, T, dv, device=dev, dtype=torch.bfloat16)
    outs = []
    for ws in (None, resolve_workspace(B * H, T, dev)):
        y = torch.empty_like(v)
        src = torch.empty((B, H, T), dtype=torch.int32, device=dev)
        args = [qc.data_ptr(), kc.data_ptr(), 4, v.data_ptr(), _lib.DTYPE_CODE[v.dtype], B, H, T,
                dv, *v.stride()[:3], y.data_ptr(), *y.stride()[:3], _lib.MISS_DENSE,
                src.data_ptr(), 4]
        if ws is None:
            _lib.check(_lib.lib().lema_hard(*args, _lib.stream_of(v)))
        else:
            _lib.check(_lib.lib().lema_hard_ws(*args, ws.data_ptr(), ws.numel(),
                                               _lib.stream_of(v)))
        outs.append((y, src))
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    want = oracle.latest_prev_match(qc.cpu().numpy(), kc.cpu().numpy())
    assert np.array_equal(outs[1][1].cpu().numpy().reshape(B * H, T), want)


def test_summary_workspace_too_small(dev):
    from latest_exact_match_attention_amd import _lib
    N, T = 2, LONG
    q = torch.zeros((N, T), dtype=torch.int32, device=dev)
    src = torch.empty((N, T), dtype=torch.int64, device=dev)
    n = _lib.lib().lema_resolve_workspace_bytes(N, T)
    w = torch.empty(n, dtype=torch.uint8, device=dev)
    rc = _lib.lib().lema_latest_prev_match_ws(q.data_ptr(), q.data_ptr(), 4, N, T, src.data_ptr(),
                                              8, w.data_ptr(), n - 256, _lib.stream_of(q))
    assert rc != 0 and b"workspace" in _lib.lib().lema_last_error()


@pytest.mark.parametrize("T", [2500, 4096])
@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("alphabet", [1 << 24, 40])
def test_grouped_rows_interleaved_y(dev, T, code_dtype, alphabet):
    """64 heads (rows in whole groups of 64: the grouped workgroup order) with v and y viewed
    from [B, T, H * dv] like the projections (y rows interleaved: plain stores merged in L2),
    codes that seldom repeat (the key filter on) or often (off): y and src bit-exact."""
    B, H, dv = 2, 64, 24
    rng = np.random.default_rng(T + alphabet)
    qc = rng.integers(0, alphabet, (B * H, T))
    kc = rng.integers(0, alphabet, (B * H, T))
    qc[:, T // 2::5] = kc[:, T // 3: T // 3 + len(range(T // 2, T, 5))]   # some far matches
    vp = torch.randn(B, T, H * dv, device=dev).to(torch.bfloat16)
    v = vp.view(B, T, H, dv).transpose(1, 2)
    y, src = lema_from_codes(torch.from_numpy(qc).to(dev).to(code_dtype).view(B, H, T),
                             torch.from_numpy(kc).to(dev).to(code_dtype).view(B, H, T), v,
                             return_src=True)
    want_src = oracle.latest_prev_match(qc, kc)
    assert np.array_equal(src.cpu().numpy().reshape(B * H, T), want_src)
    vb = bits16(v).reshape(B * H, T, dv)
    want_y = oracle.gather(vb, "bf16", want_src, 0)
    assert same_values(bits16(y).reshape(B * H, T, dv), want_y, "bf16")
    assert (want_src >= 0).any()


@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_queued_scan_high_cardinality_rows(dev, code_dtype):
    """Chunks whose query codes seldom repeat (more than 512 distinct: the filtered, queued
    scan of earlier keys): queries copy keys from 1 to 15 chunks back, one hot code fills a
    third of row 1's keys (queues overflow and are looked up many times), the all-ones code
    appears as key and query, row 2 has no repeats at all and row 3 repeats only keys of
    earlier chunks; every index equals the oracle's, through the fused op and the resolver
    alone."""
    rng = np.random.default_rng(77)
    N, T = 3, 16384
    hi = (1 << 40) if code_dtype == torch.int64 else 0
    qc = rng.integers(0, 1 << 24, (N, T)) + hi
    kc = rng.integers(0, 1 << 24, (N, T)) + hi
    for r in range(2):
        i = rng.integers(1024, T, 3000)
        back = rng.integers(1, i)
        qc[r, i] = kc[r, i - back]              # matches at every distance
    hot = 12345 + hi
    kc[1, rng.random(T) < 0.33] = hot
    qc[1, rng.integers(0, T, 40)] = hot
    kc[0, rng.integers(0, T, 50)] = -1
    qc[0, rng.integers(0, T, 50)] = -1
    # row 3: queries copy keys of earlier chunks only, so its chunks answer from before
    # themselves alone
    q3 = rng.integers(0, 1 << 24, (1, T)) + hi
    k3 = rng.integers(0, 1 << 24, (1, T)) + hi
    i = rng.integers(1024, T, 4000)
    q3[0, i] = k3[0, rng.integers(0, i - i % 1024)]
    qc, kc = np.concatenate([qc, q3]), np.concatenate([kc, k3])
    N = 4
    want = oracle.latest_prev_match(qc, kc)
    # Both kinds of filtered chunk are present: chunks none of whose keys carries one of their
    # query codes (answered from before the chunk alone, without the key map), among them
    # chunks with answers from earlier chunks, and chunks with in-chunk matches.
    kinds = {"keyless": 0, "keyless_answered": 0, "in_chunk": 0}
    for r in range(N):
        for c0 in range(0, T, 1024):
            shared = np.intersect1d(qc[r, c0:c0 + 1024], kc[r, c0:c0 + 1024]).size > 0
            if not shared:
                kinds["keyless"] += 1
                kinds["keyless_answered"] += int((want[r, c0:c0 + 1024] >= 0).any())
            elif (want[r, c0:c0 + 1024] >= c0).any():
                kinds["in_chunk"] += 1
    assert all(n > 0 for n in kinds.values()), kinds
    q = torch.from_numpy(qc).to(dev).to(code_dtype)
    k = torch.from_numpy(kc).to(dev).to(code_dtype)
    assert np.array_equal(latest_prev_match(q, k).cpu().numpy(), want)
    v = torch.randn(1, N, T, 8, device=dev)
    _, src = lema_from_codes(q.view(1, N, T), k.view(1, N, T), v, return_src=True)
    assert np.array_equal(src.cpu().numpy().reshape(N, T).astype(np.int64), want)
    assert (want[0] >= 0).sum() > 1500 and (want[1] >= 0).sum() > 1500
