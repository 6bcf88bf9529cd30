"""Seeded sweeps over mixed shapes, against the CPU oracle.

Sign-pack: each case draws heads, positions, width, dtype, layout and code width, some of them
at 2^21 rows and more; codes must equal the oracle's (code/lema/attention.py:82-97).

Prefill: each case draws batch, heads, length (around chunk boundaries of 1024 positions and
the 64-chunk summary threshold), code alphabet and structure, code width, value width and
dtype, the value layout (contiguous, or the [B, T, H * d_v] projection viewed as [B, H, T,
d_v]) and the miss fill. Indices and value bits must equal the oracle's
(code/lema/attention.py:100-158).

Store: each case draws partitions, a sequence of exchanges over group ranges (decode-sized,
chunked and bulk calls, some insert-only), code width and alphabet with codes 0 and all-ones,
value row width and the final load; outputs, counts and table content must equal one dict per
partition (code/tests/test_store.py:17-41).

Model: small LEMA models of random geometry (code widths up to 64 bits) in fp32 or bf16; the
loss must equal the functional oracle model's and every layer's exact op the sort-based
algorithm's."""
import numpy as np
import pytest
import torch

import oracle
from latest_exact_match_attention_amd import gather_values, latest_prev_match, lema_from_codes

LENGTHS = [1, 2, 63, 64, 1000, 1023, 1024, 1025, 2047, 2048, 3000, 5121, 16383, 16385,
           40000, 64 * 1024 - 1024, 64 * 1024 + 5]
TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
NP_CARRIER = {"f32": np.float32, "bf16": np.uint16, "f16": np.uint16}


def draw_case(seed: int) -> dict:
    rng = np.random.default_rng(seed)
    T = int(rng.choice(LENGTHS))
    H = int(rng.choice([1, 3, 8, 64]))
    B = int(rng.choice([1, 2, 3]))
    while B * H * T > 3_000_000 and (B > 1 or H > 1):   # the oracle stays within seconds
        if B > 1:
            B -= 1
        else:
            H = max(1, H // 4)
    dv = int(rng.choice([1, 2, 7, 16, 24, 64, 130]))
    while B * H * T * dv > 12_000_000 and (B > 1 or H > 1):   # host copies stay small
        if B > 1:
            B -= 1
        else:
            H = max(1, H // 4)
    code_bytes = int(rng.choice([4, 8]))
    alphabet = int(rng.choice([2, 40, 1000, max(2, T // 2), 1 << 24]
                              + ([1 << 40, 1 << 63] if code_bytes == 8 else [])))
    return {"seed": seed, "B": B, "H": H, "T": T, "code_bytes": code_bytes, "alphabet": alphabet,
            "structure": str(rng.choice(["uniform", "zipf", "runs"])),
            "dv": dv,
            "dtype": str(rng.choice(["f32", "bf16", "f16"])),
            "layout": str(rng.choice(["contiguous", "projection"])),
            "src_dtype": (torch.int32, torch.int64)[int(rng.integers(0, 2))]}


def draw_codes(rng, case, shape) -> np.ndarray:
    a = case["alphabet"]
    if case["structure"] == "zipf":
        c = rng.zipf(1.2, size=shape) - 1
        if a <= (1 << 62):                # larger alphabets hold every drawn value
            c %= a
    elif case["structure"] == "runs":   # long runs of one code: many hits at distance 1
        c = np.repeat(rng.integers(0, a, size=shape[:-1] + (shape[-1] // 16 + 1,)), 16,
                      axis=-1)[..., :shape[-1]]
    else:
        c = rng.integers(0, a, size=shape, dtype=np.uint64 if a > (1 << 62) else np.int64)
    c = c.astype(np.uint64)
    if case["code_bytes"] == 4:
        return c.astype(np.uint32).view(np.int32)
    return c.view(np.int64)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(96))
def test_prefill_sweep(dev, seed):
    case = draw_case(1000 + seed)
    print("case", case, flush=True)
    rng = np.random.default_rng(case["seed"])
    B, H, T, dv = case["B"], case["H"], case["T"], case["dv"]
    qc = draw_codes(rng, case, (B, H, T))
    kc = draw_codes(rng, case, (B, H, T))
    if rng.random() < 0.5:              # queries drawn from the keys: more hits
        kc = np.where(rng.random((B, H, T)) < 0.5, qc, kc)
    v32 = rng.standard_normal((B, H, T, dv)).astype(np.float32)
    v32[:, :, 0, 0] = -0.0
    dt = case["dtype"]
    tdt = TORCH[dt]
    if case["layout"] == "projection":
        base = torch.from_numpy(np.ascontiguousarray(v32.transpose(0, 2, 1, 3))).to(tdt)
        v = base.reshape(B, T, H * dv).to(dev).view(B, T, H, dv).transpose(1, 2)
    else:
        v = torch.from_numpy(v32).to(tdt).to(dev)
    q, k = torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev)

    want_src = oracle.latest_prev_match(qc.reshape(B * H, T), kc.reshape(B * H, T))
    src = latest_prev_match(q.view(B * H, T), k.view(B * H, T), out_dtype=case["src_dtype"])
    assert np.array_equal(src.cpu().numpy().astype(np.int64), want_src)

    vc = v.contiguous().cpu()
    carrier = (vc.numpy() if dt == "f32" else
               vc.view(torch.int16).numpy().view(np.uint16)).reshape(B * H, T, dv)
    y, src32 = lema_from_codes(q, k, v, return_src=True)
    assert np.array_equal(src32.cpu().numpy().reshape(B * H, T), want_src)
    got = y.contiguous().cpu()
    got = (got.numpy() if dt == "f32" else got.view(torch.int16).numpy().view(np.uint16))
    want = oracle.gather(carrier, dt, want_src, 0)
    assert _same(got.reshape(want.shape), want, dt)

    yz = gather_values(v, src.view(B, H, T), miss="zero").contiguous().cpu()
    yz = (yz.numpy() if dt == "f32" else yz.view(torch.int16).numpy().view(np.uint16))
    want = oracle.gather(carrier, dt, want_src, 1)
    assert _same(yz.reshape(want.shape), want, dt)


def _same(got: np.ndarray, want: np.ndarray, dtype: str) -> bool:
    """Bitwise equality (the sweep's values hold no NaN; -0 is compared by its bits)."""
    return bool(np.array_equal(got.view(NP_CARRIER[dtype]), want.view(NP_CARRIER[dtype])))


def test_sweep_covers_the_paths():
    """The drawn cases reach long rows (chunk summaries), rows of one chunk, both code widths,
    every dtype and layout, lengths that end inside a chunk, and launches of more items than
    the GPU holds workgroups."""
    cases = [draw_case(1000 + s) for s in range(96)]
    assert any(c["T"] >= 64 * 1024 for c in cases)
    assert any(c["T"] <= 1024 for c in cases)
    assert any(c["T"] % 1024 not in (0,) and c["T"] > 1024 for c in cases)
    assert {c["code_bytes"] for c in cases} == {4, 8}
    assert {c["dtype"] for c in cases} == {"f32", "bf16", "f16"}
    assert {c["layout"] for c in cases} == {"contiguous", "projection"}
    assert any(c["layout"] == "projection" and c["H"] == 64 for c in cases)
    # more (row, chunk) items than the GPU holds workgroups: the persistent kernel
    assert sum(c["B"] * c["H"] * -(-c["T"] // 1024) > 1024 for c in cases) >= 2


# ------------------------------------------------------------------------------ the store
STORE_CALL_T = [1, 1, 2, 100, 1024, 1025, 1500, 2049, 3000, 5000]


def draw_store_case(seed: int) -> dict:
    """Partitions, a sequence of exchanges (group range, positions per partition, insert-only or
    not), code width and alphabet, value row width and the table's load after the last call."""
    rng = np.random.default_rng(seed)
    P = int(rng.choice([1, 5, 64, 200]))
    calls, items = [], 0
    if P == 200 and rng.random() < 0.5:   # a long call over many partitions: the bulk path
        calls.append((0, P, 3000, False))
        items += P * 3000
    while len(calls) < 6 and items < 100_000:
        T = int(rng.choice(STORE_CALL_T))
        g0 = int(rng.integers(0, P))
        Pc = int(rng.integers(1, P - g0 + 1))
        if Pc * T > 650_000:               # the dict oracle stays within about a second
            Pc = max(1, 650_000 // T)
        calls.append((g0, Pc, T, bool(rng.random() < 0.2)))
        items += Pc * T
    code_bytes = int(rng.choice([4, 8]))
    alphabet = int(rng.choice([3, 50, 1000, 1 << 20] + ([1 << 62] if code_bytes == 8 else
                                                       [1 << 31])))
    return {"seed": seed, "P": P, "calls": calls, "code_bytes": code_bytes, "alphabet": alphabet,
            "d_v": int(rng.choice([4, 8, 12, 24, 64])), "load": float(rng.choice([0.3, 0.7, 0.85]))}


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(32))
def test_store_sweep(dev, seed):
    """Every exchange's output, the counts per partition and the final table content against
    one dict per partition with latest-write-wins (code/tests/test_store.py:17-41), codes 0 and
    all-ones included, 32-bit codes compared as their 32-bit patterns."""
    from latest_exact_match_attention_amd.cache import HashStore
    case = draw_store_case(5000 + seed)
    print("case", case, flush=True)
    rng = np.random.default_rng(case["seed"])
    P, d_v, cb = case["P"], case["d_v"], case["code_bytes"]
    mask = (1 << 32) - 1 if cb == 4 else (1 << 64) - 1
    data = []
    for g0, Pc, T, insert_only in case["calls"]:
        n = Pc * T
        qc = rng.integers(0, case["alphabet"], size=n, dtype=np.int64).astype(np.uint64)
        kc = rng.integers(0, case["alphabet"], size=n, dtype=np.int64).astype(np.uint64)
        for c in (qc, kc):                # the two codes a table could mistake for markers
            c[rng.random(n) < 0.01] = 0
            c[rng.random(n) < 0.01] = mask
        vals = rng.integers(0, 1 << 16, size=(n, d_v), dtype=np.uint16)
        data.append((qc, kc, vals))
    keys = set()
    for (g0, Pc, T, _), (_, kc, _) in zip(case["calls"], data):
        keys.update(zip((g0 + np.arange(kc.size) // T).tolist(), kc.tolist()))
    cap = max(64, int(len(keys) / case["load"]) + 1)
    store = HashStore(d_v, groups=P, dtype=np.uint16, capacity=cap, device=dev)
    ref = oracle.DictStore(P, 2 * d_v)
    for (g0, Pc, T, insert_only), (qc, kc, vals) in zip(case["calls"], data):
        to_dev = (lambda c: torch.from_numpy(c.astype(np.uint32).view(np.int32)).to(dev)) \
            if cb == 4 else (lambda c: torch.from_numpy(c.view(np.int64)).to(dev))
        out = None if insert_only else torch.empty((qc.size, d_v), dtype=torch.int16, device=dev)
        store.exchange(None if insert_only else to_dev(qc), to_dev(kc),
                       torch.from_numpy(vals.view(np.int16)).to(dev), out, T, g0)
        want = ref.exchange(qc, kc, vals.view(np.uint8).reshape(-1, 2 * d_v), T, g0)
        if not insert_only:
            got = out.cpu().numpy().view(np.uint8).reshape(-1, 2 * d_v)
            assert np.array_equal(got, want), (g0, Pc, T)
    assert np.array_equal(store.counts.numpy(), ref.counts())
    grp, code, val = store.dump()
    got = {(int(a), int(b) & mask): bytes(c) for a, b, c in
           zip(grp.cpu().numpy(), code.cpu().numpy(), val.cpu().numpy())}
    want = {(p, k): bytes(v) for p, d in enumerate(ref.ref) for k, v in d.items()}
    assert got == want


def test_store_sweep_covers_the_paths():
    """The drawn store cases reach decode-sized calls, the chunked path and the bulk path (long
    calls over few and over many partitions), insert-only calls, both code widths and loads of
    0.85."""
    cases = [draw_store_case(5000 + s) for s in range(32)]
    calls = [c for case in cases for c in case["calls"]]
    assert any(T == 1 for _, _, T, _ in calls)
    assert any(1 < T <= 1024 for _, _, T, _ in calls)
    assert any(T > 1024 and Pc <= 128 for _, Pc, T, _ in calls)
    assert any(T > 2048 and Pc > 128 for _, Pc, T, _ in calls)
    assert any(io for _, _, _, io in calls)
    assert {c["code_bytes"] for c in cases} == {4, 8}
    assert any(c["load"] == 0.85 for c in cases)


# ----------------------------------------------------------------------------- sign-pack
def draw_pack_case(seed: int) -> dict:
    """Heads, positions, width, dtype, layout (contiguous [B, H, T, D], or the projection
    [B, T, H * D] viewed as [B, H, T, D]) and code width; some cases reach 2^21 rows, where
    the 64-head projection view takes the tiled kernel's larger tiles."""
    rng = np.random.default_rng(seed)
    H = int(rng.choice([1, 5, 64]))
    D = int(rng.choice([1, 7, 8, 16, 24, 31, 32, 40, 64]))
    big = H == 64 and rng.random() < 0.4
    T = int(rng.integers(32769, 34000)) if big else int(rng.choice([1, 63, 64, 65, 1000, 4097]))
    B = 1 if big else int(rng.choice([1, 2, 3]))
    return {"seed": seed, "B": B, "H": H, "T": T, "D": D,
            "dtype": "bf16" if big else str(rng.choice(["f32", "bf16", "f16"])),
            "layout": "projection" if big or (H == 64 and rng.random() < 0.7) else
                      str(rng.choice(["contiguous", "projection"])),
            "code_dtype": torch.int32 if D <= 32 and rng.random() < 0.5 else torch.int64}


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(32))
def test_pack_sweep(dev, seed):
    """Codes equal the oracle's (code/lema/attention.py:82-97), with -0, NaN and the infinities
    among the values."""
    from latest_exact_match_attention_amd import pack_codes
    case = draw_pack_case(9000 + seed)
    print("case", case, flush=True)
    B, H, T, D = case["B"], case["H"], case["T"], case["D"]
    gen = torch.Generator(device="cpu").manual_seed(case["seed"])
    tdt = TORCH[case["dtype"]]
    if case["layout"] == "projection":
        base = torch.randn(B, T, H * D, generator=gen).to(tdt)
        view = lambda t: t.view(B, T, H, D).transpose(1, 2)
    else:
        base = torch.randn(B, H, T, D, generator=gen).to(tdt)
        view = lambda t: t
    flat = base.view(-1)
    n = min(flat.numel(), 5)
    flat[:n] = torch.tensor([0.0, -0.0, float("nan"), float("inf"), -float("inf")])[:n].to(tdt)
    zc = view(base).contiguous()
    carrier = zc.numpy() if case["dtype"] == "f32" else zc.view(torch.int16).numpy().view(np.uint16)
    want = oracle.pack_codes(carrier, case["dtype"])
    got = pack_codes(view(base.to(dev)), case["code_dtype"]).cpu().numpy()
    got = got.view(np.uint32).astype(np.uint64) if case["code_dtype"] == torch.int32 else \
        got.view(np.uint64)
    assert np.array_equal(got, want)


def test_pack_sweep_covers_the_paths():
    """Both tile sizes of the 64-head projection view, the dense and the generic layouts, all
    three dtypes and both code widths."""
    cases = [draw_pack_case(9000 + s) for s in range(32)]
    proj64 = [c for c in cases if c["layout"] == "projection" and c["H"] == 64]
    assert any(c["B"] * c["H"] * c["T"] >= 1 << 21 for c in proj64)
    assert any(c["B"] * c["H"] * c["T"] < 1 << 21 for c in proj64)
    assert any(c["layout"] == "contiguous" for c in cases)
    assert {c["dtype"] for c in cases} == {"f32", "bf16", "f16"}
    assert {c["code_dtype"] for c in cases} == {torch.int32, torch.int64}


# --------------------------------------------------------------------------------- model
def draw_model_case(seed: int) -> dict:
    """A small LEMA model: vocabulary, depth, width, heads, code width (up to 64 bits), value
    width, dtype and a token batch."""
    rng = np.random.default_rng(seed)
    heads = int(rng.choice([1, 2, 4, 8]))
    return {"seed": seed,
            "geo": dict(vocab_size=int(rng.choice([64, 200, 512])), depth=int(rng.integers(1, 4)),
                        dim=int(rng.choice([64, 128, 256])), num_heads=heads,
                        d_qk=int(rng.choice([4, 16, 24, 32, 40, 64])),
                        d_v=int(rng.choice([8, 16, 24, 48]))),
            "dtype": str(rng.choice(["f32", "bf16"])),
            "B": int(rng.integers(1, 3)), "T": int(rng.choice([64, 300, 1025, 2049]))}


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(16))
def test_model_sweep(dev, seed):
    """The model's loss against the functional oracle model on the same weights and tokens
    (code/lema/model.py:143-363; within 1e-2 relative in bf16, 1e-4 in fp32), and every layer's
    exact op, on that layer's own input, bit-exact against the reference's sort-based algorithm
    (code/lema/attention.py:100-132)."""
    from oracle import torch_model
    from oracle.torch_port import latest_prev_match_sorted
    from latest_exact_match_attention_amd import lema_from_codes, pack_codes
    from latest_exact_match_attention_amd.model import ModelConfig, Transformer, lm_loss
    case = draw_model_case(7000 + seed)
    print("case", case, flush=True)
    cfg = ModelConfig(**case["geo"])
    torch.manual_seed(case["seed"])
    with torch.device(dev):
        m = Transformer(cfg)
    m = m.to(TORCH[case["dtype"]]).eval().requires_grad_(False)
    m.set_hard(True)
    g = torch.Generator().manual_seed(case["seed"])
    tok = torch.randint(0, case["geo"]["vocab_size"], (case["B"], case["T"] + 1), generator=g).to(dev)
    x, y = tok[:, :-1], tok[:, 1:]
    B, T = x.shape
    with torch.no_grad():
        ours = lm_loss(m, x, y, chunk=256).item()
        want = torch_model.loss(m.state_dict(), cfg, x, y, chunk=256).item()
        tol = 1e-2 if case["dtype"] == "bf16" else 1e-4
        assert abs(ours - want) <= tol * abs(want), (ours, want)
        h = m.tok_emb(x)
        for i, blk in enumerate(m.blocks):
            zq, zk, v = blk.attn.project(blk.pre_attn(h))
            qc, kc = pack_codes(zq), pack_codes(zk)
            _, src = lema_from_codes(qc, kc, v, return_src=True)
            ref = latest_prev_match_sorted(qc.reshape(-1, T), kc.reshape(-1, T))
            assert torch.equal(src.long().reshape(-1, T), ref), i
            h = blk(h)
