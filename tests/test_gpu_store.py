"""The HBM store against the reference's store semantics (code/tests/test_store.py pattern):
every exchange output and every per-partition count must equal a per-partition dict with
latest-write-wins, across chunked, decode-sized and one-shot calls; an overfull table raises
"full"; the golden replay was produced by the reference's own store.cpp.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from latest_exact_match_attention_amd import _lib, lema_from_codes
from latest_exact_match_attention_amd.cache import HashStore, LemaCache

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
D_V = 8                                   # uint16 rows: 16 bytes, as the reference test


def run_dict_case(dev, seed, P, T, chunk, n_codes, capacity, code_dtype=torch.int64,
                  place="hbm"):
    """code/tests/test_store.py:17-41 against the store (table in HBM or host RAM)."""
    rng = np.random.default_rng(seed)
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=capacity, device=dev,
                      place=place)
    ref = oracle.DictStore(P, 2 * D_V)
    codes = rng.integers(0, n_codes, size=(2, P, T), dtype=np.int64) * 7919 % (n_codes + 2)
    vals = rng.integers(0, 1 << 16, size=(P, T, D_V), dtype=np.uint16)
    for lo in range(0, T, chunk):
        hi = min(T, lo + chunk)
        qc = np.ascontiguousarray(codes[0, :, lo:hi]).reshape(-1)
        kc = np.ascontiguousarray(codes[1, :, lo:hi]).reshape(-1)
        v = np.ascontiguousarray(vals[:, lo:hi]).reshape(-1, D_V)
        out = torch.empty((qc.size, D_V), dtype=torch.int16, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev).to(code_dtype),
                       torch.from_numpy(kc).to(dev).to(code_dtype),
                       torch.from_numpy(v.view(np.int16)).to(dev), out, hi - lo, 0)
        want = ref.exchange(qc, kc, v.view(np.uint8).reshape(-1, 2 * D_V), hi - lo, 0)
        got = out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V)
        assert np.array_equal(got, want), (seed, lo)
    assert np.array_equal(store.counts.numpy(), ref.counts()), "entries per partition"
    return store, ref


def test_store_golden_replay(dev):
    """Outputs and counts the reference's store.cpp produced for the same exchanges."""
    g = np.load(GOLDEN / "store.npz")
    codes, vals, chunks, cap = g["codes"], g["vals"], g["chunks"], int(g["cap"])
    P, T, vb = vals.shape
    store = HashStore(vb // 2, groups=P, dtype=np.uint16, capacity=cap, device=dev)
    lo = 0
    for c in chunks:
        hi = lo + int(c)
        qc = torch.from_numpy(np.ascontiguousarray(codes[0, :, lo:hi]).reshape(-1)).to(dev)
        kc = torch.from_numpy(np.ascontiguousarray(codes[1, :, lo:hi]).reshape(-1)).to(dev)
        v = torch.from_numpy(np.ascontiguousarray(vals[:, lo:hi]).reshape(-1, vb)).to(dev)
        out = torch.empty_like(v)
        store.exchange(qc, kc, v, out, hi - lo, 0)
        assert np.array_equal(out.cpu().numpy().reshape(P, hi - lo, vb), g["out"][:, lo:hi])
        lo = hi
    assert np.array_equal(store.counts.numpy(), g["counts"])


def test_store_chunks_of_500(dev):
    store, ref = run_dict_case(dev, seed=0, P=200, T=2000, chunk=500, n_codes=400,
                               capacity=90_000)
    assert store.load() > 0.5
    # the table itself: its published entries are exactly the dict's final content
    grp, code, val = store.dump()
    got = {(int(a), int(b)): bytes(c) for a, b, c in
           zip(grp.cpu().numpy(), code.cpu().numpy(), val.cpu().numpy())}
    want = {(p, k): bytes(v) for p, d in enumerate(ref.ref) for k, v in d.items()}
    assert got == want


def test_store_decode_sized(dev):
    run_dict_case(dev, seed=1, P=64, T=300, chunk=1, n_codes=150, capacity=11_000)


def test_store_one_shot(dev):
    run_dict_case(dev, seed=2, P=400, T=1000, chunk=1000, n_codes=300, capacity=130_000)


def test_store_long_call_spans_subchunks(dev):
    """T = 2040 per call over 600 partitions: the chunked path, two sub-chunks (1024 and 1016
    positions) in order within one exchange."""
    assert _lib.lib().lema_store_workspace_bytes(600 * 2040, 2040, 4) == 0
    run_dict_case(dev, seed=5, P=600, T=2040, chunk=2040, n_codes=60, capacity=120_000,
                  code_dtype=torch.int32)


def test_store_short_long_call_few_partitions(dev):
    """T = 2500 over 30 partitions takes the bulk path (one sub-call of three chunks)."""
    assert _lib.lib().lema_store_workspace_bytes(30 * 2500, 2500, 4) > 0
    run_dict_case(dev, seed=5, P=30, T=2500, chunk=2500, n_codes=60, capacity=6000,
                  code_dtype=torch.int32)


@pytest.mark.parametrize("T,chunk,P", [(300, 1, 64), (2000, 500, 200), (3000, 3000, 16)])
def test_store_in_host_ram(dev, T, chunk, P):
    """The table in pinned host RAM (the reference's placement), worked on in place by the
    same kernels over the host link: decode-sized steps, chunked calls and a bulk call equal
    the dict, entries included, and the table is the host tensor the CPU reads."""
    store, ref = run_dict_case(dev, seed=T, P=P, T=T, chunk=chunk, n_codes=300,
                               capacity=200_000, place="ram")
    assert store.place == "ram" and not store.table.is_cuda
    grp, code, val = store.dump()
    got = {(int(a), int(b)): bytes(c) for a, b, c in zip(grp.numpy(), code.numpy(), val.numpy())}
    assert got == {(p, k): bytes(v) for p, d in enumerate(ref.ref) for k, v in d.items()}


def test_store_in_host_ram_overfull_raises(dev):
    with pytest.raises(RuntimeError, match="full"):
        run_dict_case(dev, seed=3, P=50, T=100, chunk=100, n_codes=100, capacity=1000,
                      place="ram")


def test_store_overfull_raises(dev):
    with pytest.raises(RuntimeError, match="full"):
        run_dict_case(dev, seed=3, P=50, T=100, chunk=100, n_codes=100, capacity=1000)


@pytest.mark.parametrize("place", ["hbm", "ram"])
def test_store_contended_decode(dev, place):
    """1024 partitions claiming slots of a small shared table every step (load ~0.9 at the
    end): concurrent claims from every XCD must never hand one slot to two keys, in device
    memory and in host RAM."""
    P, steps, cap = 1024, 60, 70_000
    rng = np.random.default_rng(9)
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=cap, device=dev, place=place)
    ref = oracle.DictStore(P, 2 * D_V)
    for s in range(steps):
        qc = rng.integers(0, 2**63, P, dtype=np.int64)
        qc[::3] = rng.integers(0, 50, P)[::3]           # some queries hit earlier keys
        kc = rng.integers(0, 50, P, dtype=np.int64) if s % 2 else rng.integers(0, 2**63, P)
        v = rng.integers(0, 1 << 16, size=(P, D_V), dtype=np.uint16)
        out = torch.empty((P, D_V), dtype=torch.int16, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev),
                       torch.from_numpy(v.view(np.int16)).to(dev), out, 1, 0)
        want = ref.exchange(qc, kc, v.view(np.uint8).reshape(-1, 2 * D_V), 1, 0)
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V), want), s
    assert np.array_equal(store.counts.numpy(), ref.counts())
    grp, _, _ = store.dump()
    assert grp.numel() == len(store)                   # every claimed slot published once


@pytest.mark.parametrize("T", [1, 700, 3000])
def test_store_mixed_widths_zero_extend(dev, T):
    """Keys inserted as int64 codes below 2^32 are found by int32 queries of the same 32-bit
    pattern (bit 31 set in half of them) and the other way round; the table holds the
    zero-extended code, as the reference's int64 code (decode-sized, chunked and bulk
    calls)."""
    rng = np.random.default_rng(T)
    P = 16
    pats = (np.arange(1, 200, dtype=np.int64) * 0x9E3779B1) & 0xFFFFFFFF
    assert (pats >= 1 << 31).sum() > 50
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=40_000, device=dev)
    ref = oracle.DictStore(P, 2 * D_V)
    for step in range(3):
        qc = rng.choice(pats, size=P * T)
        kc = rng.choice(pats, size=P * T)
        v = rng.integers(0, 1 << 16, size=(P * T, D_V), dtype=np.uint16)
        q32 = torch.from_numpy(qc.astype(np.uint32).view(np.int32)).to(dev)
        k64 = torch.from_numpy(kc).to(dev)
        if step == 1:              # the other pairing: int64 queries, int32 keys
            q32 = torch.from_numpy(qc).to(dev)
            k64 = torch.from_numpy(kc.astype(np.uint32).view(np.int32)).to(dev)
        out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
        store.exchange(q32, k64, torch.from_numpy(v.view(np.int16)).to(dev), out, T, 0)
        want = ref.exchange(qc, kc, v.view(np.uint8).reshape(-1, 2 * D_V), T, 0)
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V), want), step
    assert np.array_equal(store.counts.numpy(), ref.counts())
    grp, code, _ = store.dump()
    got = set(zip(grp.cpu().numpy().tolist(), code.cpu().numpy().tolist()))
    assert got == {(p, k) for p, d in enumerate(ref.ref) for k in d}


def test_store_table_is_reference_format(dev):
    """A table filled on the GPU is continued by the C restatement of store.cpp on the host
    (same slot format and home-slot hash): the results stay those of the dict."""
    rng = np.random.default_rng(4)
    P, T, vb, cap = 16, 64, 16, 2048
    store = HashStore(vb // 2, groups=P, dtype=np.uint16, capacity=cap, device=dev)
    ref = oracle.DictStore(P, vb)
    codes = rng.integers(0, 40, size=(4, P, T), dtype=np.int64)
    vals = rng.integers(0, 256, size=(2, P, T, vb), dtype=np.uint8)
    qc, kc = codes[0].reshape(-1), codes[1].reshape(-1)
    v = vals[0].reshape(-1, vb)
    out = torch.empty((P * T, vb), dtype=torch.uint8, device=dev)
    store.exchange(torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev),
                   torch.from_numpy(v).to(dev), out, T, 0)
    assert np.array_equal(out.cpu().numpy(), ref.exchange(qc, kc, v, T, 0))
    host = oracle.HostStore(vb, P, cap)
    host.table[:] = store.table.cpu().numpy()
    host.counts[:] = store.counts.numpy()
    qc2, kc2 = codes[2].reshape(-1), codes[3].reshape(-1)
    v2 = vals[1].reshape(-1, vb)
    out2 = np.empty_like(v2)
    host.exchange(qc2, kc2, v2, out2, T, 0)
    assert np.array_equal(out2, ref.exchange(qc2, kc2, v2, T, 0))
    assert np.array_equal(host.counts, ref.counts())


class _Cfg:
    depth, num_heads, d_v = 2, 4, 16


@pytest.mark.parametrize("step", [1, 7, 64, 300])
def test_cache_chunked_equals_dense(dev, step):
    """Fed through the store in any chunking, a layer retrieves what the dense op gathers
    (values of matched keys; the store's miss is +0) -- code/tests/test_gpu.py:68-90 at the
    op level."""
    B, H, T, dv = 2, _Cfg.num_heads, 300, _Cfg.d_v
    rng = np.random.default_rng(step)
    qc = torch.from_numpy(rng.integers(0, 30, (B, H, T))).to(dev)
    kc = torch.from_numpy(rng.integers(0, 30, (B, H, T))).to(dev)
    v = torch.randn(B, H, T, dv, device=dev, dtype=torch.bfloat16)
    dense, src = lema_from_codes(qc, kc, v, return_src=True)
    dense = torch.where((src >= 0).unsqueeze(-1), dense, torch.zeros_like(dense))
    cache = LemaCache(_Cfg, dtype=torch.bfloat16, max_cache_len=T, batch=B, device=dev)
    parts = [cache.layer(1).exchange(qc[:, :, s:s + step], kc[:, :, s:s + step],
                                     v[:, :, s:s + step]) for s in range(0, T, step)]
    got = torch.cat(parts, dim=2)
    assert torch.equal(got.view(torch.int16), dense.view(torch.int16))
    assert cache.entries() == int(cache.counts().sum()) > 0
    assert cache.counts()[0].sum() == 0                 # layer 0's partitions untouched


def test_decode_steps_in_a_graph_equal_eager(dev):
    """Decode steps captured into one HIP graph and replayed produce exactly what the eager
    steps produce (code/tests/test_gpu.py:117-141 at the store level); the graph is replayed
    once, between eager host work and a synchronisation."""
    P, steps, cap, dv = 256, 24, 40_000, 24
    gen = torch.Generator(device=dev).manual_seed(3)
    pre_k = torch.randint(0, 2**32, (P * 64,), dtype=torch.int64, device=dev, generator=gen)
    pre_v = torch.randn((P * 64, dv), device=dev, generator=gen).to(torch.bfloat16)
    qc = torch.randint(0, 2**32, (steps, P), dtype=torch.int64, device=dev, generator=gen)
    qc[:, ::4] = pre_k.view(P, 64)[::4, :steps].t()      # every 4th partition hits a prefill key
    kc = torch.randint(0, 2**32, (steps, P), dtype=torch.int64, device=dev, generator=gen)
    vv = torch.randn((steps, P, dv), device=dev, generator=gen).to(torch.bfloat16)
    stores = [HashStore(dv, groups=P, dtype=torch.bfloat16, capacity=cap, device=dev)
              for _ in range(2)]
    for st in stores:
        st.exchange(None, pre_k, pre_v, None, 64, 0)
    eager = torch.empty_like(vv)
    for s in range(steps):
        stores[0].exchange(qc[s], kc[s], vv[s], eager[s], 1, 0)
    graphed = torch.empty_like(vv)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for s in range(steps):
            stores[1].exchange(qc[s], kc[s], vv[s], graphed[s], 1, 0, check=False)
    assert int(stores[1].counts_device.sum()) == P * 64      # capture ran nothing
    torch.randn(1000, device=dev).sum().item()               # eager work in between
    g.replay()
    torch.cuda.synchronize()
    stores[1].check_full()
    assert torch.equal(graphed.view(torch.int16), eager.view(torch.int16))
    assert torch.equal(stores[1].counts, stores[0].counts)
    assert (eager[:, ::4] != 0).any(-1).float().mean() > 0.9


# ------------------------------------------------------------------ the bulk path
# Calls with T > 2048 run as sub-calls of up to 32768 positions with in-chunk
# resolution, per-chunk key summaries and a scratch table of the sub-call's (partition, code)
# pairs: the results must be the dict's in every case the chunked path covers.

def test_bulk_one_shot_and_continued(dev):
    """Two long calls in a row (5 chunks, the last partial): in-chunk, cross-chunk and
    cross-call matches all occur."""
    run_dict_case(dev, seed=11, P=5, T=9000, chunk=4500, n_codes=300, capacity=40_000,
                  code_dtype=torch.int32)


def test_bulk_crosses_a_sub_call(dev):
    """T = 70,000: sub-calls of 32,768, 32,768 and 4,464 positions, in order; codes repeat
    across the boundaries."""
    run_dict_case(dev, seed=12, P=2, T=70_000, chunk=70_000, n_codes=20_000,
                  capacity=100_000, code_dtype=torch.int32)


def test_bulk_hot_codes_in_every_chunk(dev):
    """Eight codes over 30 chunks: every code's chunk mask is nearly full and queries whose
    chunk lacks an earlier key take the latest chunk below theirs."""
    run_dict_case(dev, seed=13, P=3, T=30_000, chunk=30_000, n_codes=8, capacity=1_000,
                  code_dtype=torch.int32)


def test_bulk_sentinel_and_zero_codes(dev):
    """0xFFFFFFFF (int32 -1) is a code like any other, and so is 0."""
    rng = np.random.default_rng(14)
    P, T = 4, 6000
    qc = rng.integers(0, 5, size=P * T).astype(np.int64) - 1        # -1 .. 3
    kc = rng.integers(0, 5, size=P * T).astype(np.int64) - 1
    far = rng.random(P * T) < 0.5                                    # queries that miss
    qc[far] = rng.integers(10, 1 << 30, size=int(far.sum()))
    vals = rng.integers(0, 1 << 16, size=(P * T, D_V), dtype=np.uint16)
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=4096, device=dev)
    ref = oracle.DictStore(P, 2 * D_V)
    out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
    store.exchange(torch.from_numpy(qc).to(dev).to(torch.int32),
                   torch.from_numpy(kc).to(dev).to(torch.int32),
                   torch.from_numpy(vals.view(np.int16)).to(dev), out, T, 0)
    # the dict sees the 32-bit patterns the store sees
    want = ref.exchange(qc & 0xFFFFFFFF, kc & 0xFFFFFFFF, vals.view(np.uint8).reshape(-1, 2 * D_V),
                        T, 0)
    assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V), want)
    assert np.array_equal(store.counts.numpy(), ref.counts())
    assert set(store.dump()[1].cpu().numpy().tolist()) == {0xFFFFFFFF, 0, 1, 2, 3}


def test_bulk_region_at_design_load(dev):
    """Whole sub-calls of distinct key codes, so each partition's region of the scratch table
    holds 32,768 codes (half full, its design limit), and queries that copy the key 1 to
    40,000 positions back (in the chunk, in an earlier chunk, in the previous sub-call) or
    miss."""
    rng = np.random.default_rng(17)
    P, T = 2, 65_536
    # an odd multiplier is a bijection modulo 2^30: distinct codes below 2^30
    kc = (np.arange(P * T, dtype=np.int64) * 2_654_435_761) % (1 << 30)
    qc = rng.integers(0, 1 << 30, size=P * T, dtype=np.int64)
    pos = np.arange(P * T) % T
    back = pos - rng.integers(1, 40_001, size=P * T)
    copy = (rng.random(P * T) < 0.5) & (back >= 0)
    qc[copy] = kc[(np.arange(P * T) - pos + back)[copy]]
    vals = rng.integers(0, 1 << 16, size=(P * T, D_V), dtype=np.uint16)
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=400_000, device=dev)
    ref = oracle.DictStore(P, 2 * D_V)
    out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
    store.exchange(torch.from_numpy(qc).to(dev).to(torch.int32),
                   torch.from_numpy(kc).to(dev).to(torch.int32),
                   torch.from_numpy(vals.view(np.int16)).to(dev), out, T, 0)
    want = ref.exchange(qc, kc, vals.view(np.uint8).reshape(-1, 2 * D_V), T, 0)
    got = out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V)
    assert np.array_equal(got, want)
    assert (got != 0).any(-1).mean() > 0.3   # about 0.35 of the queries copy an earlier key
    assert np.array_equal(store.counts.numpy(), ref.counts())
    store.check_full()


def _splitmix_fin(x):
    """splitmix64's finaliser on uint64 arrays (the bulk path's group-table hash)."""
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def _bulk_group_cap(T, parts=8):
    s = min(T, 32 * 1024)
    cap = 256 * parts
    while cap < 2 * s:
        cap *= 2
    return cap


def test_bulk_spilled_part_32bit(dev):
    """32-bit key codes chosen so that one of a partition's eight group-table parts gets more
    codes than its LDS table takes (3/4 of its words): that part's queries and inserts search
    the chunk summaries instead, code 0 among them. Another partition uses the same part with
    few codes and a third ordinary codes; two calls, against the dict."""
    rng = np.random.default_rng(18)
    P, T = 3, 6000
    cand = rng.integers(1, 1 << 31, size=200_000, dtype=np.int64)
    q0 = cand[(_splitmix_fin(cand) >> np.uint64(61)) == 0]           # codes of part 0
    assert int(_splitmix_fin(0) >> np.uint64(61)) == 0               # code 0 is one of them
    pools = [np.concatenate([[0], q0[:5500]]), q0[5500:6000], cand[:3000]]
    limit = _bulk_group_cap(T) // 8 // 4 * 3
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=200_000, device=dev)
    ref = oracle.DictStore(P, 2 * D_V)
    for call in range(2):
        kc = np.concatenate([rng.choice(pool, size=T) for pool in pools])
        assert len(set(kc[:T].tolist())) > limit and len(set(kc[T:2 * T].tolist())) < limit
        qc = np.concatenate([rng.choice(pool, size=T) for pool in pools])
        miss = rng.random(P * T) < 0.2
        qc[miss] = rng.integers(1 << 30, 1 << 31, size=int(miss.sum()))
        vals = rng.integers(0, 1 << 16, size=(P * T, D_V), dtype=np.uint16)
        out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev).to(torch.int32),
                       torch.from_numpy(kc).to(dev).to(torch.int32),
                       torch.from_numpy(vals.view(np.int16)).to(dev), out, T, 0)
        want = ref.exchange(qc, kc, vals.view(np.uint8).reshape(-1, 2 * D_V), T, 0)
        got = out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V)
        assert np.array_equal(got, want), call
    assert np.array_equal(store.counts.numpy(), ref.counts())
    store.check_full()


@pytest.mark.parametrize("d_v", [4, 12, 20, 32, 40, 64, 144])
def test_bulk_long_value_rows(dev, d_v):
    """Rows of 8 to 288 bytes through two long calls. The wave copies the rows it names
    together, each row by a power-of-two group of lanes: 8-byte pieces for rows of 8, 24 and
    40 bytes (1, 3 and 5 pieces), 16-byte pieces for 64, 80 and 128 bytes, and 18 pieces over
    16 lanes (two each) for 288 bytes."""
    run_store_rows_case(dev, seed=100 + d_v, d_v=d_v, P=3, Ts=(5000, 2600))


def run_store_rows_case(dev, seed, d_v, P, Ts):
    rng = np.random.default_rng(seed)
    store = HashStore(d_v, groups=P, dtype=np.uint16, capacity=60_000, device=dev)
    ref = oracle.DictStore(P, 2 * d_v)
    for T in Ts:
        qc = rng.integers(0, 2000, P * T)
        kc = rng.integers(0, 2000, P * T)
        v = rng.integers(0, 256, size=(P * T, 2 * d_v), dtype=np.uint8)
        out = torch.empty((P * T, 2 * d_v), dtype=torch.uint8, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev).to(torch.int32),
                       torch.from_numpy(kc).to(dev).to(torch.int32),
                       torch.from_numpy(v).to(dev), out, T, 0)
        assert np.array_equal(out.cpu().numpy(), ref.exchange(qc, kc, v, T, 0)), T
    assert np.array_equal(store.counts.numpy(), ref.counts())


def exchange_chunked(st, qc, kc, values, out, T, g0):
    """The same exchange through lema_store_exchange, which takes no workspace and so runs
    every call in 1024-position sub-chunks (the bulk path is off)."""
    from latest_exact_match_attention_amd import _lib
    L = _lib.lib()
    cb = kc.element_size()
    _lib.check(L.lema_store_exchange(
        st.table.data_ptr(), st.cap, st.vbytes, qc.data_ptr() if qc is not None else None,
        kc.data_ptr(), cb, values.data_ptr(), out.data_ptr() if out is not None else None,
        kc.numel(), T, g0, st.counts_device.data_ptr(), st.full_flag.data_ptr(),
        _lib.stream_of(kc)))
    st.check_full()


def _three_paths(dev, qc, kc, v, P, T, cap):
    """Outputs, stores and counts of one exchange through the bulk path with int32 and int64
    codes and through the chunked path."""
    res = []
    for dt, bulk in ((torch.int32, True), (torch.int64, True), (torch.int64, False)):
        st = HashStore(D_V, groups=P, dtype=np.uint16, capacity=cap, device=dev)
        out = torch.empty_like(v)
        q, k = torch.from_numpy(qc).to(dev).to(dt), torch.from_numpy(kc).to(dev).to(dt)
        if bulk:
            st.exchange(q, k, v, out, T, 0)
        else:
            exchange_chunked(st, q, k, v, out, T, 0)
        res.append((out, st))
    return res


def test_bulk_equals_chunked_path_and_insert_only(dev):
    """The same long exchange through the bulk path (int32 and int64 codes of the same values)
    and the chunked path leaves the same entries and returns the same values; an insert-only
    long call then serves later queries."""
    rng = np.random.default_rng(15)
    P, T, cap = 6, 8192, 60_000
    qc = rng.integers(0, 3000, size=P * T)
    kc = rng.integers(0, 3000, size=P * T)
    v = torch.from_numpy(rng.integers(-30000, 30000, size=(P * T, D_V), dtype=np.int16)).to(dev)
    dumps, outs = [], []
    for out, st in _three_paths(dev, qc, kc, v, P, T, cap):
        g, c, val = st.dump()
        dumps.append({(int(a), int(b)): bytes(x) for a, b, x in
                      zip(g.cpu().numpy(), c.cpu().numpy(), val.cpu().numpy())})
        outs.append(out)
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    assert all(dumps[0] == d for d in dumps[1:])
    for dt in (torch.int32, torch.int64):
        st = HashStore(D_V, groups=P, dtype=np.uint16, capacity=cap, device=dev)
        st.exchange(None, torch.from_numpy(kc).to(dev).to(dt), v, None, T, 0)
        q = torch.from_numpy(kc.reshape(P, T)[:, ::2].copy()).to(dev).to(dt).reshape(-1)
        got = torch.empty((q.numel(), D_V), dtype=torch.int16, device=dev)
        st.exchange(q, torch.full_like(q, -7), torch.zeros_like(got), got, T // 2, 0)
        ref = oracle.DictStore(P, 2 * D_V)
        vv = v.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V)
        ref.exchange(np.full(P * T, -123), kc, vv, T, 0)
        k7 = (1 << 32) - 7 if dt == torch.int32 else -7
        want = ref.exchange(q.cpu().numpy().astype(np.int64), np.full(q.numel(), k7),
                            np.zeros((q.numel(), 2 * D_V), np.uint8), T // 2, 0)
        assert np.array_equal(got.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V), want), dt


def test_bulk_many_partitions_equals_chunked_path(dev):
    """2,100 partitions x T = 4,200 (2,100 group tables, each partition's claims tallied from
    its workgroups): the bulk path (int32 and int64 codes) and the chunked path agree on
    outputs, entries and per-partition counts."""
    rng = np.random.default_rng(16)
    P, T, cap = 2100, 4200, 9_000_000
    assert _lib.lib().lema_store_workspace_bytes(P * T, T, 8) > 0
    qc = rng.integers(0, 700, size=P * T)
    kc = rng.integers(0, 700, size=P * T)
    v = torch.from_numpy(rng.integers(-30000, 30000, size=(P * T, D_V), dtype=np.int16)).to(dev)
    outs, dumps, counts = [], [], []
    for out, st in _three_paths(dev, qc, kc, v, P, T, cap):
        g, c, val = st.dump()
        key = g * 1024 + c                                   # codes < 700, groups < 2100
        order = torch.argsort(key)
        dumps.append((key[order], val[order]))
        outs.append(out)
        counts.append(st.counts)
    for i in (1, 2):
        assert torch.equal(outs[0], outs[i])
        assert torch.equal(dumps[0][0], dumps[i][0]) and torch.equal(dumps[0][1], dumps[i][1])
        assert torch.equal(counts[0], counts[i])
    assert int(counts[0].sum()) == dumps[0][0].numel()


@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_bulk_group_offsets(dev, code_dtype):
    """Long calls at non-zero group offsets (a layer's partitions start at layer x B x H):
    groups [5, 8) then [0, 5) then [2, 10) of one 10-group store, overlapping, against the dict;
    entries of different groups with equal codes stay apart, and counts land on the right
    groups."""
    rng = np.random.default_rng(21)
    store = HashStore(D_V, groups=10, dtype=np.uint16, capacity=200_000, device=dev)
    ref = oracle.DictStore(10, 2 * D_V)
    for g0, P, T in ((5, 3, 5000), (0, 5, 3000), (2, 8, 2600)):
        qc = rng.integers(0, 4000, size=P * T)
        kc = rng.integers(0, 4000, size=P * T)
        vals = rng.integers(0, 1 << 16, size=(P * T, D_V), dtype=np.uint16)
        out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev).to(code_dtype),
                       torch.from_numpy(kc).to(dev).to(code_dtype),
                       torch.from_numpy(vals.view(np.int16)).to(dev), out, T, g0)
        want = ref.exchange(qc, kc, vals.view(np.uint8).reshape(-1, 2 * D_V), T, g0)
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V), want), g0
    assert np.array_equal(store.counts.numpy(), ref.counts())


def test_bulk_64bit_codes_all_ones_and_zero(dev):
    """64-bit codes through the bulk path: the all-ones code (int64 -1, the group table's
    free marker, kept apart there) and 0 are codes like any other, beside codes with high
    bits set, against the dict over two long calls."""
    rng = np.random.default_rng(19)
    P, T = 4, 6000
    pool = np.array([-1, 0, 1, -2, (1 << 62) + 5, -(1 << 40), 123456789012345], dtype=np.int64)
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=20_000, device=dev)
    ref = oracle.DictStore(P, 2 * D_V)
    for call in range(2):
        qc = rng.choice(pool, size=P * T)
        kc = rng.choice(pool, size=P * T)
        far = rng.random(P * T) < 0.3
        qc[far] = rng.integers(1 << 40, 1 << 62, size=int(far.sum()))
        vals = rng.integers(0, 1 << 16, size=(P * T, D_V), dtype=np.uint16)
        out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev),
                       torch.from_numpy(vals.view(np.int16)).to(dev), out, T, 0)
        want = ref.exchange(qc, kc, vals.view(np.uint8).reshape(-1, 2 * D_V), T, 0)
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V), want), call
    assert np.array_equal(store.counts.numpy(), ref.counts())
    assert set(store.dump()[1].cpu().numpy().astype(np.int64).tolist()) == set(pool.tolist())


def test_bulk_64bit_spilled_part(dev):
    """64-bit key codes chosen so that one of a partition's eight group-table parts gets more
    codes than its LDS table takes: that part's queries and inserts search the chunk
    summaries. One spilled partition holds code 0 in that part, another the all-ones code;
    beside them an unspilled part and ordinary codes, two calls against the dict."""
    rng = np.random.default_rng(20)
    P, T = 4, 6000
    cand = rng.integers(-(1 << 62), 1 << 62, size=400_000, dtype=np.int64) * 2 + 1
    part_of = lambda c: _splitmix_fin(np.asarray(c, dtype=np.int64).view(np.uint64)) >> np.uint64(61)
    part = part_of(cand)
    z, s = int(part_of(0)), int(part_of(-1))        # the parts of code 0 and the all-ones code
    pz, ps = cand[part == z], cand[part == s]
    pools = [np.concatenate([[0], pz[:5000]]),     # fills code 0's part
             np.concatenate([[-1], ps[:5000]]),    # fills the all-ones code's part
             pz[5000:5300],                        # the same part as the first, few codes
             cand[:3000]]                          # ordinary codes
    limit = _bulk_group_cap(T) // 8 // 4 * 3
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=300_000, device=dev)
    ref = oracle.DictStore(P, 2 * D_V)
    for call in range(2):
        kc = np.concatenate([rng.choice(pool, size=T) for pool in pools])
        assert len(set(kc[:T].tolist())) > limit and len(set(kc[T:2 * T].tolist())) > limit
        assert len(set(kc[2 * T:3 * T].tolist())) < limit
        kc[[0, T + 1]] = [0, -1]                   # both special codes are keys
        qc = np.concatenate([rng.choice(pool, size=T) for pool in pools])
        miss = rng.random(P * T) < 0.2
        qc[miss] = rng.integers(1 << 40, 1 << 62, size=int(miss.sum())) * 2
        vals = rng.integers(0, 1 << 16, size=(P * T, D_V), dtype=np.uint16)
        out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev), torch.from_numpy(kc).to(dev),
                       torch.from_numpy(vals.view(np.int16)).to(dev), out, T, 0)
        want = ref.exchange(qc, kc, vals.view(np.uint8).reshape(-1, 2 * D_V), T, 0)
        assert np.array_equal(out.cpu().numpy().view(np.uint8).reshape(-1, 2 * D_V), want), call
    assert np.array_equal(store.counts.numpy(), ref.counts())
    store.check_full()


@pytest.mark.parametrize("d_v,dtype", [(4, np.float16), (12, np.float16), (2, np.float32)])
def test_store_value_rows_of_8_byte_pieces(dev, d_v, dtype):
    """Rows of 8, 24 and 8 bytes (not multiples of 16) take the 8-byte piece copies: decode
    steps, a chunked call and a long (bulk) call against the dict."""
    rng = np.random.default_rng(d_v)
    P = 6
    vb = d_v * np.dtype(dtype).itemsize
    store = HashStore(d_v, groups=P, dtype=dtype, capacity=30_000, device=dev)
    ref = oracle.DictStore(P, vb)
    for T in (1, 1, 700, 3000, 1):
        qc = rng.integers(0, 300, P * T)
        kc = rng.integers(0, 300, P * T)
        v = rng.integers(0, 256, size=(P * T, vb), dtype=np.uint8)
        out = torch.empty((P * T, vb), dtype=torch.uint8, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev).to(torch.int32),
                       torch.from_numpy(kc).to(dev).to(torch.int32),
                       torch.from_numpy(v).to(dev), out, T, 0)
        assert np.array_equal(out.cpu().numpy(), ref.exchange(qc, kc, v, T, 0)), T
    assert np.array_equal(store.counts.numpy(), ref.counts())


def _host_entries(table: torch.Tensor, vbytes: int) -> dict:
    """(group, code) -> value bytes of a table in the reference's slot format."""
    words = table[:, :16].contiguous().view(torch.int64)
    live = words[:, 1] >= 2
    g, c = (words[live, 1] - 2).tolist(), words[live, 0].tolist()
    vals = table[live, 16:16 + vbytes].numpy()
    return {(a, b): bytes(v) for a, b, v in zip(g, c, vals)}


@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_bulk_1024_partitions_against_reference_store(dev, code_dtype):
    """1,024 partitions x T = 4,096 (the bulk path at the partition count of a 16-stream,
    64-head prefill), first on a fresh table where every new key claims a slot, then a second
    call that mostly overwrites: outputs, entries and per-partition counts equal the
    reference's own store.cpp (oracle/_ref) fed the same calls on a host table."""
    ref = oracle.ref_store()
    assert ref is not None, "oracle/_ref/lema_store_ref.so is not built"
    P, T, cap = 1024, 4096, 6_000_000
    cb = 4 if code_dtype == torch.int32 else 8
    assert _lib.lib().lema_store_workspace_bytes(P * T, T, cb) > 0
    rng = np.random.default_rng(1024)
    store = HashStore(D_V, groups=P, dtype=np.uint16, capacity=cap, device=dev)
    host = torch.zeros((cap, 16 + 2 * D_V), dtype=torch.uint8)
    host_counts = torch.zeros(P, dtype=torch.int64)
    for call in range(2):
        qc = rng.integers(0, 3000, P * T)
        kc = rng.integers(0, 3000, P * T)
        v = rng.integers(-30000, 30000, size=(P * T, D_V), dtype=np.int16)
        out = torch.empty((P * T, D_V), dtype=torch.int16, device=dev)
        store.exchange(torch.from_numpy(qc).to(dev).to(code_dtype),
                       torch.from_numpy(kc).to(dev).to(code_dtype), torch.from_numpy(v).to(dev),
                       out, T, 0)
        oh = torch.empty((P * T, D_V), dtype=torch.int16)
        host_counts += ref.exchange(host, torch.from_numpy(qc), torch.from_numpy(kc),
                                    torch.from_numpy(v), oh, T, 0, cap, 2 * D_V)
        assert torch.equal(out.cpu(), oh), call
        assert torch.equal(store.counts, host_counts), call
    g, c, val = store.dump()
    got = {(a, b): bytes(x) for a, b, x in
           zip(g.cpu().tolist(), c.cpu().tolist(), val.cpu().numpy())}
    assert got == _host_entries(host, 2 * D_V)
    assert len(got) > 2_000_000
