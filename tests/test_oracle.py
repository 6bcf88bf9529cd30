"""Pin the CPU oracle (CPU only). Each oracle function is checked against something that does
not share its code: the reference's own store compiled from code/lema/csrc/store.cpp, the
dictionary rule of verification/lema.py:19-33, an O(T^2) brute force, IEEE facts, and cases
whose answer is known in closed form. A plausible slip (non-strict causality, earliest
instead of latest, a dropped sign bit, a wrong bit order, lookup after insert) fails at
least one of them.
"""
import numpy as np
import pytest

import oracle

U64 = np.uint64


# ------------------------------------------------------------------------ pack codes
def _f32_bits_of(bits16: np.ndarray) -> np.ndarray:
    return (bits16.astype(np.uint32) << 16).view(np.float32)


def test_pack_every_bf16_pattern():
    """Exhaustive over all 65536 bf16 bit patterns at D = 1: the bit is the IEEE
    comparison of the widened value with zero (-0 -> 1, NaN -> 0)."""
    z = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).reshape(-1, 1)
    got = oracle.pack_codes(z, "bf16")
    want = (_f32_bits_of(z[:, 0]) >= 0).astype(U64)
    assert np.array_equal(got, want)
    assert got[0x8000] == 1 and got[0x7FC0] == 0 and got[0xFF80] == 0 and got[0x7F80] == 1


def test_pack_every_f16_pattern():
    z = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).reshape(-1, 1)
    got = oracle.pack_codes(z, "f16")
    want = (z[:, 0].view(np.float16) >= 0).astype(U64)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("D", [1, 7, 24, 32, 33, 63, 64])
def test_pack_bit_order(D):
    """Bit j of the code is dim j (LSB = dim 0): decode every bit back."""
    rng = np.random.default_rng(D)
    z = rng.standard_normal((500, D)).astype(np.float32)
    codes = oracle.pack_codes(z, "f32")
    for j in range(D):
        assert np.array_equal((codes >> U64(j)) & U64(1), (z[:, j] >= 0).astype(U64))
    if D < 64:
        assert (codes >> U64(D) == 0).all()


def test_pack_closed_forms():
    D = 64
    z = np.full((3, D), -1.0, dtype=np.float32)
    z[1] = 0.0
    z[2] = -1.0
    z[2, 63] = 2.0
    codes = oracle.pack_codes(z, "f32")
    assert codes[0] == 0
    assert codes[1] == U64(2**64 - 1)                  # all zeros pack to all ones
    assert codes[2] == U64(1 << 63)                    # the int64 sign bit at D = 64
    assert codes.view(np.int64)[2] < 0
    with pytest.raises(ValueError):
        oracle.pack_codes(np.zeros((1, 65), np.float32), "f32")


# ----------------------------------------------------------------- latest prev match
def test_latest_match_dict_rule_and_brute_force():
    rng = np.random.default_rng(0)
    for trial in range(60):
        T = int(rng.integers(1, 200))
        alpha = int(rng.choice([1, 2, 3, 5, 17, 1000]))
        qc = rng.integers(0, alpha, (2, T))
        kc = rng.integers(0, alpha, (2, T))
        src = oracle.latest_prev_match(qc, kc)
        for n in range(2):
            assert list(src[n]) == oracle.dict_rule(qc[n], kc[n])
            assert np.array_equal(src[n], oracle.brute_force(qc[n], kc[n]))


def test_latest_match_closed_forms():
    T = 257
    i = np.arange(T)
    cases = [
        (np.full(T, 9), np.full(T, 9), i - 1),                   # latest, not earliest
        (i, i, np.full(T, -1)),                                   # strictly causal
        (i, i + T, np.full(T, -1)),                               # nothing in common
        # query i asks for code i + 1, which key i + 1 writes only later: no match
        (i + 1, i, np.full(T, -1)),
    ]
    for qc, kc, want in cases:
        got = oracle.latest_prev_match(qc[None], kc[None])[0]
        assert np.array_equal(got, want)
    # shifted copy: query i asks for the key written at i - 3
    got = oracle.latest_prev_match((i - 3)[None], i[None])[0]
    assert np.array_equal(got, np.where(i >= 3, i - 3, -1))
    # T = 1 never matches
    assert oracle.latest_prev_match(np.array([[4]]), np.array([[4]]))[0, 0] == -1


def test_latest_match_64bit_codes():
    """Codes differing only in the top bit, or equal to the all-ones pattern, stay
    distinct/equal as 64-bit patterns."""
    top = np.int64(np.iinfo(np.int64).min)
    qc = np.array([[0, top, -1, 0, top, -1]], dtype=np.int64)
    kc = np.array([[top, 0, -1, -1, 5, 0]], dtype=np.int64)
    got = oracle.latest_prev_match(qc, kc)[0]
    assert list(got) == oracle.dict_rule(qc[0], kc[0])
    assert list(got) == [-1, 0, -1, 1, 0, 3]


def test_latest_match_invariants_plumbing_size():
    """dense_plumbing size (B1 H8 T4096, 16-bit codes): every index obeys the definition."""
    from latest_exact_match_attention_amd.workloads import dense_plumbing
    qc, kc, _ = dense_plumbing(0)
    qc, kc = qc.reshape(8, -1), kc.reshape(8, -1)
    src = oracle.latest_prev_match(qc, kc)
    T = qc.shape[1]
    for n in range(8):
        s = src[n]
        hit = s >= 0
        assert (s < np.arange(T)).all()
        assert np.array_equal(kc[n][s[hit]], qc[n][hit])
        # no later key in (s, i) carries the code: per code, walk keys in order
        last = {}
        for t in range(T):
            assert s[t] == last.get(int(qc[n, t]), -1)
            last[int(kc[n, t])] = t


# --------------------------------------------------------------------------- gather
def test_gather_ieee_misses():
    v = np.zeros((1, 3, 4), dtype=np.float32)
    v[0, 0] = [-3.0, np.inf, np.nan, 2.0]
    v[0, 1] = [1, 2, 3, 4]
    v[0, 2] = [5, 6, 7, 8]
    src = np.array([[-1, 0, 1]])
    y = oracle.gather(v, "f32", src, 0)
    assert y[0, 0, 0] == 0 and np.signbit(y[0, 0, 0])          # -3 * 0 = -0
    assert np.isnan(y[0, 0, 1]) and np.isnan(y[0, 0, 2])        # inf * 0, nan * 0
    assert y[0, 0, 3] == 0 and not np.signbit(y[0, 0, 3])
    assert np.array_equal(y[0, 1], v[0, 0], equal_nan=True)
    assert np.array_equal(y[0, 2], v[0, 1])
    yz = oracle.gather(v, "f32", src, 1)
    assert (yz[0, 0].view(np.uint32) == 0).all()                # store path: +0 bytes


def test_gather_bf16_matches_f32_on_representable_values():
    rng = np.random.default_rng(5)
    v32 = rng.standard_normal((3, 20, 8)).astype(np.float32)
    v32 = _f32_bits_of((v32.view(np.uint32) >> 16).astype(np.uint16))   # bf16-exact values
    v32[:, 0, 0] = -1.0
    vb = (v32.view(np.uint32) >> 16).astype(np.uint16)
    src = rng.integers(-1, 20, (3, 20))
    yb = oracle.gather(vb, "bf16", src, 0)
    y32 = oracle.gather(v32, "f32", src, 0)
    assert np.array_equal(_f32_bits_of(yb).view(np.uint32), y32.view(np.uint32))


# ---------------------------------------------------------------------------- store
def _check_store(seed, P, T, chunk, n_codes, capacity, nthreads=1, vb=16):
    """code/tests/test_store.py:17-41 on the C restatement."""
    rng = np.random.default_rng(seed)
    store = oracle.HostStore(vb, P, capacity, nthreads=nthreads)
    ref = oracle.DictStore(P, vb)
    codes = rng.integers(0, n_codes, size=(2, P, T), dtype=np.int64) * 7919 % (n_codes + 2)
    vals = rng.integers(0, 256, size=(P, T, vb), dtype=np.uint8)
    for lo in range(0, T, chunk):
        hi = min(T, lo + chunk)
        qc = np.ascontiguousarray(codes[0, :, lo:hi]).reshape(-1)
        kc = np.ascontiguousarray(codes[1, :, lo:hi]).reshape(-1)
        v = np.ascontiguousarray(vals[:, lo:hi]).reshape(-1, vb)
        out = np.empty_like(v)
        store.exchange(qc, kc, v, out, hi - lo, 0)
        assert np.array_equal(out, ref.exchange(qc, kc, v, hi - lo, 0))
    assert np.array_equal(store.counts, ref.counts())
    return len(store) / store.cap


def test_store_dict_oracle_threaded():
    assert _check_store(0, P=200, T=2000, chunk=500, n_codes=400, capacity=90_000,
                        nthreads=4) > 0.5


def test_store_dict_oracle_decode_sized():
    _check_store(1, P=64, T=300, chunk=1, n_codes=150, capacity=11_000)


def test_store_dict_oracle_one_shot():
    _check_store(2, P=400, T=1000, chunk=1000, n_codes=300, capacity=130_000, nthreads=8)


def test_store_overfull_raises():
    with pytest.raises(RuntimeError, match="full"):
        _check_store(3, P=50, T=100, chunk=100, n_codes=100, capacity=1000)


def test_store_matches_reference_store_bytes():
    """The restatement and the reference's own store.cpp leave the same table, byte for
    byte, and return the same outputs and counts (single thread, so placement is
    deterministic)."""
    ref = oracle.ref_store()
    if ref is None:
        pytest.skip("oracle/_ref was not built (reference sources absent at build time)")
    import torch
    rng = np.random.default_rng(11)
    P, T, vb, cap = 16, 300, 24, 6000
    codes = rng.integers(0, 200, size=(2, P, T), dtype=np.int64) * 7919 % 202
    vals = rng.integers(0, 256, size=(P, T, vb), dtype=np.uint8)
    table = torch.zeros((cap, 16 + vb), dtype=torch.uint8)
    mine = oracle.HostStore(vb, P, cap, nthreads=1)
    counts = np.zeros(P, dtype=np.int64)
    torch.set_num_threads(1)
    for lo, hi in ((0, 100), (100, 101), (101, 300)):
        c = hi - lo
        qc = np.ascontiguousarray(codes[0, :, lo:hi]).reshape(-1)
        kc = np.ascontiguousarray(codes[1, :, lo:hi]).reshape(-1)
        v = np.ascontiguousarray(vals[:, lo:hi]).reshape(-1, vb)
        out = torch.empty((P * c, vb), dtype=torch.uint8)
        counts += ref.exchange(table, torch.from_numpy(qc), torch.from_numpy(kc),
                               torch.from_numpy(v), out, c, 0, cap, vb).numpy()
        mout = np.empty_like(v)
        mine.exchange(qc, kc, v, mout, c, 0)
        assert np.array_equal(mout, out.numpy())
    assert np.array_equal(mine.counts, counts)
    assert np.array_equal(mine.table, table.numpy())


def test_store_home_is_in_range_and_group_mixed():
    cap = 1000
    homes = [oracle.store_home(c, g, cap) for c in range(50) for g in range(4)]
    assert all(0 <= h < cap for h in homes)
    assert oracle.store_home(7, 0, cap) != oracle.store_home(7, 1, cap) or \
        oracle.store_home(8, 0, cap) != oracle.store_home(8, 1, cap)


# ---------------------------------------------------------- CPU-baseline torch port
def test_torch_port_matches_dict_rule():
    """oracle/torch_port.py (the sort-based algorithm timed as the CPU baseline) gives the
    same indices and outputs as the dictionary rule."""
    import torch
    from oracle.torch_port import latest_prev_match_sorted, lema_hard_codes
    rng = np.random.default_rng(4)
    for T, alpha in ((1, 1), (50, 3), (700, 40), (2000, 100000)):
        qc = rng.integers(-5, alpha, (3, T))
        kc = rng.integers(-5, alpha, (3, T))
        got = latest_prev_match_sorted(torch.from_numpy(qc), torch.from_numpy(kc)).numpy()
        assert np.array_equal(got, oracle.latest_prev_match(qc, kc))
    v = rng.standard_normal((1, 3, 2000, 8)).astype(np.float32)
    y = lema_hard_codes(torch.from_numpy(qc).view(1, 3, -1), torch.from_numpy(kc).view(1, 3, -1),
                        torch.from_numpy(v)).numpy()
    want = oracle.gather(v[0], "f32", oracle.latest_prev_match(qc, kc), 0)
    assert np.array_equal(y[0], want)
