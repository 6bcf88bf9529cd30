"""Write the golden fixtures of this directory (inputs and expected outputs, .npz).

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path, so the expected outputs are made here:
  * latest_match.npz, pack.npz, gather.npz -- by the C oracle, after checking each case
    against an independent restatement (the dictionary rule of verification/lema.py:19-33,
    an O(T^2) brute force, per-element IEEE tests);
  * store.npz -- by the reference's own C++ store (code/lema/csrc/store.cpp, compiled into
    oracle/_ref/ by oracle/Makefile), checked against a per-partition dict
    (code/tests/test_store.py:17-41) and against the C oracle's restatement of the store.
Rerunning it must reproduce the committed files bit for bit (tests/test_golden.py checks
the CPU side of that).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402

U64 = np.uint64


def latest_match_cases():
    """Edge rows first, then random small-alphabet rows; all rows T = 96."""
    T = 96
    rows = []
    rows.append((np.full(T, 5), np.full(T, 5)))                       # all equal: src = i - 1
    rows.append((np.arange(T), np.arange(T) + 1000))                   # disjoint: all -1
    rows.append((np.arange(T), np.arange(T)))                          # self only: all -1
    rows.append((np.arange(T) % 2, (np.arange(T) + 1) % 2))            # alternating
    special = np.array([0, 1, -1, np.iinfo(np.int64).min, np.iinfo(np.int64).max, 2**32 - 1,
                        2**32], dtype=np.int64)
    rng = np.random.default_rng(1234)
    rows.append((special[rng.integers(0, len(special), T)],
                 special[rng.integers(0, len(special), T)]))            # sentinel-ish codes
    for a in (2, 3, 8, 40, 1 << 20):
        rows.append((rng.integers(0, a, T), rng.integers(0, a, T)))
    qc = np.stack([r[0] for r in rows]).astype(np.int64)
    kc = np.stack([r[1] for r in rows]).astype(np.int64)
    src = oracle.latest_prev_match(qc, kc)
    for n in range(len(rows)):
        assert list(src[n]) == oracle.dict_rule(qc[n], kc[n])
        assert (src[n] == oracle.brute_force(qc[n], kc[n])).all()
    assert (src[0] == np.arange(T) - 1).all() and (src[1] == -1).all() and (src[2] == -1).all()
    return dict(qc=qc, kc=kc, src=src)


def pack_cases():
    rng = np.random.default_rng(99)
    out = {}
    specials = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40,
                         3.0e38, -3.0e38], dtype=np.float32)
    for D in (24, 64):
        z = rng.standard_normal((64, D)).astype(np.float32)
        z[rng.random((64, D)) < 0.2] = specials[rng.integers(0, len(specials), 1)][0]
        z.reshape(-1)[: len(specials)] = specials
        codes = oracle.pack_codes(z, "f32")
        bits = (z >= 0)                                            # numpy IEEE compare
        want = np.zeros(64, dtype=U64)
        for j in range(D):
            want |= bits[:, j].astype(U64) << U64(j)
        assert (codes == want).all()
        out[f"z_f32_d{D}"] = z
        out[f"codes_f32_d{D}"] = codes
        zb = rng.integers(0, 1 << 16, size=(64, D), dtype=np.uint16)    # any bf16 pattern
        out[f"z_bf16_d{D}"] = zb
        out[f"codes_bf16_d{D}"] = oracle.pack_codes(zb, "bf16")
        zh = rng.integers(0, 1 << 16, size=(64, D), dtype=np.uint16)    # any f16 pattern
        out[f"z_f16_d{D}"] = zh
        out[f"codes_f16_d{D}"] = oracle.pack_codes(zh, "f16")
    return out


def gather_cases():
    rng = np.random.default_rng(7)
    N, T, dv = 6, 50, 24
    v = rng.standard_normal((N, T, dv)).astype(np.float32)
    v[0, 0, :4] = [-1.0, np.inf, -np.inf, np.nan]        # the dense miss row's specials
    v[1, 0, :] = -2.0
    src = np.where(rng.random((N, T)) < 0.3, -1, rng.integers(0, T, (N, T)))
    src[:, 0] = -1
    out = dict(v_f32=v, src=src.astype(np.int64))
    out["y_f32_dense"] = oracle.gather(v, "f32", src, 0)
    out["y_f32_zero"] = oracle.gather(v, "f32", src, 1)
    vb = (v.view(np.uint32) >> 16).astype(np.uint16)     # truncated to bf16 bit patterns
    out["v_bf16"] = vb
    out["y_bf16_dense"] = oracle.gather(vb, "bf16", src, 0)
    out["y_bf16_zero"] = oracle.gather(vb, "bf16", src, 1)
    y = out["y_f32_dense"]
    miss = src < 0
    assert np.array_equal(y[~miss], v[np.nonzero(~miss)[0], src[~miss]], equal_nan=True)
    assert np.signbit(y[1, 0]).all() and (y[1, 0] == 0).all()          # -2 * 0 = -0
    assert np.isnan(y[0, 0, 1:4]).all()                                 # inf/nan * 0 = nan
    return out


def store_cases():
    ref = oracle.ref_store()
    if ref is None:
        raise SystemExit("store.npz needs oracle/_ref (make -C oracle with the reference "
                         "sources mounted)")
    import torch
    P, T, vb = 8, 40, 16
    chunks = [16, 1, 1, 7, 15]
    rng = np.random.default_rng(3)
    n_codes = 12
    codes = rng.integers(0, n_codes, size=(2, P, T)) * 7919 % (n_codes + 2)
    codes[:, 0, :5] = [[0, 1, -1, 0, 1], [1, 0, -1, -1, 0]]
    codes = codes.astype(np.int64)
    vals = rng.integers(0, 256, size=(P, T, vb), dtype=np.uint8)
    cap = 96
    table = torch.zeros((cap, 16 + vb), dtype=torch.uint8)
    dstore = oracle.DictStore(P, vb)
    ostore = oracle.HostStore(vb, P, cap)
    outs = []
    counts = np.zeros(P, dtype=np.int64)
    lo = 0
    for c in chunks:
        hi = lo + c
        qc = np.ascontiguousarray(codes[0, :, lo:hi]).reshape(-1)
        kc = np.ascontiguousarray(codes[1, :, lo:hi]).reshape(-1)
        v = np.ascontiguousarray(vals[:, lo:hi]).reshape(-1, vb)
        out = torch.empty((P * c, vb), dtype=torch.uint8)
        added = ref.exchange(table, torch.from_numpy(qc), torch.from_numpy(kc),
                             torch.from_numpy(v), out, c, 0, cap, vb)
        counts += added.numpy()
        want = dstore.exchange(qc, kc, v, c, 0)
        assert np.array_equal(out.numpy(), want)
        oout = np.empty_like(v)
        ostore.exchange(qc, kc, v, oout, c, 0)
        assert np.array_equal(oout, want)
        outs.append(out.numpy().reshape(P, c, vb))
        lo = hi
    assert np.array_equal(counts, dstore.counts())
    assert np.array_equal(ostore.table, table.numpy())        # same slots, byte for byte
    return dict(codes=codes, vals=vals, chunks=np.array(chunks), cap=np.array(cap),
                out=np.concatenate(outs, axis=1), counts=counts)


def main():
    np.savez_compressed(HERE / "latest_match.npz", **latest_match_cases())
    np.savez_compressed(HERE / "pack.npz", **pack_cases())
    np.savez_compressed(HERE / "gather.npz", **gather_cases())
    np.savez_compressed(HERE / "store.npz", **store_cases())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
