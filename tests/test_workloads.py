"""The synthetic long-context codes against their definition, restated with Python integers
(no torch): the counter hash, the copy links and the query copies."""
import math

import numpy as np
import torch

from latest_exact_match_attention_amd.workloads import long_context_codes

M64 = (1 << 64) - 1
GOLD = 0x9E3779B97F4A7C15


def mix(x):
    x &= M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def h(seed, stream, head, pos):
    key = (GOLD * (seed * 8 + stream + 1)) & M64
    return mix(mix((pos & M64) ^ key) ^ ((head * GOLD) & M64))


def unit(x):
    return (x >> 11) * 2.0 ** -53


def geometric(x, p):
    u = ((x >> 11) + 1) * 2.0 ** -53
    return 1 + math.floor(math.log(u) / math.log1p(-p))


def key_code(seed, head, pos, pc=0.1, pg=1e-5):
    while unit(h(seed, 0, head, pos)) < pc and pos - geometric(h(seed, 1, head, pos), pg) >= 0:
        pos -= geometric(h(seed, 1, head, pos), pg)
    return h(seed, 2, head, pos) & 0xFFFFFFFF


def query_code(seed, head, pos, pc=0.1, pg=1e-5):
    src = pos - geometric(h(seed, 4, head, pos), pg)
    if unit(h(seed, 3, head, pos)) < pc and src >= 0:
        return key_code(seed, head, src, pc, pg)
    return h(seed, 5, head, pos) & 0xFFFFFFFF


def test_long_context_codes_follow_the_definition():
    H, t0, t1 = 3, 250_000, 250_400
    qc, kc = long_context_codes(7, H, t0, t1)
    for hd in range(H):
        for i in range(0, t1 - t0, 7):
            assert int(kc[hd, i]) == key_code(7, hd, t0 + i), (hd, i)
            assert int(qc[hd, i]) == query_code(7, hd, t0 + i), (hd, i)


def test_long_context_copies_hit_and_slices_agree():
    qc, kc = long_context_codes(0, 2, 0, 300_000, p_geom=1e-3)     # short links for the test
    q2, k2 = long_context_codes(0, 2, 100_000, 200_000, p_geom=1e-3)
    assert torch.equal(qc[:, 100_000:200_000], q2) and torch.equal(kc[:, 100_000:200_000], k2)
    assert int(qc.max()) < 2 ** 32 and int(qc.min()) >= 0
    # a query that copies finds its code among the earlier keys of its head
    for hd in range(2):
        k = kc[hd].numpy()
        first = {}
        for j, c in enumerate(k):
            first.setdefault(int(c), j)
        q = qc[hd].numpy()
        hits = np.array([first.get(int(c), 1 << 40) < i for i, c in enumerate(q)])
        assert 0.07 < hits.mean() < 0.13                # ~p_copy of the queries
        # keys copy too: the fraction of repeated key codes is about p_copy
        assert 0.07 < 1 - len(first) / len(k) < 0.13
