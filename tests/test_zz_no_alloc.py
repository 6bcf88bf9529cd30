"""lema_store_exchange_noalloc (the store exchange on the library's own scratch array, no
allocation) against lema_store_exchange_ws (a caller-owned workspace), through the C ABI:
two long calls in a row -- the first over more partitions than one scratch slice holds, the
second smaller -- then a decode-sized step, on two tables that start empty. Every output row,
every per-partition count and the published entries must be identical."""
import numpy as np
import pytest
import torch

from latest_exact_match_attention_amd import _lib
from latest_exact_match_attention_amd.cache import HashStore

pytestmark = pytest.mark.gpu
D_V = 24                                     # bf16 rows of 48 bytes, the workload's


def noalloc(store, qc, kc, v, out, T, g0):
    cb = kc.element_size()
    n = kc.numel()
    _lib.check(_lib.lib().lema_store_exchange_noalloc(
        store.table.data_ptr(), store.cap, store.vbytes,
        qc.data_ptr() if qc is not None else None, kc.data_ptr(), cb, v.data_ptr(),
        out.data_ptr() if out is not None else None, n, T, g0, store.counts_device.data_ptr(),
        store.full_flag.data_ptr(), _lib.stream_of(kc)))


def entries(store):
    g, c, val = store.dump()
    key = g * (1 << 33) + (c & 0xFFFFFFFF)
    order = torch.argsort(key)
    return key[order].cpu(), val[order].cpu()


@pytest.mark.parametrize("code_dtype", [torch.int32, torch.int64])
def test_noalloc_equals_workspace_exchange(dev, code_dtype):
    L = _lib.lib()
    rng = np.random.default_rng(5)
    groups, cap = 80, 9_000_000
    a = HashStore(D_V, groups=groups, dtype=torch.bfloat16, capacity=cap, device=dev)
    b = HashStore(D_V, groups=groups, dtype=torch.bfloat16, capacity=cap, device=dev)
    cb = 4 if code_dtype == torch.int32 else 8
    # (partitions, T, group offset): a call needing several scratch slices, a smaller one
    # fitting one slice, a decode-sized step (no scratch at all)
    calls = [(64, 40_000, 0), (12, 3_000, 60), (80, 1, 0)]
    first_ws = L.lema_store_workspace_bytes(64 * 40_000, 40_000, cb)
    assert first_ws > _lib.NOALLOC_SCRATCH_BYTES          # the first call runs in slices
    assert 0 < L.lema_store_workspace_bytes(12 * 3_000, 3_000, cb) < first_ws
    for P, T, g0 in calls:
        qc = rng.integers(0, 30_000, P * T)
        kc = rng.integers(0, 30_000, P * T)
        qc[::7] = rng.integers(0, 2**32, qc[::7].size)     # misses, bit 31 set in half
        q = torch.from_numpy(qc).to(dev).to(code_dtype)
        k = torch.from_numpy(kc).to(dev).to(code_dtype)
        v = torch.randn((P * T, D_V), device=dev).to(torch.bfloat16)
        out_a = torch.full_like(v, 7.0)
        out_b = torch.empty_like(v)
        noalloc(a, q, k, v, out_a, T, g0)
        a.check_full()
        b.exchange(q, k, v, out_b, T, g0)
        assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), (P, T)
        assert torch.equal(a.counts, b.counts), (P, T)
    ka, va = entries(a)
    kb, vb = entries(b)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert len(a) > 1_000_000


def test_noalloc_insert_only_and_errors(dev):
    L = _lib.lib()
    a = HashStore(D_V, groups=4, dtype=torch.bfloat16, capacity=200_000, device=dev)
    b = HashStore(D_V, groups=4, dtype=torch.bfloat16, capacity=200_000, device=dev)
    kc = torch.randint(0, 5_000, (4 * 20_000,), device=dev, dtype=torch.int64)
    v = torch.randn((kc.numel(), D_V), device=dev).to(torch.bfloat16)
    noalloc(a, None, kc, v, None, 20_000, 0)
    b.exchange(None, kc, v, None, 20_000, 0)
    ka, va = entries(a)
    kb, vb = entries(b)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert torch.equal(a.counts, b.counts)
    rc = L.lema_store_exchange_noalloc(a.table.data_ptr(), a.cap, 48, None, kc.data_ptr(), 8,
                                       v.data_ptr(), None, kc.numel(), 30_001, 0,
                                       a.counts_device.data_ptr(), a.full_flag.data_ptr(),
                                       _lib.stream_of(kc))
    assert rc == _lib.BAD_ARG and b"partitions x T" in L.lema_last_error()


def test_noalloc_replays_in_a_graph(dev):
    """The entry point under HIP graph capture, its intended use: after one eager call (which
    looks the scratch address up), a long call spanning several scratch slices and a decode
    step are captured on one stream. Replayed twice, each time with fresh codes and values
    written into the captured inputs, every output, the counts and the table's entries equal
    the same calls on a twin store through lema_store_exchange_ws."""
    rng = np.random.default_rng(11)
    groups, cap = 64, 9_000_000
    a = HashStore(D_V, groups=groups, dtype=torch.bfloat16, capacity=cap, device=dev)
    b = HashStore(D_V, groups=groups, dtype=torch.bfloat16, capacity=cap, device=dev)
    P, T = 64, 40_000
    assert _lib.lib().lema_store_workspace_bytes(P * T, T, 4) > _lib.NOALLOC_SCRATCH_BYTES

    def draw(n, spread):
        c = rng.integers(0, spread, n)
        c[::5] = rng.integers(0, 2**31, c[::5].size)
        return torch.from_numpy(c).to(dev).to(torch.int32)

    bufs = {"long": (P * T, T), "step": (P, 1)}
    ins = {k: [torch.empty(n, dtype=torch.int32, device=dev),
               torch.empty(n, dtype=torch.int32, device=dev),
               torch.empty((n, D_V), dtype=torch.bfloat16, device=dev),
               torch.empty((n, D_V), dtype=torch.bfloat16, device=dev)]
           for k, (n, _) in bufs.items()}

    def refill():
        for k, (n, _) in bufs.items():
            q, kk, v, _o = ins[k]
            q.copy_(draw(n, 40_000))
            kk.copy_(draw(n, 40_000))
            v.copy_(torch.randn((n, D_V), device=dev).to(torch.bfloat16))

    def run_b():
        outs = {}
        for k, (n, t) in bufs.items():
            q, kk, v, _o = ins[k]
            outs[k] = torch.empty((n, D_V), dtype=torch.bfloat16, device=dev)
            b.exchange(q, kk, v, outs[k], t, 0)
        return outs

    def compare(outs):
        for k in bufs:
            assert torch.equal(ins[k][3].view(torch.int16), outs[k].view(torch.int16)), k
        assert torch.equal(a.counts, b.counts)

    # eager warm-up on the same buffers, then the capture
    refill()
    for k, (n, t) in bufs.items():
        q, kk, v, o = ins[k]
        noalloc(a, q, kk, v, o, t, 0)
    compare(run_b())
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for k, (n, t) in bufs.items():
                q, kk, v, o = ins[k]
                noalloc(a, q, kk, v, o, t, 0)
    torch.cuda.current_stream(dev).wait_stream(s)
    for rep in range(2):
        refill()
        torch.cuda.synchronize(dev)
        g.replay()
        torch.cuda.synchronize(dev)
        a.check_full()
        compare(run_b())
    ka, va = entries(a)
    kb, vb = entries(b)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
