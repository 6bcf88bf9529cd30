"""The store at the sizes of its two benchmark workloads, against the reference's own
store (code/lema/csrc/store.cpp compiled from its source into oracle/_ref/) on a host table
fed the same inputs: every output row and every per-partition count bit for bit.

  batched decode   1,024 partitions (16 sequences x 64 heads), 48-byte bf16 rows,
                   262,144 uniform 32-bit keys prefilled per partition into a 34.5 GB table
                   at load 0.5, then 64 decode steps (T = 1) captured in one HIP graph
  long context     64 partitions (heads), the first two calls of 2^20 positions of the
                   long-context code mix (90% uniform, 10% copies at geometric distance)
                   into the workload's 137 GB table
"""
import math
import sys

import pytest
import torch

import oracle
from latest_exact_match_attention_amd.cache import HashStore
from latest_exact_match_attention_amd.workloads import LONG_CONTEXT, long_context_codes

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def ref():
    r = oracle.ref_store()
    assert r is not None, "oracle/_ref/lema_store_ref.so is not built (make -C oracle ref)"
    return r


def test_decode_workload_at_full_size(dev, ref):
    P, n0, dv, steps = 16 * 64, 262_144, 24, 64
    vbytes = 2 * dv
    cap = math.ceil(P * (n0 + 1024) / 0.5)          # the decode workload's table
    torch.set_num_threads(min(16, torch.get_num_threads()))
    gen = torch.Generator(device=dev).manual_seed(7)
    store = HashStore(dv, groups=P, dtype=torch.bfloat16, capacity=cap, device=dev)
    host = torch.zeros((cap, 16 + vbytes), dtype=torch.uint8)
    host_counts = torch.zeros(P, dtype=torch.int64)
    S = 8192
    for lo in range(0, n0, S):
        kc = torch.randint(0, 2**32, (P, S), dtype=torch.int64, device=dev, generator=gen)
        v = torch.randn((P, S, dv), device=dev, generator=gen).to(torch.bfloat16)
        store.exchange(None, kc.view(-1), v.view(-1, dv), None, S, 0, check=False)
        kh, vh = kc.view(-1).cpu(), v.view(-1, dv).view(torch.int16).cpu()
        host_counts += ref.exchange(host, kh, kh, vh, torch.empty_like(vh), S, 0, cap, vbytes)
        if lo % (8 * S) == 0:
            say(f"decode workload: prefill {lo + S}/{n0} keys per partition")
    store.check_full()
    assert torch.equal(store.counts, host_counts)
    assert 0.49 < store.load() < 0.5

    qc = torch.randint(0, 2**32, (steps, P), dtype=torch.int64, device=dev, generator=gen)
    kc = torch.randint(0, 2**32, (steps, P), dtype=torch.int64, device=dev, generator=gen)
    qc[1::2, ::3] = kc[0:-1:2, ::3]          # every other step, a third of the queries hit
    vv = torch.randn((steps, P, dv), device=dev, generator=gen).to(torch.bfloat16)
    out = torch.empty_like(vv)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for s in range(steps):
            store.exchange(qc[s], kc[s], vv[s], out[s], 1, 0, check=False)
    graph.replay()
    torch.cuda.synchronize()
    store.check_full()
    say("decode workload: graph replayed")
    qh, kh, vh = qc.cpu(), kc.cpu(), vv.view(torch.int16).cpu()
    got = out.view(torch.int16).cpu()
    for s in range(steps):
        oh = torch.empty_like(vh[s])
        host_counts += ref.exchange(host, qh[s], kh[s], vh[s], oh, 1, 0, cap, vbytes)
        assert torch.equal(got[s], oh), f"step {s}"
    assert torch.equal(store.counts, host_counts)
    assert bool((got[1::2, ::3] != 0).any(-1).all())       # the planted hits were found
    del store, host
    torch.cuda.empty_cache()


def test_long_context_workload_first_calls(dev, ref):
    H, L, dv = LONG_CONTEXT["H"], LONG_CONTEXT["call"], LONG_CONTEXT["dv"]
    calls = 2
    vbytes = 2 * dv
    cap = math.ceil(H * LONG_CONTEXT["T"] / 0.5)    # the workload's own table (137 GB)
    store = HashStore(dv, groups=H, dtype=torch.bfloat16, capacity=cap, device=dev)
    cap_h = math.ceil(H * L * calls / 0.5)
    host = torch.zeros((cap_h, 16 + vbytes), dtype=torch.uint8)
    host_counts = torch.zeros(H, dtype=torch.int64)
    for c in range(calls):
        qc64, kc64 = long_context_codes(0, H, c * L, (c + 1) * L, dev)
        qc, kc = qc64.to(torch.int32).contiguous(), kc64.to(torch.int32).contiguous()
        g = torch.Generator(device=dev).manual_seed(1000 + c)
        v = torch.randn((H * L, dv), device=dev, generator=g).to(torch.bfloat16)
        out = torch.empty_like(v)
        store.exchange(qc.view(-1), kc.view(-1), v, out, L, 0)
        vh = v.view(torch.int16).cpu()
        oh = torch.empty_like(vh)
        host_counts += ref.exchange(host, qc64.view(-1).cpu(), kc64.view(-1).cpu(), vh, oh, L,
                                    0, cap_h, vbytes)
        got = out.view(torch.int16).cpu()
        assert torch.equal(got, oh), f"call {c}"
        assert torch.equal(store.counts, host_counts), f"call {c}"
        hits = float((got != 0).any(-1).float().mean())
        say(f"long-context workload: call {c + 1}/{calls} identical, hit rate {hits:.4f}")
        assert hits > 0.05
    del store, host
    torch.cuda.empty_cache()


def test_long_context_workload_all_calls(dev):
    """The whole long-context run: all 16 calls of 2^20 positions of the 64 heads through the
    workload's 137 GB table. Each value row carries its key's own (head, position + 1) in its
    first 8 bytes (the store copies rows as opaque bytes), so every returned row names the key
    it came from, and a miss returns 0. Per head, the reference's sort-based algorithm
    (code/lema/attention.py:100-132, oracle/torch_port.py, on the device) over all 2^24
    positions gives the latest earlier key with the query's code. Every query of every call
    must return exactly that key, and the final per-head counts must equal the number of
    distinct key codes of the head (code/lema/cache.py:27-30: any chunking gives the one-shot
    result)."""
    from oracle.torch_port import latest_prev_match_sorted
    H, T, L, dv = LONG_CONTEXT["H"], LONG_CONTEXT["T"], LONG_CONTEXT["call"], LONG_CONTEXT["dv"]
    calls = T // L
    cap = math.ceil(H * T / 0.5)
    store = HashStore(dv, groups=H, dtype=torch.bfloat16, capacity=cap, device=dev)
    head = torch.arange(H, dtype=torch.int64, device=dev).view(H, 1)
    qc_all = torch.empty((H, T), dtype=torch.int64, device=dev)
    kc_all = torch.empty((H, T), dtype=torch.int64, device=dev)
    got = torch.empty((H, T), dtype=torch.int64, device=dev)
    for c in range(calls):
        t0 = c * L
        qc64, kc64 = long_context_codes(0, H, t0, t0 + L, dev)
        qc_all[:, t0:t0 + L] = qc64
        kc_all[:, t0:t0 + L] = kc64
        v = torch.zeros((H, L, dv), dtype=torch.int16, device=dev)
        pos = torch.arange(t0, t0 + L, dtype=torch.int64, device=dev).view(1, L)
        v.view(torch.int64)[:, :, 0] = (head << 32) | (pos + 1)    # rows: 6 int64 words
        out = torch.empty((H * L, dv), dtype=torch.bfloat16, device=dev)
        store.exchange(qc64.to(torch.int32).view(-1), kc64.to(torch.int32).view(-1),
                       v.view(H * L, dv).view(torch.bfloat16), out, L, 0)
        got[:, t0:t0 + L] = out.view(torch.int64).view(H, L, dv // 4)[:, :, 0]
        del v, out
        say(f"long-context full run: call {c + 1}/{calls} done, table load {store.load():.3f}")
    assert store.load() > 0.44
    hits = 0
    for h in range(H):
        src = latest_prev_match_sorted(qc_all[h:h + 1], kc_all[h:h + 1])[0]
        want = torch.where(src >= 0, (h << 32) | (src + 1), torch.zeros_like(src))
        bad = int((got[h] != want).sum())
        assert bad == 0, f"head {h}: {bad} of {T} queries differ from the oracle"
        hits += int((src >= 0).sum())
        n_keys = torch.unique(kc_all[h]).numel()
        assert int(store.counts[h]) == n_keys, (h, int(store.counts[h]), n_keys)
        if h % 16 == 15:
            say(f"long-context full run: heads 0-{h} equal the oracle over all {calls} calls")
    say(f"long-context full run: {H * T} queries over {calls} calls identical, hit rate "
        f"{hits / (H * T):.4f}")
    assert hits / (H * T) > 0.05
    del store, qc_all, kc_all, got
    torch.cuda.empty_cache()
