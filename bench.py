"""Benchmark of the LEMA hot path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload zipf_prefill|decode]

zipf_prefill (default): B8 H16 T16384, 24-bit Zipf(1.1) codes over 4096 distinct codes per
(b, h), d_v 64 bf16. A step is one fused resolve+gather launch over the whole batch, inputs
resident in HBM: per query it reads the query and key code (4 + 4 B) and a value row
(128 B, compulsory once) and writes the match index (4 B) and the output row (128 B):
268 B/query algorithmic, 562 MB per step. `value` = matched queries resolved per second.

`roofline` prices the fused kernel's algorithmic bytes against MI355X's 8 TB/s HBM peak,
with the kernel time measured by HIP events on the stream it is launched on. `traffic` is
the HBM bytes per launch from the rocprofv3 FETCH_SIZE/WRITE_SIZE summary committed in
profiles/ (null if absent). `cpu_baseline` times the reference's sort-based CPU algorithm
(torch ops on the host's cores) on a bounded sample of the same workload.

decode: batched decode against the HBM store -- 16 sequences x 64 heads = 1024 partitions,
d_v 24 bf16, the store prefilled with 262,144 uniform 32-bit keys per partition (load 0.5,
34.5 GB), then 1024 steps each looking up one fresh uniform query and inserting one fresh key
per partition, captured in one HIP graph. `value` = decode steps per second. The reference's
own C++ store (code/lema/csrc/store.cpp, compiled into oracle/_ref/) runs the same prefill and
steps on the host's cores as the CPU baseline, and every step's outputs and the final counts
must agree bit for bit.

One GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BYTES_PER_QUERY = 4 + 4 + 4 + 128 + 128


def parse():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="zipf_prefill", choices=["zipf_prefill", "decode"])
    ap.add_argument("--decode-prefill", type=int, default=262144,
                    help="keys prefilled per partition for the decode workload")
    ap.add_argument("--decode-steps", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=16,
                    help="(b, h) rows of the workload timed for the CPU baseline")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one plain device copy of the value tensor (known bytes), "
                         "to calibrate profiler memory counters")
    return ap.parse_args()


def load_traffic(name: str):
    """HBM bytes per launch measured by rocprofv3 PMC counters (profiles/traffic.json)."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get(name, {}).get("bytes_per_launch")
    except Exception:
        return None


def cpu_baseline_prefill(qc, kc, v32, rows: int):
    """The reference's CPU algorithm (attention.py:100-158 via oracle/torch_port.py) on the
    first `rows` (b, h) rows of the workload, bf16 values, all host cores."""
    import torch
    from oracle.torch_port import lema_hard_codes
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    B, H, T = qc.shape
    q = torch.from_numpy(qc.reshape(B * H, T)[:rows]).view(1, rows, T)
    k = torch.from_numpy(kc.reshape(B * H, T)[:rows]).view(1, rows, T)
    v = torch.from_numpy(v32.reshape(B * H, T, -1)[:rows]).to(torch.bfloat16).view(1, rows, T, -1)
    for _ in range(2):
        lema_hard_codes(q, k, v)
    times = []
    t_end = time.perf_counter() + 20.0
    while len(times) < 10 and (time.perf_counter() < t_end or len(times) < 3):
        t0 = time.perf_counter()
        lema_hard_codes(q, k, v)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": rows * T / med, "unit": "queries/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of {B * H} (b,h) rows x T={T} ({rows * T} queries), bf16 "
                      f"d_v {v.shape[-1]}; median of {len(times)} runs, "
                      f"{med * 1e3:.1f} ms per run"}


def bench_prefill(a):
    import numpy as np
    import torch
    from latest_exact_match_attention_amd import build
    from latest_exact_match_attention_amd.attention import launch_hard
    from latest_exact_match_attention_amd.workloads import ZIPF_PREFILL, zipf_prefill

    if not build.LIB.exists():
        build.build()
    cfg = ZIPF_PREFILL
    B, H, T, dv = cfg["B"], cfg["H"], cfg["T"], cfg["dv"]
    qc, kc, v32 = zipf_prefill(0)
    dev = torch.device("cuda", 0)
    qd = torch.from_numpy(qc.reshape(B * H, T)).to(dev).to(torch.int32)
    kd = torch.from_numpy(kc.reshape(B * H, T)).to(dev).to(torch.int32)
    vd = torch.from_numpy(v32).to(dev).to(torch.bfloat16)
    y = torch.empty_like(vd)
    src = torch.empty((B, H, T), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    if a.copy_probe:
        y.copy_(vd)                      # reads and writes exactly vd.numel() * 2 bytes
        torch.cuda.synchronize()
    for _ in range(a.warmup):
        launch_hard(qd, kd, vd, y, src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(a.steps):
        launch_hard(qd, kd, vd, y, src)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    hits = float((src >= 0).float().mean().item())
    nq = B * H * T
    achieved = BYTES_PER_QUERY * nq / (ms * 1e-3) / 1e9
    cpu = None if a.no_cpu_baseline else cpu_baseline_prefill(qc, kc, v32, a.cpu_rows)
    return {
        "metric": "prefill matched queries/sec @T=16k; decode steps/sec; % of HBM peak",
        "value": nq / (ms * 1e-3),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32 codes, bf16 values",
        "data": "synthetic (seeded numpy: Zipf codes, N(0,1) values)",
        "config": {"workload": "zipf_prefill", "B": B, "H": H, "T": T, "code_bits": cfg["bits"],
                   "distinct_codes": cfg["distinct"], "zipf_s": cfg["s"], "d_v": dv,
                   "value_dtype": "bf16", "hit_rate": round(hits, 4),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic("resolve_kernel/zipf_prefill"),
                     "kernel": "resolve_kernel (fused resolve + gather)",
                     "bytes_per_query": BYTES_PER_QUERY, "queries_per_launch": nq},
        "cpu_baseline": cpu,
    }


DECODE_BYTES_PER_ITEM = 8 + 8 + 48 + 48 + 64 + 2 * 64   # codes, value in/out, 3 slot touches


def bench_decode(a):
    """Batched decode steps against the HBM store, hipGraph-captured, vs the reference store
    on the host (same inputs, outputs compared bit for bit)."""
    import math
    import numpy as np
    import torch
    from latest_exact_match_attention_amd import build
    from latest_exact_match_attention_amd.cache import HashStore

    if not build.LIB.exists():
        build.build()
    seqs, heads, dv = 16, 64, 24
    P, n0, steps = seqs * heads, a.decode_prefill, a.decode_steps
    max_load = 0.5
    cap = math.ceil(P * (n0 + steps) / max_load)
    vbytes = dv * 2
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(0)
    store = HashStore(dv, groups=P, dtype=torch.bfloat16, capacity=cap, device=dev)
    ref = None
    if not a.no_cpu_baseline:
        import oracle
        ref = oracle.ref_store()
        if ref is None:
            print("oracle/_ref/lema_store_ref.so missing: no CPU baseline", file=sys.stderr)
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    host_table = torch.zeros((cap, 16 + vbytes), dtype=torch.uint8) if ref is not None else None
    host_counts = torch.zeros(P, dtype=torch.int64)

    # prefill, partition-major slices of S positions: the GPU store inserts them, the host
    # store exchanges the same keys (its looked-up values are discarded)
    S = 8192
    t_cpu_prefill = 0.0
    t_start = time.perf_counter()
    for lo in range(0, n0, S):
        if lo % (8 * S) == 0:
            print(f"decode prefill: {lo}/{n0} keys per partition inserted "
                  f"({time.perf_counter() - t_start:.1f} s)", file=sys.stderr, flush=True)
        w = min(S, n0 - lo)
        kc = torch.randint(0, 2**32, (P, w), dtype=torch.int64, device=dev, generator=gen)
        v = torch.randn((P, w, dv), device=dev, generator=gen).to(torch.bfloat16)
        store.exchange(None, kc.view(-1), v.view(-1, dv), None, w, 0, check=False)
        if ref is not None:
            kh, vh = kc.view(-1).cpu(), v.view(-1, dv).view(torch.int16).cpu()
            oh = torch.empty_like(vh)
            t0 = time.perf_counter()
            host_counts += ref.exchange(host_table, kh, kh, vh, oh, w, 0, cap, vbytes)
            t_cpu_prefill += time.perf_counter() - t0
    store.check_full()

    # the steps' inputs, resident in HBM before the timed region
    qc = torch.randint(0, 2**32, (steps, P), dtype=torch.int64, device=dev, generator=gen)
    kc = torch.randint(0, 2**32, (steps, P), dtype=torch.int64, device=dev, generator=gen)
    vv = torch.randn((steps, P, dv), device=dev, generator=gen).to(torch.bfloat16)
    out = torch.empty_like(vv)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for s_ in range(steps):
            store.exchange(qc[s_], kc[s_], vv[s_], out[s_], 1, 0, check=False)
    stream = torch.cuda.current_stream(dev)
    x = torch.empty(1 << 26, device=dev)
    for _ in range(20):                      # clocks up; the store is not touched
        x.mul_(1.0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    store.check_full()
    ms_step = e0.elapsed_time(e1) / steps
    hits = None

    cpu = None
    parity = None
    if ref is not None:
        qh, kh = qc.cpu(), kc.cpu()
        vh = vv.view(torch.int16).cpu()
        oh = torch.empty_like(vh)
        times = []
        for s_ in range(steps):
            t0 = time.perf_counter()
            host_counts += ref.exchange(host_table, qh[s_], kh[s_], vh[s_], oh[s_], 1, 0, cap,
                                        vbytes)
            times.append(time.perf_counter() - t0)
        got = out.view(torch.int16).cpu()
        same_out = bool(torch.equal(got, oh))
        same_counts = bool(torch.equal(store.counts, host_counts))
        hits = float((got.view(steps, P, dv) != 0).any(-1).float().mean())
        med = sorted(times)[len(times) // 2]
        cpu = {"value": 1.0 / med, "unit": "decode steps/s", "cores": threads,
               "kind": "reference",
               "sample": f"all {steps} steps of the workload through code/lema/csrc/store.cpp "
                         f"(compiled from source, OpenMP, grain 128/T) on a host table in "
                         f"the same state; median {med * 1e6:.1f} us/step, mean "
                         f"{sum(times) / len(times) * 1e6:.1f} us/step; its prefill took "
                         f"{t_cpu_prefill:.1f} s"}
        parity = {"step_outputs_identical": same_out, "counts_identical": same_counts}
        if not (same_out and same_counts):
            print(f"decode parity FAILED: outputs {same_out} counts {same_counts}",
                  file=sys.stderr)
    per_step_bytes = DECODE_BYTES_PER_ITEM * P
    achieved = per_step_bytes / (ms_step * 1e-3) / 1e9
    return {
        "metric": "prefill matched queries/sec @T=16k; decode steps/sec; % of HBM peak",
        "value": 1e3 / ms_step,
        "unit": "decode steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 0,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64 codes, bf16 values (opaque 48-byte rows)",
        "data": "synthetic (torch device RNG: uniform 32-bit codes, N(0,1) values)",
        "config": {"workload": "decode", "partitions": P, "sequences": seqs, "heads": heads,
                   "d_v": dv, "prefilled_per_partition": n0, "capacity": cap,
                   "table_bytes": cap * (16 + vbytes), "load_after": round(store.load(), 4),
                   "graph": f"{steps} steps in one HIP graph", "hit_rate": hits,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "latency (dependent HBM round trips per step)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "store_step_kernel",
                     "bytes_per_item": DECODE_BYTES_PER_ITEM, "items_per_launch": P},
        "cpu_baseline": cpu,
        "parity": parity,
    }


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got "
              f"--gpus {a.gpus}", file=sys.stderr)
        return 2
    out = bench_decode(a) if a.workload == "decode" else bench_prefill(a)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
