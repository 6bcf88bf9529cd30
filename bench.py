"""Benchmark of the LEMA hot path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|zipf_prefill|decode|...]

all (default): the zipf_prefill line below, with the decode, long_context and lm_forward
workloads run after it in the same process and carried as sub-records of the one JSON line
("decode", "long_context", "lm_forward": each with its own value, unit, ms_per_step,
roofline, cpu_baseline and parity flags). --steps and --warmup apply to the prefill line;
the sub-records use their own workload's defaults (lm_forward: 3 steps after 1 warm-up).

zipf_prefill: B8 H16 T16384, 24-bit Zipf(1.1) codes over 4096 distinct codes per
(b, h), d_v 64 bf16. A step is one fused resolve+gather launch over the whole batch, inputs
resident in HBM: per query it reads the query and key code (4 + 4 B) and a value row
(128 B, compulsory once) and writes the match index (4 B) and the output row (128 B):
268 B/query algorithmic, 562 MB per step. `value` = matched queries resolved per second.
The untimed warm-up runs the W steps asked for and continues until 0.5 s of launches have run
(clocks settle); the timed region is exactly K launches.

`roofline` prices the fused kernel's algorithmic bytes against MI355X's 8 TB/s HBM peak,
with the kernel time measured by HIP events on the stream it is launched on. `traffic` is
the L2-miss bytes per launch (served by HBM or the 256 MB Infinity Cache) from the rocprofv3
FETCH_SIZE/WRITE_SIZE summary committed in profiles/ (null if absent). Back-to-back launches
over the same batch find part of it in the Infinity Cache; `cold_cache` times the same
launch, and the same device copy, each after a read of a 1 GiB buffer that evicts L2 and the
Infinity Cache. `cpu_baseline` times the reference's sort-based CPU algorithm
(torch ops on the host's cores) on a bounded sample of the same workload.

decode: batched decode against the HBM store -- 16 sequences x 64 heads = 1024 partitions,
d_v 24 bf16, the store prefilled with 262,144 uniform 32-bit keys per partition (load 0.5,
34.5 GB), then 1024 steps each looking up one fresh uniform query and inserting one fresh key
per partition, captured in one HIP graph. `value` = decode steps per second. The reference's
own C++ store (code/lema/csrc/store.cpp, compiled into oracle/_ref/) runs the same prefill and
steps on the host's cores as the CPU baseline, and every step's outputs and the final counts
must agree bit for bit.

lm_forward: the full LEMA language model forward with its loss -- vocab 50304, 24 layers,
d_model 1536, 64 heads (d_qk = d_v = 24, 24-bit codes), SwiGLU 6144, bf16, random init
(torch.manual_seed(0)), B4 x T16384 uniform token ids. A step is one forward + chunked
cross-entropy; `value` = tokens per second. The projections, MLP and head are bf16 GEMMs on
the matrix cores (torch); each layer's exact op is the fused HIP kernel. `roofline` prices
the step's GEMM FLOPs against the dense bf16 MFMA peak; `lema_kernel` gives the fused op's
own HBM fraction at the layer shape, back to back on layer 0's codes and after the cache
eviction of the prefill line (inside the forward it runs between other kernels' traffic). `cpu_baseline` runs the model forward restated in torch
with the reference's sort-based exact op on the host's cores, fp32, on a short sample.

long_context: B1 H64, T = 2^24 fed through the HBM store in 16 calls of 2^20 positions
(one `HashStore.exchange` per call, P = 64 partitions x T = 2^20), 32-bit codes: each key is
uniform with probability 0.9, else a copy of the key d positions back, d ~ Geometric(1e-5)
(mean 1e5); each query likewise copies an earlier key or is uniform; d_v 24 bf16 ~N(0,1).
Codes come from a counter-based hash of (seed, head, position) and values from a per-call
seeded generator, made on the device for each call before it is timed. `value` = queries
per second over the timed exchanges. The first call also runs through the reference's own
C++ store on the host (`--long-parity-calls` of them): outputs and counts must agree bit for
bit, and its time is the CPU baseline. Each value row's first 8 bytes name its key (head,
position + 1); after the timed calls, every query of every call is checked against the
reference's sort-based algorithm run per head over all positions on the device, and the final
counts against each head's distinct key codes (`parity.all_calls`; `--no-full-parity` skips it).

decode_model: single-token decoding of the lm_forward model (24 layers, d_model 1536, 64
heads, bf16) for a batch of 16 streams after a 4,096-token prompt, through the HBM store with
worst-case codes (fresh random 64-bit codes every layer and step, the reference's inference
benchmark hook): one HIP graph replay per token, every layer's store exchange inside it.
`value` = tokens per second (batch / step time); `roofline` prices the weights and store
traffic a step must read against HBM peak.

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
WARM_SECONDS = 0.5      # least untimed warm-up of the prefill workload (clocks settle)
MFMA_BF16_PEAK_TFLOPS = 2500.0
LM_CONFIG = dict(vocab_size=50304, depth=24, dim=1536, num_heads=64, dim_ff=6144)
# The reference's own 0.8B inference geometry (code/experiments/main_inference/run_paper.sh:72,
# "G08 ... --head-dim 64"; 834,086,400 parameters) and its published LEMA numbers with the
# host-RAM store on one RTX 3090 (code/experiments/main_inference/out/*.jsonl).
REF08B_CONFIG = dict(vocab_size=50304, depth=24, dim=1536, num_heads=24, d_qk=64, d_v=64,
                     dim_ff=4096)
REF08B_PUBLISHED = {
    "decode_b1_worst_case_ms_per_token_at_16k": [3.049, "gen_08B_ram.jsonl:11"],
    "decode_b16_trained_ms_per_token_at_16": [4.280, "genB16_08B_trained_ram.jsonl:1"],
    "prefill_b1_worst_case_tokens_per_s_at_16384": [19238, "prefill_08B_ram.jsonl:8"],
    "hardware": "one RTX 3090 + host-RAM store (16 host threads)",
}
BYTES_PER_QUERY = 4 + 4 + 4 + 128 + 128


def parse():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="all",
                    choices=["all", "zipf_prefill", "decode", "lm_forward", "long_context",
                             "decode_model"])
    ap.add_argument("--dm-batch", type=int, default=16)
    ap.add_argument("--dm-prompt", type=int, default=4096)
    ap.add_argument("--dm-steps", type=int, default=256)
    ap.add_argument("--dm-geometry", choices=["lm", "ref08b"], default="lm",
                    help="decode_model geometry: the lm_forward model (64 heads of 24) or the "
                         "reference's 0.8B inference model (24 heads of 64, SwiGLU 4096)")
    ap.add_argument("--long-calls", type=int, default=16,
                    help="calls of 2^20 positions of the long_context workload to run")
    ap.add_argument("--long-parity-calls", type=int, default=1,
                    help="leading calls also run through the reference store on the host")
    ap.add_argument("--no-full-parity", action="store_true",
                    help="long_context: skip checking every call's outputs against the "
                         "sort-based oracle after the timed calls")
    ap.add_argument("--lm-batch", type=int, default=4)
    ap.add_argument("--lm-seq", type=int, default=16384)
    ap.add_argument("--lm-cpu-tokens", type=int, default=512,
                    help="tokens (batch 1) of the lm_forward CPU-baseline sample")
    ap.add_argument("--decode-prefill", type=int, default=262144,
                    help="keys prefilled per partition for the decode workload")
    ap.add_argument("--decode-steps", type=int, default=1024)
    ap.add_argument("--decode-place", choices=["hbm", "ram"], default="hbm",
                    help="decode: the store table in device memory or in pinned host RAM")
    ap.add_argument("--step-stamps", action="store_true",
                    help="decode: run the diagnostics build (build --stamps), whose step kernel "
                         "reads the clock after each phase, and report the breakdown and the "
                         "cost of an empty graph node")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=16,
                    help="(b, h) rows of the workload timed for the CPU baseline")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one plain device copy of the value tensor (known bytes), "
                         "to calibrate profiler memory counters")
    return ap.parse_args()


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baselines."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


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
            "cpu_model": cpu_model(),
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
    # Untimed warm-up: the W steps asked for, continued until 0.5 s of launches have run, so
    # the timed steps see settled clocks (a launch is ~0.1 ms; 10 of them end while the clocks
    # still ramp, which reads ~5% slow).
    t_warm = time.perf_counter()
    done = 0
    while done < a.warmup or time.perf_counter() - t_warm < WARM_SECONDS:
        for _ in range(10):
            launch_hard(qd, kd, vd, y, src)
        done += 10
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
    # after the timed region; the copies overwrite y
    cold = cold_ms(lambda: launch_hard(qd, kd, vd, y, src), stream)
    copy_gbps = measured_copy_gbps(vd, y, stream, lib_copy=True)
    torch_copy_gbps = measured_copy_gbps(vd, y, stream)
    copy_cold = measured_copy_gbps(vd, y, stream, lib_copy=True, cold=True)
    achieved_cold = BYTES_PER_QUERY * nq / (cold * 1e-3) / 1e9
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
                     "traffic": load_traffic("resolve_lag_kernel/zipf_prefill"),
                     "kernel": "resolve_lag_kernel (fused resolve + gather, persistent)",
                     "bytes_per_query": BYTES_PER_QUERY, "queries_per_launch": nq,
                     "copy_measured": {"GBps": copy_gbps, "frac": achieved / copy_gbps,
                                       "what": "lema_device_copy of the value tensor (read + "
                                               f"write {2 * vd.numel() * vd.element_size()} "
                                               "bytes), HIP events, median of 20",
                                       "torch_copy_GBps": torch_copy_gbps}},
        "cold_cache": {"ms_per_step": cold, "value": nq / (cold * 1e-3),
                       "achieved_GBps": achieved_cold, "frac": achieved_cold / HBM_PEAK_GBS,
                       "copy_GBps": copy_cold, "copy_frac": achieved_cold / copy_cold,
                       "what": f"each launch (and each copy) timed alone by HIP events after a "
                               f"read of {FLUSH_BYTES >> 30} GiB that evicts L2 and the Infinity "
                               f"Cache; median of {COLD_REPS}"},
        "cpu_baseline": cpu,
    }


FLUSH_BYTES = 1 << 30   # larger than L2 (8 x 4 MB) and the Infinity Cache (256 MB) together
COLD_REPS = 15
_flush = {}


def evict_caches(stream) -> None:
    """Read FLUSH_BYTES of device memory (a float32 sum, nothing large written), so that what
    runs next finds none of its data in L2 or the Infinity Cache."""
    import torch
    dev = stream.device
    if dev not in _flush:
        _flush[dev] = (torch.ones(FLUSH_BYTES // 2, dtype=torch.bfloat16, device=dev),
                       torch.empty((), dtype=torch.float32, device=dev))
    buf, acc = _flush[dev]
    torch.sum(buf, dim=(0,), dtype=torch.float32, out=acc)


def cold_ms(run, stream, reps: int = COLD_REPS) -> float:
    """Median time (ms) of run() by HIP events, each call right after evict_caches."""
    import torch
    run()
    times = []
    for _ in range(reps):
        evict_caches(stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    times.sort()
    return times[len(times) // 2]


def measured_copy_gbps(src, dst, stream, reps: int = 20, lib_copy: bool = False,
                       cold: bool = False) -> float:
    """A device copy's rate on this GPU (bytes read + written per second, GB/s): the streaming
    rate HBM actually reaches, beside the 8 TB/s specification. lib_copy: the library's
    lema_device_copy (consecutive workgroups on consecutive 32 KB regions), else torch's.
    cold: each copy timed after evict_caches (median of COLD_REPS)."""
    import torch
    from latest_exact_match_attention_amd import _lib
    nbytes = src.numel() * src.element_size()

    def run():
        if lib_copy:
            _lib.check(_lib.lib().lema_device_copy(src.data_ptr(), dst.data_ptr(), nbytes,
                                                   stream.cuda_stream))
        else:
            dst.copy_(src)
    if cold:
        return 2 * nbytes / (cold_ms(run, stream) * 1e-3) / 1e9
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    times.sort()
    return 2 * src.numel() * src.element_size() / (times[len(times) // 2] * 1e-3) / 1e9


DECODE_BYTES_PER_ITEM = 8 + 8 + 48 + 48 + 64 + 2 * 64   # codes, value in/out, 3 slot touches


def bench_decode(a):
    """Batched decode steps against the HBM store, hipGraph-captured, vs the reference store
    on the host (same inputs, outputs compared bit for bit)."""
    import math
    import numpy as np
    import torch
    from latest_exact_match_attention_amd import build
    from latest_exact_match_attention_amd.cache import HashStore

    from latest_exact_match_attention_amd import _lib
    if a.step_stamps:
        if not build.STAMPS_LIB.exists():
            build.build(stamps=True)
        L_st = _lib.use_stamps_library()
    elif not build.LIB.exists():
        build.build()
    seqs, heads, dv = 16, 64, 24
    P, n0, steps = seqs * heads, a.decode_prefill, a.decode_steps
    max_load = 0.5
    cap = math.ceil(P * (n0 + steps) / max_load)
    vbytes = dv * 2
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(0)
    store = HashStore(dv, groups=P, dtype=torch.bfloat16, capacity=cap, device=dev,
                      place=a.decode_place)
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
    stamps = None
    if a.step_stamps:
        stamps = torch.zeros((steps, P, 5), dtype=torch.int64, device=dev)
        L_st.lema_debug_step_stamps(stamps.data_ptr())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for s_ in range(steps):
            store.exchange(qc[s_], kc[s_], vv[s_], out[s_], 1, 0, check=False)
    if a.step_stamps:
        L_st.lema_debug_step_stamps(None)
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
    breakdown = step_breakdown(stamps, L_st, P, steps, stream) if a.step_stamps else None

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
               "kind": "reference", "cpu_model": cpu_model(),
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
                   "table_place": a.decode_place,
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
        **({"step_stamps": breakdown} if breakdown is not None else {}),
    }


def step_breakdown(stamps, L, P: int, steps: int, stream) -> dict:
    """Phases of the decode steps from the diagnostics build's clock readings (100 MHz, per
    item: start, codes loaded, first windows read, claim done, value and count written), and
    the per-step cost of a graph of empty kernels with the same grid."""
    import numpy as np
    import torch
    d = stamps.cpu().numpy()
    t = [d[..., k].astype(np.int64) for k in range(5)]
    start, end = t[0].min(1), t[4].max(1)
    us = lambda x: float(x) / 100.0

    def med_p99(x):
        return [us(np.median(x)), us(np.percentile(x, 99))]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(steps):
            _lib_check(L.lema_debug_empty_step(P, torch.cuda.current_stream().cuda_stream))
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return {
        "clock": "s_memrealtime, 100 MHz; each reading after the item's memory operations so far",
        "empty_graph_node_us": e0.elapsed_time(e1) / steps * 1e3,
        "step_period_us_median": us(np.median(start[1:] - start[:-1])),
        "step_span_us_median": us(np.median(end - start)),
        "between_steps_us_median": us(np.median(start[1:] - end[:-1])),
        "item_start_spread_us_median": us(np.median(t[0].max(1) - t[0].min(1))),
        "codes_us": med_p99(t[1] - t[0]),
        "windows_us": med_p99(t[2] - t[1]),
        "claim_us": med_p99(t[3] - t[2]),
        "stores_us": med_p99(t[4] - t[3]),
        "item_total_us": med_p99(t[4] - t[0]),
    }


def _lib_check(status: int) -> None:
    from latest_exact_match_attention_amd import _lib
    _lib.check(status)


def lm_flops_per_token(cfg) -> float:
    """Matrix-multiply FLOPs of one token's forward: q, k, v, o, gate, up, down per layer and
    the head (2 FLOPs per multiply-add)."""
    d, ff, H = cfg.dim, cfg.dim_ff, cfg.num_heads
    per_layer = 2 * d * H * (2 * cfg.d_qk + cfg.d_v) + 2 * H * cfg.d_v * d + 6 * d * ff
    return cfg.depth * per_layer + 2 * d * cfg.vocab_size


def cpu_baseline_lm(model, cfg, tokens: int):
    """The forward restated in torch with the reference's sort-based exact op
    (oracle/torch_model.py), fp32 on the host's cores, batch 1 x `tokens`."""
    import torch
    from oracle import torch_model
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    sd = {k: v.float().cpu() for k, v in model.state_dict().items()}
    g = torch.Generator().manual_seed(1)
    tok = torch.randint(0, 50304, (1, tokens + 1), generator=g)
    x, y = tok[:, :-1], tok[:, 1:]
    times = []
    with torch.no_grad():
        torch_model.loss(sd, cfg, x, y)
        t_end = time.perf_counter() + 20.0
        while len(times) < 5 and (time.perf_counter() < t_end or len(times) < 2):
            t0 = time.perf_counter()
            torch_model.loss(sd, cfg, x, y)
            times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": tokens / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"batch 1 x {tokens} tokens of the same model (fp32 weights), forward + "
                      f"loss; median of {len(times)} runs, {med:.2f} s per run; per-token "
                      f"cost grows with T only through the exact op's sort"}


def bench_lm(a):
    import torch
    from latest_exact_match_attention_amd import build, pack_codes
    from latest_exact_match_attention_amd.attention import launch_hard
    from latest_exact_match_attention_amd.model import (ModelConfig, Transformer, lm_loss,
                                                        project_qk_prefill)

    if not build.LIB.exists():
        build.build()
    cfg = ModelConfig(**LM_CONFIG)
    B, T = a.lm_batch, a.lm_seq
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Transformer(cfg)
    finally:
        torch.set_default_dtype(prev)
    model.eval().requires_grad_(False)
    model.set_hard(True)
    g = torch.Generator().manual_seed(0)
    tok = torch.randint(0, 50304, (B, T + 1), generator=g).to(dev)
    x, y = tok[:, :-1], tok[:, 1:]
    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        for _ in range(a.warmup):
            loss = lm_loss(model, x, y)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(a.steps):
            loss = lm_loss(model, x, y)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / a.steps
        # the fused exact op alone at the layer shape (layer 0's codes and values)
        blk = model.blocks[0]
        zq, zk, v = blk.attn.project(blk.norm1(model.tok_emb(x)))
        qc = pack_codes(zq, torch.int32).view(B * cfg.num_heads, T)
        kc = pack_codes(zk, torch.int32).view(B * cfg.num_heads, T)
        yv = torch.empty_like(v)
        for _ in range(3):
            launch_hard(qc, kc, v, yv)
        torch.cuda.synchronize()
        n_l = 20
        e0.record(stream)
        for _ in range(n_l):
            launch_hard(qc, kc, v, yv)
        e1.record(stream)
        torch.cuda.synchronize()
        ms_l = e0.elapsed_time(e1) / n_l
        ms_lc = cold_ms(lambda: launch_hard(qc, kc, v, yv), stream)
        # the same op into a head-contiguous y [B, H, T, d_v]: every 128-byte line of y is then
        # written by one workgroup, where the model's interleaved y (the o_proj input) has each
        # line assembled in L2 from 48-byte pieces of 8 workgroups
        yc = torch.empty((B, cfg.num_heads, T, cfg.d_v), dtype=v.dtype, device=dev)
        launch_hard(qc, kc, v, yc)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n_l):
            launch_hard(qc, kc, v, yc)
        e1.record(stream)
        torch.cuda.synchronize()
        ms_lcont = e0.elapsed_time(e1) / n_l
        ms_lcont_cold = cold_ms(lambda: launch_hard(qc, kc, v, yc), stream)
        del yc
        src = torch.empty((B, cfg.num_heads, T), dtype=torch.int32, device=dev)
        launch_hard(qc, kc, v, yv, src)
        hits = float((src >= 0).float().mean())
        # the sign-pack alone on the layer's query pre-activations (transposed view, bf16)
        e0.record(stream)
        for _ in range(n_l):
            pack_codes(zq, torch.int32)
        e1.record(stream)
        torch.cuda.synchronize()
        ms_p = e0.elapsed_time(e1) / n_l
        # one layer's q and k codes: both projections straight to codes in one launch (the
        # model's FUSED_QK_PACK, off), against the library path the forward takes (two
        # hipBLASLt GEMMs writing zq and zk, two packs)
        hn = blk.norm1(model.tok_emb(x))
        at = blk.attn

        def unfused_qk():
            a_, b_, _ = hn.shape
            zq_ = at.q_proj(hn).view(a_, b_, cfg.num_heads, cfg.d_qk).transpose(1, 2)
            zk_ = at.k_proj(hn).view(a_, b_, cfg.num_heads, cfg.d_qk).transpose(1, 2)
            return pack_codes(zq_, torch.int32), pack_codes(zk_, torch.int32)

        fused_qk = lambda: project_qk_prefill(hn, at, torch.int32)
        fq, fk = fused_qk()
        uq, uk = unfused_qk()
        qk_same = bool(torch.equal(fq, uq) and torch.equal(fk, uk))
        del uq, uk
        # three rounds, the two paths alternating, medians (a path's first round after the
        # other reads slow while the clocks settle)
        rounds = {"fused": [], "library": []}
        for _ in range(3):
            for name, fn in (("fused", fused_qk), ("library", unfused_qk)):
                for _ in range(3):
                    fn()
                torch.cuda.synchronize()
                e0.record(stream)
                for _ in range(n_l):
                    fn()
                e1.record(stream)
                torch.cuda.synchronize()
                rounds[name].append(e0.elapsed_time(e1) / n_l)
        ms_qk = {k: sorted(v)[1] for k, v in rounds.items()}
    ntok = B * T
    flops = lm_flops_per_token(cfg) * ntok
    tflops = flops / (ms * 1e-3) / 1e12
    nq = B * cfg.num_heads * T
    bpq = 4 + 4 + 4 + 2 * 2 * cfg.d_v
    gbs = bpq * nq / (ms_l * 1e-3) / 1e9
    cpu = None if a.no_cpu_baseline else cpu_baseline_lm(model, cfg, a.lm_cpu_tokens)
    return {
        "metric": "prefill matched queries/sec @T=16k; decode steps/sec; % of HBM peak",
        "value": ntok / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 (GEMMs fp32-accumulated), int32 codes",
        "data": "synthetic (uniform token ids, seed 0; random-init weights, seed 0)",
        "config": {"workload": "lm_forward", "model": cfg.summary(), "vocab": cfg.vocab_size,
                   "global_batch": B, "seq_len": T, "loss": float(loss),
                   "layer0_hit_rate": round(hits, 4), "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": tflops / MFMA_BF16_PEAK_TFLOPS,
                     "traffic": None, "kernel": "whole forward (GEMM FLOPs / step time)",
                     "flops_per_token": lm_flops_per_token(cfg)},
        "lema_kernel": {"kernel": "resolve_lag_kernel (fused resolve + gather), one layer",
                        "us": ms_l * 1e3, "queries": nq, "bytes_per_query": bpq,
                        "achieved_gbs": gbs, "frac": gbs / HBM_PEAK_GBS,
                        "us_cold_cache": ms_lc * 1e3,
                        "frac_cold_cache": bpq * nq / (ms_lc * 1e-3) / 1e9 / HBM_PEAK_GBS,
                        "y_layout": "interleaved [B, T, H*d_v] (the o_proj input)",
                        "contiguous_y": {
                            "y_layout": "head-contiguous [B, H, T, d_v]",
                            "us": ms_lcont * 1e3,
                            "frac": bpq * nq / (ms_lcont * 1e-3) / 1e9 / HBM_PEAK_GBS,
                            "us_cold_cache": ms_lcont_cold * 1e3,
                            "frac_cold_cache": bpq * nq / (ms_lcont_cold * 1e-3) / 1e9
                                               / HBM_PEAK_GBS}},
        "qk_pack_kernel": {
            "kernel": "qk_pack_kernel (q and k projections straight to codes), one layer",
            "us": ms_qk["fused"] * 1e3,
            "tflops": 2 * B * T * 2 * cfg.dim * cfg.dim / (ms_qk["fused"] * 1e-3) / 1e12,
            "frac": 2 * B * T * 2 * cfg.dim * cfg.dim / (ms_qk["fused"] * 1e-3) / 1e12
                    / MFMA_BF16_PEAK_TFLOPS,
            "library_path_us": ms_qk["library"] * 1e3,
            "rounds_us": {k: [round(x * 1e3, 1) for x in v] for k, v in rounds.items()},
            "library_path": "two hipBLASLt GEMMs (zq, zk to HBM) and two pack_tile_kernel",
            "codes_identical": qk_same},
        "pack_kernel": {"kernel": "pack_tile_kernel, one layer's query codes",
                        "us": ms_p * 1e3, "rows": nq, "bytes_per_row": 2 * cfg.d_qk + 4,
                        "achieved_gbs": (2 * cfg.d_qk + 4) * nq / (ms_p * 1e-3) / 1e9,
                        "frac": (2 * cfg.d_qk + 4) * nq / (ms_p * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "cpu_baseline": cpu,
    }


def bench_long(a):
    import math
    import torch
    from latest_exact_match_attention_amd import build
    from latest_exact_match_attention_amd.cache import HashStore
    from latest_exact_match_attention_amd.workloads import LONG_CONTEXT, long_context_codes

    if not build.LIB.exists():
        build.build()
    H, T, L, dv = LONG_CONTEXT["H"], LONG_CONTEXT["T"], LONG_CONTEXT["call"], LONG_CONTEXT["dv"]
    calls = max(1, min(a.long_calls, T // L))
    dev = torch.device("cuda", 0)
    cap = math.ceil(H * T / 0.5)
    store = HashStore(dv, groups=H, dtype=torch.bfloat16, capacity=cap, device=dev)
    ref = None
    n_par = 0 if a.no_cpu_baseline else max(0, min(a.long_parity_calls, calls))
    if n_par:
        import oracle
        ref = oracle.ref_store()
        if ref is None:
            print("oracle/_ref/lema_store_ref.so missing: no CPU baseline", file=sys.stderr)
            n_par = 0
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    if n_par:
        cap_h = math.ceil(H * L * n_par / 0.5)
        host_table = torch.zeros((cap_h, 16 + 2 * dv), dtype=torch.uint8)
        host_counts = torch.zeros(H, dtype=torch.int64)
    stream = torch.cuda.current_stream(dev)
    if a.copy_probe:                     # one plain copy of 256 MiB: calibrates the counters
        probe = torch.zeros(128 << 20, dtype=torch.int16, device=dev)
        torch.empty_like(probe).copy_(probe)
        torch.cuda.synchronize()
        del probe
    total_ms, per_call, cpu_s, same, counts_same = 0.0, [], [], True, True
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # Every value row's first 8 bytes name its key, (head << 32) | (position + 1), so each
    # returned row says which key it came from (0: a miss); the rows stay opaque to the store.
    full = not a.no_full_parity
    if full:
        qc_all = torch.empty((H, L * calls), dtype=torch.int64, device=dev)
        kc_all = torch.empty_like(qc_all)
        got_all = torch.empty_like(qc_all)
    head = torch.arange(H, dtype=torch.int64, device=dev).view(H, 1)
    # untimed warm-up: the first call's inputs through a separate store sized for one call,
    # which loads the kernels and leaves a workspace of the call's size in torch's allocator;
    # the timed calls then start on the workload's own fresh table
    wq, wk = long_context_codes(0, H, 0, L, dev)
    warm = HashStore(dv, groups=H, dtype=torch.bfloat16, capacity=math.ceil(H * L / 0.5),
                     device=dev)
    wv = torch.zeros((H * L, dv), dtype=torch.bfloat16, device=dev)
    warm.exchange(wq.to(torch.int32).view(-1), wk.to(torch.int32).view(-1), wv,
                  torch.empty_like(wv), L, 0)
    del warm, wq, wk, wv
    torch.cuda.synchronize()
    for c in range(calls):
        qc64, kc64 = long_context_codes(0, H, c * L, (c + 1) * L, dev)
        qc, kc = qc64.to(torch.int32).contiguous(), kc64.to(torch.int32).contiguous()
        g = torch.Generator(device=dev).manual_seed(1000 + c)
        v = torch.randn((H * L, dv), device=dev, generator=g).to(torch.bfloat16)
        pos = torch.arange(c * L, (c + 1) * L, dtype=torch.int64, device=dev).view(1, L)
        v.view(torch.int64).view(H, L, dv // 4)[:, :, 0] = (head << 32) | (pos + 1)
        out = torch.empty_like(v)
        torch.cuda.synchronize()
        e0.record(stream)
        store.exchange(qc.view(-1), kc.view(-1), v, out, L, 0, check=False)
        e1.record(stream)
        torch.cuda.synchronize()
        store.check_full()
        ms = e0.elapsed_time(e1)
        total_ms += ms
        per_call.append(round(ms, 3))
        print(f"long_context call {c + 1}/{calls}: {ms:.2f} ms", file=sys.stderr, flush=True)
        if full:
            qc_all[:, c * L:(c + 1) * L] = qc64
            kc_all[:, c * L:(c + 1) * L] = kc64
            got_all[:, c * L:(c + 1) * L] = out.view(torch.int64).view(H, L, dv // 4)[:, :, 0]
        if c < n_par:
            qh, kh = qc64.view(-1).cpu(), kc64.view(-1).cpu()
            vh = v.view(torch.int16).cpu()
            oh = torch.empty_like(vh)
            t0 = time.perf_counter()
            host_counts += ref.exchange(host_table, qh, kh, vh, oh, L, 0, cap_h, 2 * dv)
            cpu_s.append(time.perf_counter() - t0)
            same = same and bool(torch.equal(out.view(torch.int16).cpu(), oh))
            counts_same = counts_same and bool(torch.equal(store.counts, host_counts))
            print(f"  reference store: {cpu_s[-1]:.2f} s, outputs identical: {same}, "
                  f"counts identical: {counts_same}", file=sys.stderr, flush=True)
        del qc64, kc64, qc, kc, v, out
    full_par = None
    if full:
        # after the timed calls: per head, the reference's sort-based algorithm over every
        # position of the run (oracle/torch_port.py, on the device) names each query's key
        from oracle.torch_port import latest_prev_match_sorted
        bad, hits, counts_ok = 0, 0, True
        for h in range(H):
            src = latest_prev_match_sorted(qc_all[h:h + 1], kc_all[h:h + 1])[0]
            want = torch.where(src >= 0, (h << 32) | (src + 1), torch.zeros_like(src))
            bad += int((got_all[h] != want).sum())
            hits += int((src >= 0).sum())
            counts_ok = counts_ok and int(store.counts[h]) == torch.unique(kc_all[h]).numel()
        full_par = {"calls_checked": calls, "queries_checked": H * L * calls,
                    "queries_differing": bad, "counts_equal_distinct_keys": counts_ok,
                    "hit_rate": round(hits / (H * L * calls), 4),
                    "oracle": "sort-based latest match over all positions per head "
                              "(code/lema/attention.py:100-132), on the device"}
        print(f"long_context: all {calls} calls against the sort-based oracle: {bad} of "
              f"{H * L * calls} queries differ, counts equal distinct keys: {counts_ok}",
              file=sys.stderr, flush=True)
        if bad or not counts_ok:
            print("long_context full-run parity FAILED", file=sys.stderr)
        del qc_all, kc_all, got_all
    nq = H * L * calls
    bpq = 4 + 4 + 4 + 2 * 2 * dv
    achieved = bpq * nq / (total_ms * 1e-3) / 1e9
    cpu = None
    parity = None
    if n_par:
        parity = {"calls_checked": n_par, "outputs_identical": same,
                  "counts_identical_after_checked_calls": counts_same}
    if full_par is not None:
        parity = dict(parity or {}, reference_store_calls=n_par, all_calls=full_par)
        cpu = {"value": H * L * n_par / sum(cpu_s), "unit": "queries/s", "cores": threads,
               "kind": "reference", "cpu_model": cpu_model(),
               "sample": f"the first {n_par} call(s) of 64 x 2^20 positions through "
                         f"code/lema/csrc/store.cpp (compiled from source, OpenMP) on a host "
                         f"table of {cap_h} slots; {sum(cpu_s):.2f} s"}
        if not (same and counts_same):
            print("long_context parity FAILED", file=sys.stderr)
    return {
        "metric": "prefill matched queries/sec @T=16k; decode steps/sec; % of HBM peak",
        "value": nq / (total_ms * 1e-3),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": calls,
        "warmup": 1,
        "ms_per_step": total_ms / calls,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32 codes (32-bit), bf16 values (opaque 48-byte rows)",
        "data": "synthetic (counter-based hash codes, seed 0; per-call seeded N(0,1) values, "
                "each row's first 8 bytes naming its key)",
        "config": {"workload": "long_context", "B": 1, "H": H, "T": L * calls,
                   "positions_per_call": L, "calls": calls, "d_v": dv, "capacity": cap,
                   "table_bytes": cap * (16 + 2 * dv), "load_after": round(store.load(), 4),
                   "ms_per_call": per_call, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic("bulk_kernels/long_context"),
                     "kernel": "store exchange (all launches of a call)",
                     "bytes_per_query": bpq, "queries_per_call": H * L},
        "cpu_baseline": cpu,
        "parity": parity,
    }


def bench_decode_model(a):
    import math
    import torch
    from latest_exact_match_attention_amd import build
    from latest_exact_match_attention_amd.decode import decoder, worst_case_codes
    from latest_exact_match_attention_amd.model import ModelConfig, Transformer

    if not build.LIB.exists():
        build.build()
    cfg = ModelConfig(**(LM_CONFIG if a.dm_geometry == "lm" else REF08B_CONFIG))
    B, L, steps = a.dm_batch, a.dm_prompt, a.dm_steps
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Transformer(cfg)
    finally:
        torch.set_default_dtype(prev)
    model.eval().requires_grad_(False)
    model.set_hard(True)
    total = L + steps + a.warmup + 4
    cache = model.new_cache("hbm", max_cache_len=total, batch=B, max_load=0.7,
                            codes_hook=worst_case_codes(cfg.depth))
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 50304, (B, L), generator=g).to(dev)
    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        # the same prefill into a scratch cache first, so the timed one runs warm (its GEMM
        # shapes and store calls seen once)
        scratch = model.new_cache("hbm", max_cache_len=total, batch=B, max_load=0.7,
                                  codes_hook=worst_case_codes(cfg.depth))
        model(prompt[:, :-1], cache=scratch, return_logits=False)
        del scratch
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model(prompt[:, :-1], cache=cache, return_logits=False)
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        dec = decoder(model, cache, tok=prompt[:, -1:])
        for _ in range(a.warmup):
            dec.step(check=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            dec.step(check=False)
        e1.record(stream)
        torch.cuda.synchronize()
        cache.store.check_full()
    ms = e0.elapsed_time(e1) / steps
    P = cfg.depth * B * cfg.num_heads
    weight_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    store_bytes = P * DECODE_BYTES_PER_ITEM
    achieved = (weight_bytes + store_bytes) / (ms * 1e-3) / 1e9
    return {
        "metric": "prefill matched queries/sec @T=16k; decode steps/sec; % of HBM peak",
        "value": B / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": a.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 (GEMMs fp32-accumulated), int64 codes",
        "data": "synthetic (uniform prompt tokens; random-init weights; worst-case codes)",
        "config": {"workload": "decode_model", "model": cfg.summary(), "batch": B,
                   "prompt": L, "store_partitions": P, "store_slots": cache.store.cap,
                   "store_bytes": cache.nbytes(), "entries_after": cache.entries(),
                   "prefill_s": round(t_prefill, 3),
                   "prefill_tokens_per_s": round(B * (L - 1) / t_prefill, 1),
                   "graph": "one replay per token (all layers and their store exchanges)",
                   "parallelism": "single GPU",
                   **({"reference_published": REF08B_PUBLISHED}
                      if a.dm_geometry == "ref08b" else {})},
        "roofline": {"bound": "hbm (weights read once per step)", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": None, "kernel": "whole decode step",
                     "bytes_per_step": weight_bytes + store_bytes},
        "cpu_baseline": None,
    }


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (there is no multi-GPU path); got "
              f"--gpus {a.gpus}", file=sys.stderr)
        return 2
    runs = {"decode": bench_decode, "lm_forward": bench_lm, "long_context": bench_long,
            "decode_model": bench_decode_model, "zipf_prefill": bench_prefill}
    if a.workload != "all":
        print(json.dumps(runs[a.workload](a)), flush=True)
        return 0
    out = bench_prefill(a)
    print(f"zipf_prefill: {out['ms_per_step'] * 1e3:.1f} us/step, "
          f"{out['roofline']['frac']:.3f} of HBM peak", file=sys.stderr, flush=True)
    for name, steps, warmup in SUB_WORKLOADS:
        import torch
        torch.cuda.empty_cache()
        sub = argparse.Namespace(**vars(a))
        sub.workload = name
        if steps is not None:
            sub.steps, sub.warmup = steps, warmup
        rec = runs[name](sub)
        out[name] = {k: v for k, v in rec.items() if k not in SUB_DROP}
        print(f"{name}: {rec['value']:.4g} {rec['unit']}, {rec['ms_per_step']:.4g} ms/step",
              file=sys.stderr, flush=True)
    print(json.dumps(out), flush=True)
    return 0


# the workloads carried as sub-records of the default line: (name, steps, warm-up) with None
# keeping the workload's own step counts
SUB_WORKLOADS = (("decode", None, None), ("long_context", None, None), ("lm_forward", 3, 1))
SUB_DROP = ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline")


if __name__ == "__main__":
    sys.exit(main())
