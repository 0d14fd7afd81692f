#!/usr/bin/env python3
"""FP8 + Huffman sidecar -> BF16 decode throughput on one MI355X.

Headline workload (config 5): every linear weight of a Llama-3-8B-shaped
random-init model -- 32 layers x {q, k, v, o, gate, up, down} plus lm_head
128256x4096 -- as seeded N(0, 0.02^2) BF16, quantized per output channel to
FP8 e4m3, with its Huffman sidecar (max_len 7, 1024 substreams per bucket)
built by the GPU sidecar builder. A step is one pass that rebuilds all 225
BF16 weights from FP8 bytes + sidecar, in one launch of the batched decode
plan; every input is resident in HBM before the timed region starts.

The default run (``--workload all``) first measures the other configurations
as sub-results -- config 2 (one 8B layer), config 4 (that layer's decode next
to its BF16 GEMMs), config 3 (one 70B layer with outliers and ESC codes) and
the AWQ int4 by-scale 8B layer -- then times the headline, then runs the CPU
baselines. Single workloads (``--workload model8b`` ...) print their own
line; the profiling commands in profiles/ use them.

Output: one JSON line on stdout (progress goes to stderr). ``value`` is the
BF16 bytes written per second (GB/s) over the timed steps; ``roofline``
prices the decode kernel's algorithmic bytes per launch (FP8 bytes, bitstream,
LUTs, bucket metadata, BF16 output) against MI355X's 8 TB/s HBM peak, with the
kernel's duration taken from HIP events on the launch stream; ``cpu_baseline``
is the CPU restatement of the same decode (the parity oracle's decoder),
multi-threaded on this host's cores and on one thread, over a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "BF16 decompress GB/s (out) + % HBM peak; full 8B-model FP8→BF16 ms"
PROFILES = os.path.join(ROOT, "profiles")
# committed rocprofv3 FETCH_SIZE/WRITE_SIZE summaries that price each workload's launch
TRAFFIC = {
    "model8b": "fp8_decode_model8b_traffic.md",
    "layer8b": "fp8_decode_layer8b_traffic.md",
    "layer70b": "fp8_decode_layer70b_traffic.md",
    "awq8b_by_scale": "awq_decode_layer8b.md",
    "awq8b_row_buckets": "awq_decode_layer8b.md",
}

WORKLOADS = {
    "model8b": "cfg5: Llama-3-8B-shaped full model, 32 layers x 7 linears + lm_head 128256x4096",
    "layer8b": "cfg2: one Llama-3-8B layer, 7 linears",
    "layer70b": "cfg3: one Llama-3-70B layer, 7 linears, sigma 0.015 with 0.1% outliers at +-8 sigma",
    "gemm8b": "cfg4: one Llama-3-8B layer decoded into preallocated scratch + BF16 GEMMs, T in {1,16,128,1024}",
    "awq8b": "AWQ int4 (group 128, zero point 8) one Llama-3-8B layer, max_len 11: by-scale sidecar "
             "(group buckets) and row-bucket sidecar (per-row scales)",
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    # A new plan's first launch takes about twice the steady time and the next
    # three up to 10% longer; from the fifth on the launch time holds to about
    # 0.1% at a level the buffers' placement sets.
    p.add_argument("--warmup", type=int, default=300)
    p.add_argument("--workload", choices=("all", "model8b", "layer8b", "layer70b", "gemm8b", "awq8b"), default="all",
                   help="all: the headline (config 5) with configs 2, 3, 4 and the AWQ layer as sub-results; "
                        "model8b: the headline alone; layer8b: config 2; layer70b: config 3; gemm8b: config 4; "
                        "awq8b: AWQ int4 decode of one 8B layer, both layouts")
    p.add_argument("--awq-k", type=int, default=1024,
                   help="substreams per bucket of the AWQ sidecars (the reference builders default to 256)")
    p.add_argument("--awq-layout", choices=("by_scale", "row_buckets"), default="by_scale",
                   help="--compare-libs --workload awq8b: the sidecar layout whose layer plan is timed")
    p.add_argument("--fp8-k", type=int, default=1024,
                   help="--compare-libs on an FP8 workload: substreams per bucket of its sidecars (the headline uses "
                        "1024; the reference's compress script defaults to 1024, its builder to 256)")
    p.add_argument("--cpu-seconds", type=float, default=8.0, help="time budget of each multi-threaded CPU sample")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="CPU baseline threads (0: the CPUs this process may run on, capped by OMP_NUM_THREADS)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-verify", action="store_true", help="skip the bit-exact check of the outputs")
    p.add_argument("--no-per-tensor", action="store_true",
                   help="layer workloads: skip the per-tensor timings (profiling runs that count one launch kind)")
    p.add_argument("--compare-libs", nargs="+", default=None, metavar="LIB",
                   help="instead of the benchmark: time the decode plan of --workload (model8b by default; awq8b: the "
                        "AWQ by-scale layer) with each "
                        "of these libmpserve_amd builds (python -m mpserve_amd.build --define ... --out LIB) in this "
                        "one process, launches interleaved in rounds; prints one JSON line of medians")
    p.add_argument("--compare-rounds", type=int, default=6, help="--compare-libs: rounds (20 launches per library each)")
    p.add_argument("--vram-pretouch-gib", type=int, default=48, metavar="GIB",
                   help="before anything else, allocate, fill and free this much device memory (0: skip); on a "
                        "fresh box the decode of buffers placed on never-used memory runs about 6%% slower")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="after the timed steps, run 3 plain int32 elementwise copies of MIB MiB each "
                        "(reference kernel of known bytes for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args(argv)


# --------------------------------------------------------------------------- bytes
def algorithmic_bytes(n: int, m: int, sc) -> int:
    """Bytes a decode of one tensor must move: FP8 bytes + bitstream + LUTs +
    bucket metadata read, BF16 written."""
    N = n * m
    W = sc["bitstream_u64"].numel()
    G = sc["decode_syms_u16"].shape[0]
    B = sc["bucket_table_i32"].shape[0]
    k = sc["bucket_thread_startbit_u32"].shape[1] - 1
    R = sc["row_indices_i32"].numel()
    return N + 8 * W + 320 * G + B * (1024 + 4 * (k + 1) + 8 + 4 + 8) + 8 + 4 + 4 * R + 2 * N


def awq_algorithmic_bytes(n: int, m: int, sc) -> int:
    """Bytes one AWQ int4 decode must move: int4 bytes + bitstream + each table
    once (2048 u16 symbols + 1024 length bytes) + bucket and row/group metadata
    read, BF16 written."""
    N = n * m
    B = sc["bucket_table_i32"].shape[0]
    k = sc["bucket_thread_startbit_u32"].shape[1] - 1
    meta = B * (16 * 4 + 4 * (k + 1) + 8 + 4)
    if "group_rows_i32" in sc:
        meta += 8 * sc["group_rows_i32"].numel()
    else:
        meta += B * 8 + 4 * sc["row_indices_i32"].numel()
    return N + 8 * sc["bitstream_u64"].numel() + 5120 * sc["decode_syms_u16"].shape[0] + meta + 2 * N


# builder outputs the compress script does not persist (bucket_U/unique_gid/fp8_uidx)
_NOT_STORED = ("bucket_U_i32", "bucket_unique_gid_i32", "bucket_fp8_uidx_i16")


def sidecar_bytes(sc) -> int:
    """Bytes of the sidecar tensors a checkpoint stores next to the FP8 bytes."""
    return sum(t.numel() * t.element_size() for k, t in sc.items() if k not in _NOT_STORED)


def read_traffic(key: str):
    """HBM bytes per decode launch from a committed rocprofv3 PMC summary, if one covers this workload."""
    path = os.path.join(PROFILES, TRAFFIC.get(key, ""))
    try:
        text = open(path).read()
    except OSError:
        return None, None
    m = re.search(r"^traffic_bytes_per_launch\[%s\]\s*=\s*([0-9.eE+]+)" % re.escape(key), text, re.M)
    if not m:
        return None, None
    return float(m.group(1)), os.path.relpath(path, ROOT)


def roofline(alg: int, kernel_ms: float, traffic_key: str) -> dict:
    achieved = alg / (kernel_ms * 1e-3) / 1e9
    traffic, src = read_traffic(traffic_key)
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "algorithmic_bytes": int(alg),
            "kernel_ms": round(kernel_ms, 4), "traffic_source": src}


# --------------------------------------------------------------------------- CPU baseline
def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpus_allowed() -> int:
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)


def cpu_threads(requested: int) -> int:
    """Threads of the multi-threaded baseline: the CPUs this process may run on,
    capped by OMP_NUM_THREADS (a GPU box sets it to its per-GPU CPU share)."""
    if requested > 0:
        return requested
    n = cpus_allowed()
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def _timed_sample(run, seconds: float):
    """Call run(i) (returns elements decoded) until ``seconds`` of its own time pass."""
    done, elapsed, calls = 0, 0.0, 0
    while elapsed < seconds or calls == 0:
        t0 = time.perf_counter()
        done += run(calls)
        elapsed += time.perf_counter() - t0
        calls += 1
    return done, elapsed, calls


def cpu_baseline(decode_one, items, what: str, seconds: float, threads: int) -> dict:
    """The oracle's decoder of the same sidecar format on ``threads`` threads
    and on one thread, cycling over ``items`` ((name, n, m, args) on the host)
    for about ``seconds`` (one thread: half that). ``decode_one(args, threads)``
    decodes one tensor and checks it bit-exact."""
    def run_with(t):
        def run(i):
            _, n, m, a = items[i % len(items)]
            decode_one(a, t)
            return n * m
        return run

    done, el, calls = _timed_sample(run_with(threads), seconds)
    done1, el1, calls1 = _timed_sample(run_with(1), seconds / 2)
    return {"value": round(2 * done / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{what}: {calls} tensor decodes ({done / 1e6:.1f} M elements, {2 * done / 1e9:.2f} GB BF16 "
                      f"out) in {el:.2f} s on {threads} threads",
            "one_thread": {"value": round(2 * done1 / el1 / 1e9, 3), "unit": "GB/s",
                           "sample": f"{calls1} tensor decodes ({done1 / 1e6:.1f} M elements) in {el1:.2f} s"},
            "cpu_model": cpu_model(), "cpu_count": os.cpu_count(), "cpus_allowed": cpus_allowed(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cfg1_cpu(threads: int) -> dict:
    """Config 1, the reference's CPU-runnable case: one 4096x4096 N(0, 0.02^2) BF16
    weight (seed 0, torch's CPU generator), per-channel FP8; the oracle's CPU encode,
    then its CPU decode on ``threads`` threads and on one, checked bit-exact."""
    import numpy as np
    import torch

    import oracle
    from mpserve_amd.synthetic import make_weight

    n = m = 4096
    w = make_weight(n, m, sigma=0.02, seed=0, device="cpu")
    bf = w.bf16.view(torch.uint16).numpy()
    q = w.fp8_u8.numpy()
    t0 = time.perf_counter()
    sc = oracle.encode(bf, q, w.scale_u16.numpy(), 7, 1024)
    enc_ms = (time.perf_counter() - t0) * 1e3
    dec = {}
    exact = True
    for t in (threads, 1):
        out = np.empty((n, m), dtype=np.uint16)
        t0 = time.perf_counter()
        oracle.decode(sc, q, n, m, 7, oracle.MODE_LOSSLESS, t, out)
        dec[t] = (time.perf_counter() - t0) * 1e3
        exact = exact and bool(np.array_equal(out, bf))
    side = sum(v.nbytes for k, v in sc.items() if k not in _NOT_STORED)
    return {"workload": "cfg1: one 4096x4096 weight, seed 0, sigma 0.02; CPU encode then CPU decode (no GPU)",
            "encode_ms": round(enc_ms, 1), "decode_ms": round(dec[threads], 1), "decode_threads": threads,
            "decode_ms_one_thread": round(dec[1], 1), "bit_exact": exact,
            "buckets": int(sc["bucket_table_i32"].shape[0]), "sidecar_over_bf16": round(side / (2 * n * m), 4),
            "implementation": "the parity oracle (oracle/fp8_huffman_oracle.c), the CPU restatement of the "
                              "reference's builder and decoder", "cpu_model": cpu_model()}


def fp8_host_sample(entries):
    """Host copies of FP8 entries for the CPU baseline: (name, n, m, decode args)."""
    import torch

    items = []
    for name, fp8, sc, src in entries:
        n, m = int(fp8.shape[0]), int(fp8.shape[1])
        items.append((name, n, m, (fp8.cpu().numpy(), {k: v.cpu().numpy() for k, v in sc.items()},
                                   src.view(torch.uint16).cpu().numpy(), n, m, name)))
    return items


def fp8_cpu_baseline(items, what: str, seconds: float, threads: int) -> dict:
    import numpy as np

    import oracle

    def decode_one(a, t):
        q, sc, ref, n, m, name = a
        out = np.empty((n, m), dtype=np.uint16)
        oracle.decode(sc, q, n, m, 7, oracle.MODE_LOSSLESS, t, out)
        if not np.array_equal(out, ref):
            raise RuntimeError(f"CPU baseline decode of {name} is not bit-exact")

    return cpu_baseline(decode_one, items, what, seconds, threads)


def awq_cpu_baseline(items, what: str, seconds: float, threads: int) -> dict:
    import numpy as np

    import oracle

    def decode_one(a, t):
        q, sc, ref, n, m, name = a
        if not np.array_equal(oracle.awq_decode(sc, q, n, m, nthreads=t), ref):
            raise RuntimeError(f"CPU baseline AWQ decode of {name} is not bit-exact")

    return cpu_baseline(decode_one, items, what, seconds, threads)


# --------------------------------------------------------------------------- GPU helpers
def timed_events(launch, stream, steps: int, warmup: int, flush=None) -> float:
    """Average ms per launch from HIP events around each launch on ``stream``;
    ``flush()``, when given, runs before each timed launch, outside its events."""
    import torch

    for _ in range(warmup):
        launch()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for s, e in ev:
        if flush is not None:
            flush()
        s.record(stream)
        launch()
        e.record(stream)
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in ev) / steps


_FLUSH_BUFS = {}


def cache_flush(dev, mib: int = 1024):
    """A callable that reads ``mib`` MiB on the current stream. A single tensor,
    or a layer, fits the 256 MB Infinity Cache and the L2s and would be read
    from them by back-to-back launches; the sub-results' timed launches each
    follow such a read, so that they read their inputs from HBM. A read, not a
    write: it leaves the caches holding clean lines, and the previous launch's
    dirty output lines are written back during it, so that no write-back of the
    flush itself lands inside the timed launch."""
    import torch

    if dev not in _FLUSH_BUFS:
        _FLUSH_BUFS[dev] = (torch.ones(mib << 18, dtype=torch.int32, device=dev),
                            torch.zeros((), dtype=torch.int64, device=dev))
    buf, acc = _FLUSH_BUFS[dev]

    def flush():
        torch.sum(buf, dim=0, dtype=torch.int64, out=acc)

    return flush


def build_fp8_entries(weights, dev, k=1024):
    """(name, fp8, sidecar, bf16 source) of each weight, built on the GPU with k substreams per bucket."""
    import torch

    from mpserve_amd.encode import build_fp8_sidecar
    from mpserve_amd.synthetic import make_weight

    t0 = time.perf_counter()
    entries = []
    for i, (name, n, m, seed, sigma, outlier_p) in enumerate(weights):
        w = make_weight(n, m, sigma=sigma, seed=seed, outlier_p=outlier_p, device=dev)
        sc = build_fp8_sidecar(w.bf16, w.fp8_u8, w.scale_u16, max_len=7, threads_per_block=k)
        entries.append((name, w.fp8_u8, sc, w.bf16))
        if i % 7 == 6 or i == len(weights) - 1:
            log(f"built {i + 1}/{len(weights)} ({time.perf_counter() - t0:.1f} s)")
    torch.cuda.synchronize()
    return entries, time.perf_counter() - t0


def check_outputs(entries, outs, what: str) -> None:
    import torch

    for (name, _, _, src), o in zip(entries, outs):
        if not torch.equal(o.view(torch.uint16), src.view(torch.uint16)):
            raise RuntimeError(f"{what}: decode of {name} is not bit-exact")


def esc_tables(entries) -> int:
    return sum(int(((sc["decode_lens_u8"] & 0x88) != 0).any(dim=1).sum().item()) for _, _, sc, _ in entries)


def time_per_tensor(entries, outs, stream, reps: int = 20):
    """Each tensor decoded alone, timed with events on its stream: through the
    drop-in op (from its second call on a sidecar it launches that sidecar's
    cached plan), through the op with that cache off (one launch over whole
    buckets, as the reference decodes), and through an explicit plan."""
    import torch

    import MPServe_cuda
    from mpserve_amd.decode import DecodePlan, sidecar_decode_args
    from mpserve_amd.mpserve_cuda import clear_decode_plans

    rows = []
    flush = cache_flush(outs[0].device) if outs else None
    for (name, fp8, sc, src), o in zip(entries, outs):
        n, m = int(fp8.shape[0]), int(fp8.shape[1])
        call = sidecar_decode_args(fp8, sc)
        alg = algorithmic_bytes(n, m, sc)
        row = {"tensor": name, "shape": [n, m], "buckets": int(sc["bucket_table_i32"].shape[0]),
               "esc_tables": int(((sc["decode_lens_u8"] & 0x88) != 0).any(dim=1).sum().item())}
        plan = DecodePlan([(fp8, sc, o)])
        row["plan_work_items"] = plan.info()["work_items"]

        def op_whole_buckets():
            os.environ["MPSERVE_DECODE_PLANS"] = "0"
            try:
                MPServe_cuda.huffman_decode_fp8(*call, out=o)
            finally:
                os.environ.pop("MPSERVE_DECODE_PLANS", None)

        for key, launch in (("op", lambda: MPServe_cuda.huffman_decode_fp8(*call, out=o)),
                            ("op_whole_buckets", op_whole_buckets),
                            ("plan", lambda: plan.decode(stream))):
            o.zero_()
            ms = timed_events(launch, stream, reps, 3, flush)
            if not torch.equal(o.view(torch.uint16), src.view(torch.uint16)):
                raise RuntimeError(f"per-tensor decode ({key}) of {name} is not bit-exact")
            row[f"{key}_ms"] = round(ms, 4)
            row[f"{key}_pct_hbm_peak_rw"] = round(100.0 * alg / ms / 1e6 / HBM_PEAK_GBS, 2)
        plan.close()
        rows.append(row)
        log(f"{name} {n}x{m}: op {row['op_ms']:.4f} ms ({row['op_pct_hbm_peak_rw']}%), whole buckets "
            f"{row['op_whole_buckets_ms']:.4f} ms, plan of {row['plan_work_items']} items {row['plan_ms']:.4f} ms")
    clear_decode_plans()
    return rows


def layer_result(key: str, entries, dev, args, per_tensor: bool = True) -> dict:
    """One layer's weights in one plan launch (configs 2 and 3), with per-tensor timings."""
    import torch

    from mpserve_amd.decode import DecodePlan

    stream = torch.cuda.current_stream(dev)
    outs = [torch.empty(src.shape, dtype=torch.bfloat16, device=dev) for _, _, _, src in entries]
    plan = DecodePlan((fp8, sc, o) for (_, fp8, sc, _), o in zip(entries, outs))
    alg = sum(algorithmic_bytes(int(f.shape[0]), int(f.shape[1]), sc) for _, f, sc, _ in entries)
    steps, warmup = max(20, args.steps // 2), max(20, args.warmup // 4)
    kernel_ms = timed_events(lambda: plan.decode(stream), stream, steps, warmup, cache_flush(dev))
    if not args.no_verify:
        check_outputs(entries, outs, key)
    if plan.read_status() != 0:
        raise RuntimeError(f"{key}: the decode flagged the sidecars")
    elems = sum(o.numel() for o in outs)
    res = {"workload": WORKLOADS[key], "steps": steps, "warmup": warmup, "kernel_ms": round(kernel_ms, 4),
           "out_gbs": round(2 * elems / kernel_ms / 1e6, 2), "elements": elems,
           "roofline": roofline(alg, kernel_ms, key), "plan_work_items": plan.info()["work_items"],
           "esc_tables": esc_tables(entries),
           "sidecar_over_bf16": round(sum(sidecar_bytes(sc) for _, _, sc, _ in entries) / (2 * elems), 4),
           # LDS per workgroup (the bucket's 256 expanded tables + the bitstream queues) and waves per CU
           "lds_occupancy": {"bytes_per_workgroup": plan.info()["lds_bytes"], "of_cu_lds": 163840,
                             "workgroups_per_cu": 1, "waves_per_cu": 16},
           "cpu_baseline": None}
    log(f"{key}: {kernel_ms:.4f} ms per layer launch, {100 * res['roofline']['frac']:.2f}% of 8 TB/s")
    plan.close()
    if per_tensor:
        res["per_tensor"] = time_per_tensor(entries, outs, stream)
    return res


def gemm_result(entries, dev) -> dict:
    """Config 4: per-layer latency of an 8B layer served from FP8 + sidecar. The
    layer's 7 weights are decoded (one plan launch) into preallocated BF16
    scratch, then its 7 BF16 GEMMs y = x W^T run for x [T, K], T in {1, 16, 128,
    1024}. Sequential: decode, then GEMMs, on one stream. Overlapped: a chain of
    8 layers in which layer i + 1's weights decode on a side stream (into the
    second of two scratch sets) while layer i's GEMMs run."""
    import torch
    import torch.nn.functional as F

    from mpserve_amd.decode import DecodePlan

    stream = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(dev)
    bufs = ([torch.empty(src.shape, dtype=torch.bfloat16, device=dev) for _, _, _, src in entries],
            [torch.empty(src.shape, dtype=torch.bfloat16, device=dev) for _, _, _, src in entries])
    plans = tuple(DecodePlan((fp8, sc, o) for (_, fp8, sc, _), o in zip(entries, b)) for b in bufs)
    for p in plans:
        p.decode(stream)
    torch.cuda.synchronize()
    for b in bufs:
        check_outputs(entries, b, "gemm8b scratch")
    chain = 8
    g = torch.Generator(device=dev).manual_seed(4)

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(reps):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps

    rows = []
    for T in (1, 16, 128, 1024):
        xs = [torch.randn((T, o.shape[1]), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
              for o in bufs[0]]

        def gemms(ws):
            for x, w in zip(xs, ws):
                F.linear(x, w)

        def sequential():
            plans[0].decode(stream)
            gemms(bufs[0])

        def overlapped():
            dec = [torch.cuda.Event(), torch.cuda.Event()]
            used = [torch.cuda.Event(), torch.cuda.Event()]
            side.wait_stream(stream)
            plans[0].decode(side)
            dec[0].record(side)
            for i in range(chain):
                b = i % 2
                if i + 1 < chain:
                    nb = (i + 1) % 2
                    if i >= 1:
                        side.wait_event(used[nb])  # layer i - 1's GEMMs are done with that scratch
                    plans[nb].decode(side)
                    dec[nb].record(side)
                stream.wait_event(dec[b])
                gemms(bufs[b])
                used[b].record(stream)
            stream.wait_stream(side)

        t_gemm = timed(lambda: gemms(bufs[0]), 50)
        t_dec = timed(lambda: plans[0].decode(stream), 50)
        t_seq = timed(sequential, 50)
        t_ovl = timed(overlapped, 10) / chain
        rows.append({"T": T, "gemm_ms": round(t_gemm, 4), "decode_ms": round(t_dec, 4),
                     "sequential_ms": round(t_seq, 4), "overlapped_ms": round(t_ovl, 4),
                     "decode_share_sequential": round((t_seq - t_gemm) / t_seq, 4),
                     "decode_share_overlapped": round(max(0.0, t_ovl - t_gemm) / t_ovl, 4)})
        log(f"gemm8b T={T}: GEMMs {t_gemm:.4f} ms, decode {t_dec:.4f} ms, sequential {t_seq:.4f} ms, "
            f"overlapped {t_ovl:.4f} ms per layer")
    for p in plans:
        if p.read_status() != 0:
            raise RuntimeError("gemm8b: the decode flagged the sidecars")
        p.close()
    share16 = [r for r in rows if r["T"] == 16][0]["decode_share_sequential"]
    return {"workload": WORKLOADS["gemm8b"], "metric": "decode share of the layer's latency (decode + 7 BF16 GEMMs)",
            "decode_share_T16_pct": round(100.0 * share16, 2), "overlap_chain_layers": chain, "results": rows}


def awq_result(dev, args, layouts=(("by_scale", 128), ("row_buckets", None))):
    """AWQ int4 decode: each weight of one 8B layer through the drop-in ops and
    one plan launch, per layout. Returns (result, host sample of the by-scale
    q/k/v/o weights for the CPU baseline)."""
    import torch

    from mpserve_amd import awq
    from mpserve_amd.synthetic import LLAMA3_8B_LAYER, make_awq_weight

    stream = torch.cuda.current_stream(dev)
    results = {}
    host = []
    for layout, group in layouts:
        items = []
        t0 = time.perf_counter()
        for j, (name, n, m) in enumerate(LLAMA3_8B_LAYER):
            w = make_awq_weight(n, m, group, seed=300 + j, device=dev)
            sc, st = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, args.awq_k, 1024, bool(group),
                                           with_stats=True)
            if group:
                call = lambda sc=sc, w=w, n=n, m=m, o=None: awq.huffman_decode_awq_int4_bucket_by_scale(  # noqa: E731
                    w.int4_u8, sc["bitstream_u64"], sc["decode_syms_u16"], sc["decode_lens_u8"],
                    sc["bucket_table_i32"], sc["bucket_group_offsets_i32"], sc["group_rows_i32"],
                    sc["group_col_start_i32"], sc["bucket_thread_startbit_u32"], sc["bucket_bit_base_i64"], n, m,
                    11, 128, out=o)
            else:
                call = lambda sc=sc, w=w, n=n, m=m, o=None: awq.huffman_decode_awq_int4_bucket(  # noqa: E731
                    w.int4_u8, sc["bitstream_u64"], sc["decode_syms_u16"], sc["decode_lens_u8"],
                    sc["bucket_table_i32"], sc["bucket_col_start_i32"], sc["bucket_col_len_i32"],
                    sc["bucket_row_offsets_i32"], sc["row_indices_i32"], sc["bucket_thread_startbit_u32"],
                    sc["bucket_bit_base_i64"], n, m, 11, out=o)
            out = torch.empty((n, m), dtype=torch.bfloat16, device=dev)
            items.append((name, n, m, w, sc, call, out, st))
            if group and j < 4:
                host.append((name, n, m, (w.int4_u8.cpu().numpy(), {k: v.cpu().numpy() for k, v in sc.items()},
                                          w.bf16.view(torch.uint16).cpu().numpy(), n, m, name)))
        log(f"awq {layout}: built 7 sidecars ({time.perf_counter() - t0:.1f} s)")
        per = []
        tot_alg = tot_ms = 0.0
        for name, n, m, w, sc, call, out, st in items:
            ms = timed_events(lambda: call(o=out), stream, max(10, args.steps // 5), 3, cache_flush(dev))
            exact = torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16))
            # only ESC collisions of the row-bucket builder (bare ESC codes) may differ
            if not exact and st["esc_collisions"] == 0:
                raise RuntimeError(f"AWQ decode ({layout}) of {name} is not bit-exact")
            alg = awq_algorithmic_bytes(n, m, sc)
            tot_alg += alg
            tot_ms += ms
            per.append({"tensor": name, "shape": [n, m], "buckets": int(sc["bucket_table_i32"].shape[0]),
                        "tables": int(sc["decode_syms_u16"].shape[0]),
                        "bitstream_bits_per_elem": round(64 * sc["bitstream_u64"].numel() / (n * m), 3),
                        "esc_keys": st["esc_keys"], "esc_collisions": st["esc_collisions"], "bit_exact": exact,
                        "ms": round(ms, 4), "pct_hbm_peak_rw": round(100 * alg / ms / 1e6 / HBM_PEAK_GBS, 2)})
        elems = sum(n * m for _, n, m, *_ in items)
        plan = awq.AwqDecodePlan([(w.int4_u8, sc, out) for _, _, _, w, sc, _, out, _ in items])
        steps, warmup = max(20, args.steps // 2), max(10, args.warmup // 10)
        plan_ms = timed_events(lambda: plan.decode(stream), stream, steps, warmup, cache_flush(dev))
        for name, _, _, w, _, _, out, st in items:
            if not torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16)) and st["esc_collisions"] == 0:
                raise RuntimeError(f"AWQ plan decode ({layout}) of {name} is not bit-exact")
        # A collided element is a bare ESC code that the decoder reads as ESC + 16 raw bits,
        # so its lane ends past the next lane's start: that (and only that) is expected then.
        from mpserve_amd._native import MPS_STATUS_DESYNC
        status = plan.read_status()
        allowed = MPS_STATUS_DESYNC if any(it[7]["esc_collisions"] for it in items) else 0
        if status & ~allowed:
            raise RuntimeError(f"AWQ plan decode ({layout}) flagged the sidecars (0x{status:x})")
        log(f"awq {layout} layer: {tot_ms:.4f} ms as 7 op launches, {plan_ms:.4f} ms as one plan launch "
            f"({plan.info()['work_items']} work items)")
        results[layout] = {"steps": steps, "warmup": warmup, "layer_ms_op_launches": round(tot_ms, 4),
                           "kernel_ms": round(plan_ms, 4), "out_gbs": round(2 * elems / plan_ms / 1e6, 2),
                           "elements": elems, "roofline": roofline(tot_alg, plan_ms, f"awq8b_{layout}"),
                           "plan_work_items": plan.info()["work_items"], "cpu_baseline": None, "per_tensor": per}
        plan.close()
    return {"workload": WORKLOADS["awq8b"], "threads_per_block": args.awq_k, "layouts": results}, host


# --------------------------------------------------------------------------- workloads
def headline(entries, dev, args, build_s: float):
    """Config 5: time the full-model plan launch. Returns (result line, plan)."""
    import torch

    from mpserve_amd.decode import DecodePlan

    outs = [torch.empty(src.shape, dtype=torch.bfloat16, device=dev) for _, _, _, src in entries]
    plan = DecodePlan((fp8, sc, o) for (_, fp8, sc, _), o in zip(entries, outs))
    elems = sum(o.numel() for o in outs)
    stream = torch.cuda.current_stream(dev)
    for _ in range(max(1, args.warmup)):
        plan.decode(stream)
    torch.cuda.synchronize()
    if not args.no_verify:
        check_outputs(entries, outs, "warm-up")
        log("warm-up outputs bit-exact")
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record(stream)
        plan.decode(stream)
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    log(f"{args.steps} steps: {ms_per_step:.3f} ms/step wall, {kernel_ms:.3f} ms per decode launch (events)")
    if not args.no_verify:
        check_outputs(entries, outs, "timed")
    if plan.read_status() != 0:
        raise RuntimeError("the model decode flagged the sidecars")
    alg = sum(algorithmic_bytes(int(f.shape[0]), int(f.shape[1]), sc) for _, f, sc, _ in entries)
    side = sum(sidecar_bytes(sc) for _, _, sc, _ in entries)
    value = 2 * elems / (ms_per_step * 1e-3) / 1e9
    rf = roofline(alg, kernel_ms, "model8b")
    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u16",
        "data": "synthetic: seeded N(0,0.02^2) BF16, per-channel FP8 e4m3, sidecar built on the GPU",
        "config": {
            "workload": WORKLOADS["model8b"], "tensors": len(entries), "elements": elems, "max_len": 7,
            "threads_per_block": 1024, "full_decode_ms": round(kernel_ms, 4),
            "pct_hbm_peak_out": round(100.0 * value / HBM_PEAK_GBS, 2),
            "pct_hbm_peak_rw": round(100.0 * rf["frac"], 2),
            "sidecar_over_bf16": round(side / (2 * elems), 4),
            "sidecar_plus_fp8_over_bf16": round((side + elems) / (2 * elems), 4),
            "build_s": round(build_s, 2), "vram_pretouch_gib": args.vram_pretouch_gib, "plan": plan.info(),
            "lds_occupancy": {"bytes_per_workgroup": plan.info()["lds_bytes"], "of_cu_lds": 163840,
                              "workgroups_per_cu": 1, "waves_per_cu": 16},
            "esc_tables": esc_tables(entries),
        },
        "roofline": rf,
        "cpu_baseline": None,
    }
    del outs
    return res, plan


def vram_pretouch(dev, gib: int) -> int:
    """Allocate, fill and free ``gib`` GiB of device memory, and return it to
    the driver. On a freshly assigned box, a process whose model sits on memory
    no earlier allocation used decodes at one level for its whole life (5.75 ms
    for the model); after this the same process measures 5.30-5.50 ms, as every
    later process on the box does without it. It runs before the inputs exist,
    outside every timed region. Returns the GiB it touched (0: skipped)."""
    import torch

    if gib <= 0:
        return 0
    t0 = time.perf_counter()
    try:
        buf = torch.empty(gib << 28, dtype=torch.int32, device=dev)
    except torch.cuda.OutOfMemoryError:
        log(f"VRAM pre-touch: {gib} GiB not available, skipped")
        return 0
    buf.fill_(0)
    torch.cuda.synchronize()
    del buf
    torch.cuda.empty_cache()
    log(f"VRAM pre-touch: {gib} GiB allocated, filled and freed ({time.perf_counter() - t0:.2f} s)")
    return gib


def copy_calibration(dev, mib: int) -> None:
    import torch

    n32 = mib * (1 << 20) // 4
    src32 = torch.ones(n32, dtype=torch.int32, device=dev)
    dst32 = torch.empty_like(src32)
    for _ in range(3):
        torch.bitwise_not(src32, out=dst32)
    torch.cuda.synchronize()
    log(f"copy calibration: 3 x bitwise_not over {mib} MiB int32 (reads and writes {n32 * 4} bytes each)")


def run_all(args, dev) -> int:
    """The headline (config 5) with configs 2, 3, 4 and the AWQ by-scale layer as sub-results."""
    import torch

    from mpserve_amd.synthetic import config_weights

    log(f"workload all: building the 8B model's 225 weights on {torch.cuda.get_device_name(dev)}")
    entries, build_s = build_fp8_entries(config_weights("model8b"), dev)
    layer0 = [e for e in entries if e[0].startswith("layers.0.")]  # config 2's layer (same seeds)
    sub = {}
    # The sub-results run first: they also keep the GPU busy ahead of the headline's warm-up.
    sub["cfg2_layer8b"] = layer_result("layer8b", layer0, dev, args)
    sub["cfg4_gemm8b"] = gemm_result(layer0, dev)
    log("building the 70B layer")
    e70, _ = build_fp8_entries(config_weights("layer70b"), dev)
    sub["cfg3_layer70b"] = layer_result("layer70b", e70, dev, args)
    host70 = fp8_host_sample([e for e in e70 if e[0].split(".")[-1] in ("q_proj", "k_proj", "v_proj")])
    del e70
    awq, awq_host = awq_result(dev, args, layouts=(("by_scale", 128),))
    sub["awq8b_by_scale"] = awq["layouts"]["by_scale"]
    sub["awq8b_by_scale"]["workload"] = "AWQ int4 (group 128, zero point 8) one Llama-3-8B layer, by-scale sidecar"
    torch.cuda.empty_cache()
    res, plan = headline(entries, dev, args, build_s)
    plan.close()
    if args.copy_calibration > 0:
        copy_calibration(dev, args.copy_calibration)
    if not args.no_cpu_baseline:
        threads = cpu_threads(args.cpu_threads)
        log(f"CPU baselines: oracle decoders on {threads} threads and on 1 thread")
        res["cpu_baseline"] = fp8_cpu_baseline(fp8_host_sample(layer0),
                                               "oracle decode of the 8B model's layer-0 weights",
                                               args.cpu_seconds, threads)
        # the config 2 layer is the model's layer 0: the same sample prices it
        sub["cfg2_layer8b"]["cpu_baseline"] = res["cpu_baseline"]
        sub["cfg3_layer70b"]["cpu_baseline"] = fp8_cpu_baseline(
            host70, "oracle decode of the 70B layer's q/k/v weights (ESC codes in q)", args.cpu_seconds, threads)
        sub["awq8b_by_scale"]["cpu_baseline"] = awq_cpu_baseline(
            awq_host, "oracle AWQ by-scale decode of the 8B layer's q/k/v/o weights", args.cpu_seconds, threads)
        log("config 1 on the CPU: oracle encode and decode of one 4096x4096 weight")
        sub["cfg1_cpu"] = cfg1_cpu(threads)
    res["subresults"] = sub
    print(json.dumps(res), flush=True)
    return 0


def run_single(args, dev) -> int:
    """One workload on its own line (the profiling commands in profiles/ use these)."""
    import torch

    from mpserve_amd.synthetic import config_weights

    threads = cpu_threads(args.cpu_threads)
    if args.workload == "awq8b":
        res, host = awq_result(dev, args)
        head = res["layouts"]["by_scale"]
        if not args.no_cpu_baseline:
            head["cpu_baseline"] = awq_cpu_baseline(
                host, "oracle AWQ by-scale decode of the 8B layer's q/k/v/o weights", args.cpu_seconds, threads)
        line = {"metric": "AWQ int4 -> BF16 decompress GB/s (out); one Llama-3-8B layer in one plan launch",
                "value": head["out_gbs"], "unit": "GB/s", "n_gpus": 1, "steps": head["steps"],
                "warmup": head["warmup"], "ms_per_step": head["kernel_ms"], "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "u16",
                "data": "synthetic: seeded N(0,0.02^2) BF16, AWQ-style int4 (group 128), sidecar built on the GPU",
                "config": res, "roofline": head["roofline"], "cpu_baseline": head["cpu_baseline"]}
        print(json.dumps(line), flush=True)
        return 0
    weights = config_weights("layer8b" if args.workload == "gemm8b" else args.workload)
    log(f"workload {args.workload}: {len(weights)} tensors, building inputs on {torch.cuda.get_device_name(dev)}")
    entries, build_s = build_fp8_entries(weights, dev)
    if args.workload == "model8b":
        res, plan = headline(entries, dev, args, build_s)
        plan.close()
        if args.copy_calibration > 0:
            copy_calibration(dev, args.copy_calibration)
        if not args.no_cpu_baseline:
            layer0 = [e for e in entries if e[0].startswith("layers.0.")]
            res["cpu_baseline"] = fp8_cpu_baseline(fp8_host_sample(layer0),
                                                   "oracle decode of the 8B model's layer-0 weights",
                                                   args.cpu_seconds, threads)
        print(json.dumps(res), flush=True)
        return 0
    if args.workload == "gemm8b":
        res = gemm_result(entries, dev)
        line = {"metric": "cfg4: decode share of an 8B layer's latency (decode + 7 BF16 GEMMs), T=16",
                "value": res["decode_share_T16_pct"], "unit": "%", "n_gpus": 1, "steps": 50, "warmup": 1,
                "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "u16+bf16",
                "data": "synthetic: seeded N(0,0.02^2) BF16, per-channel FP8 e4m3, sidecar built on the GPU",
                "config": res}
        print(json.dumps(line), flush=True)
        return 0
    res = layer_result(args.workload, entries, dev, args, per_tensor=not args.no_per_tensor)
    if args.copy_calibration > 0:
        copy_calibration(dev, args.copy_calibration)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = fp8_cpu_baseline(fp8_host_sample(entries[:3]),
                                               f"oracle decode of the {args.workload} q/k/v weights",
                                               args.cpu_seconds, threads)
    line = {"metric": f"{args.workload}: BF16 decompress GB/s (out), one layer in one plan launch",
            "value": res["out_gbs"], "unit": "GB/s", "n_gpus": 1, "steps": res["steps"], "warmup": res["warmup"],
            "ms_per_step": res["kernel_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "u16", "data": "synthetic: seeded BF16, per-channel FP8 e4m3, sidecar built on the GPU",
            "config": res, "roofline": res["roofline"], "cpu_baseline": res["cpu_baseline"]}
    print(json.dumps(line), flush=True)
    return 0


def compare_libs(args, dev) -> int:
    """Plan launch time of one workload with several builds of the library,
    measured in one process: the same inputs, one plan per library, 20 events-timed
    launches per library per round, the order reversed every other round. Box-to-box
    spread is several percent; within one process it is about 0.1%, which is what
    tuning the kernels' compile-time knobs needs. ``--workload awq8b`` compares the
    AWQ layer's plan (group 128, k = --awq-k, layout --awq-layout); otherwise an FP8
    workload's."""
    import ctypes
    import statistics

    import torch

    from mpserve_amd import _native
    from mpserve_amd.synthetic import config_weights

    stream = torch.cuda.current_stream(dev)
    h = ctypes.c_void_p(stream.cuda_stream)
    entries, outs, descs = [], [], []
    if args.workload == "awq8b":
        from mpserve_amd import awq
        from mpserve_amd.awq import _sidecar_descriptor
        from mpserve_amd.synthetic import make_awq_weight

        workload, kind, tensor_t = "awq8b", "awq", _native.MpsAwqTensor
        for j, (name, n, m, _, _, _) in enumerate(config_weights("layer8b")):
            by_scale = args.awq_layout == "by_scale"  # row buckets: one scale per row, as awq_result builds them
            w = make_awq_weight(n, m, 128 if by_scale else None, seed=300 + j, device=dev)
            sc = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, args.awq_k, 1024, by_scale)
            o = torch.empty((n, m), dtype=torch.bfloat16, device=dev)
            entries.append((name, w.int4_u8, sc, w.bf16))
            outs.append(o)
            descs.append(_sidecar_descriptor(w.int4_u8, sc, o))
    else:
        from mpserve_amd.decode import sidecar_decode_args
        from mpserve_amd.mpserve_cuda import _descriptor

        workload = "model8b" if args.workload in ("all", "gemm8b") else args.workload
        kind, tensor_t = "fp8", _native.MpsFp8Tensor
        entries, _ = build_fp8_entries(config_weights(workload), dev, args.fp8_k)
        outs = [torch.empty(src.shape, dtype=torch.bfloat16, device=dev) for _, _, _, src in entries]
        descs = [_descriptor(*sidecar_decode_args(f, sc)[:13], o) for (_, f, sc, _), o in zip(entries, outs)]
    arr = (tensor_t * len(descs))(*descs)
    libs, first_out = [], None
    for path in args.compare_libs:
        L = ctypes.CDLL(os.path.abspath(path))
        vp = ctypes.c_void_p
        create, decode, read_status, destroy = (getattr(L, f"mps_{kind}_plan_{x}")
                                                for x in ("create", "decode", "read_status", "destroy"))
        create.argtypes = [ctypes.POINTER(tensor_t), ctypes.c_int64, vp, ctypes.POINTER(vp)]
        decode.argtypes = [vp, vp]
        read_status.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_uint32)]
        destroy.argtypes = [vp]
        L.mps_last_error.restype = ctypes.c_char_p
        plan = vp()
        if create(arr, len(descs), h, ctypes.byref(plan)) != 0:
            raise RuntimeError(f"{path}: plan creation failed: {L.mps_last_error().decode()}")
        for o in outs:
            o.zero_()
        for _ in range(max(1, args.warmup // 3)):
            if decode(plan, h) != 0:
                raise RuntimeError(f"{path}: {L.mps_last_error().decode()}")
        st = ctypes.c_uint32(0)
        read_status(plan, h, ctypes.byref(st))
        exact = None if args.no_verify else all(
            torch.equal(o.view(torch.uint16), src.view(torch.uint16)) for o, (_, _, _, src) in zip(outs, entries))
        # Row-bucket AWQ sidecars with ESC collisions do not round-trip (in the
        # reference's format as here): every build must then give the first one's output.
        same = None
        if not args.no_verify:
            if first_out is None:
                first_out = [o.clone() for o in outs]
            same = all(torch.equal(o, f) for o, f in zip(outs, first_out))
        log(f"{path}: status {st.value}, bit-exact {exact}, same output as the first library {same}")
        libs.append({"path": path, "plan": plan, "decode": decode, "destroy": destroy, "status": st.value,
                     "bit_exact": exact, "same_as_first": same, "ms": []})
    for r in range(args.compare_rounds):
        for lib in (libs if r % 2 == 0 else libs[::-1]):
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
            for a, b in ev:
                a.record(stream)
                lib["decode"](lib["plan"], h)
                b.record(stream)
            torch.cuda.synchronize()
            lib["ms"].append(statistics.mean(a.elapsed_time(b) for a, b in ev))
        log(f"round {r}: " + " ".join(f"{x['ms'][-1]:.4f}" for x in libs))
    base = statistics.median(libs[0]["ms"])
    rows = []
    for lib in libs:
        med = statistics.median(lib["ms"])
        rows.append({"lib": lib["path"], "median_ms": round(med, 4), "vs_first": round(med / base - 1, 4),
                     "rounds_ms": [round(x, 4) for x in lib["ms"]], "status": lib["status"],
                     "bit_exact": lib["bit_exact"], "same_as_first": lib["same_as_first"]})
        lib["destroy"](lib["plan"])
    print(json.dumps({"metric": "plan launch ms per library build (one process, interleaved)",
                      "workload": WORKLOADS[workload], "device": torch.cuda.get_device_name(dev),
                      "arch": torch.cuda.get_device_properties(dev).gcnArchName, "libs": rows}), flush=True)
    return 0


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the FP8+Huffman decode shards by "
              "bucket with no exchange step, so there is no multi-GPU figure to report", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    args.vram_pretouch_gib = vram_pretouch(dev, args.vram_pretouch_gib)
    if args.compare_libs:
        return compare_libs(args, dev)
    if args.workload == "all":
        return run_all(args, dev)
    return run_single(args, dev)


if __name__ == "__main__":
    sys.exit(main())
