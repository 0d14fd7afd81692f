#!/usr/bin/env python3
"""FP8 + Huffman sidecar -> BF16 decode throughput on one MI355X.

Workload (default ``model8b``): every linear weight of a Llama-3-8B-shaped
random-init model -- 32 layers x {q, k, v, o, gate, up, down} plus lm_head
128256x4096 -- as seeded N(0, 0.02^2) BF16, quantized per output channel to
FP8 e4m3, with its Huffman sidecar (max_len 7, 1024 substreams per bucket)
built by the GPU sidecar builder. A step is one pass that rebuilds all 225
BF16 weights from FP8 bytes + sidecar, in one launch of the batched decode
plan; every input is resident in HBM before the timed region starts.

Output: one JSON line on stdout (progress goes to stderr). ``value`` is the
BF16 bytes written per second (GB/s) over the timed steps; ``roofline``
prices the decode kernel's algorithmic bytes per launch (FP8 bytes, bitstream,
LUTs, bucket metadata, BF16 output) against MI355X's 8 TB/s HBM peak, with the
kernel's duration taken from HIP events on the launch stream; ``cpu_baseline``
is the CPU restatement of the same decode, multi-threaded on this host's
cores, over a bounded sample (layer-0 weights, repeated up to a time budget).
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
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "fp8_decode_model8b_traffic.md")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    # The GPU reaches its steady clocks only after a few seconds of sustained
    # load: with 3 warm-up launches a fresh box measures the model decode ~4%
    # slower than after 1000 (about 6 s).
    p.add_argument("--warmup", type=int, default=1000)
    p.add_argument("--workload", choices=("model8b", "layer8b", "layer70b", "gemm8b", "awq8b"), default="model8b",
                   help="model8b: full Llama-3-8B-shaped model (the headline, config 5); layer8b: one 8B "
                        "layer (config 2); layer70b: one 70B layer with outliers and ESC codes (config 3); "
                        "gemm8b: decode share of an 8B layer's latency next to its BF16 GEMMs (config 4); "
                        "awq8b: AWQ int4 decode of one 8B layer, by-scale and row-bucket sidecars")
    p.add_argument("--awq-k", type=int, default=1024,
                   help="awq8b: substreams per bucket of the AWQ sidecars (the reference builders default to 256)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="time budget of the CPU baseline sample")
    p.add_argument("--cpu-threads", type=int, default=0, help="CPU baseline threads (0: min(16, cpu_count))")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-verify", action="store_true", help="skip the bit-exact check of the outputs")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="after the timed steps, run 3 plain int32 elementwise copies of MIB MiB each "
                        "(reference kernel of known bytes for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args(argv)


WORKLOADS = {
    "model8b": "cfg5: Llama-3-8B-shaped full model, 32 layers x 7 linears + lm_head 128256x4096",
    "layer8b": "cfg2: one Llama-3-8B layer, 7 linears",
    "layer70b": "cfg3: one Llama-3-70B layer, 7 linears, sigma 0.015 with 0.1% outliers at +-8 sigma",
    "gemm8b": "cfg4: one Llama-3-8B layer decoded into preallocated scratch + BF16 GEMMs, T in {1,16,128,1024}",
    "awq8b": "AWQ int4 (group 128, zero point 8) one Llama-3-8B layer, max_len 11, k 1024: by-scale sidecar "
             "(group buckets) and row-bucket sidecar (per-row scales)",
}


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


def run_awq(args, dev) -> int:
    """AWQ int4 decode: each weight of one 8B layer through the drop-in ops, per layout."""
    import numpy as np
    import torch

    import oracle
    from mpserve_amd import awq
    from mpserve_amd.synthetic import LLAMA3_8B_LAYER, make_awq_weight

    stream = torch.cuda.current_stream(dev)
    layouts = {}
    for layout, group in (("by_scale", 128), ("row_buckets", None)):
        items = []
        for j, (name, n, m) in enumerate(LLAMA3_8B_LAYER):
            w = make_awq_weight(n, m, group, seed=300 + j, device=dev)
            scales = w.scale_u16
            sc, st = awq.build_awq_sidecar(w.bf16, w.int4_u8, scales, 11, args.awq_k, 1024, bool(group),
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
        layouts[layout] = items
        log(f"{layout}: built 7 sidecars")

    def layer_step(items):
        for _, _, _, _, _, call, out, _ in items:
            call(o=out)

    results = {}
    for layout, items in layouts.items():
        for _ in range(max(1, args.warmup // 10)):
            layer_step(items)
        torch.cuda.synchronize()
        exact = {}
        for name, _, _, w, _, _, out, st in items:
            exact[name] = torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16))
            # only ESC collisions of the row-bucket builder (bare ESC codes) may differ
            if not exact[name] and st["esc_collisions"] == 0:
                raise RuntimeError(f"AWQ decode ({layout}) of {name} is not bit-exact")
        per = []
        tot_alg = tot_ms = 0.0
        for name, n, m, w, sc, call, out, st in items:
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(args.steps)]
            for s, e in ev:
                s.record(stream)
                call(o=out)
                e.record(stream)
            torch.cuda.synchronize()
            ms = sum(s.elapsed_time(e) for s, e in ev) / args.steps
            alg = awq_algorithmic_bytes(n, m, sc)
            tot_alg += alg
            tot_ms += ms
            per.append({"tensor": name, "shape": [n, m], "buckets": int(sc["bucket_table_i32"].shape[0]),
                        "tables": int(sc["decode_syms_u16"].shape[0]),
                        "bitstream_bits_per_elem": round(64 * sc["bitstream_u64"].numel() / (n * m), 3),
                        "esc_keys": st["esc_keys"], "esc_collisions": st["esc_collisions"],
                        "bit_exact": exact[name],
                        "ms": round(ms, 4), "rw_gbs": round(alg / ms / 1e6, 1),
                        "pct_hbm_peak_rw": round(100 * alg / ms / 1e6 / HBM_PEAK_GBS, 2)})
            log(f"{layout} {name} {n}x{m}: {ms:.4f} ms, {per[-1]['pct_hbm_peak_rw']}% of HBM peak")
        elems = sum(n * m for _, n, m, *_ in items)
        # the same layer through one AwqDecodePlan launch (every bucket of the 7 tensors)
        plan = awq.AwqDecodePlan([(w.int4_u8, sc, out) for _, _, _, w, sc, _, out, _ in items])
        for _ in range(max(1, args.warmup // 10)):
            plan.decode(stream)
        torch.cuda.synchronize()
        for name, _, _, w, _, _, out, st in items:
            if not torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16)) and st["esc_collisions"] == 0:
                raise RuntimeError(f"AWQ plan decode ({layout}) of {name} is not bit-exact")
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        for s0, e0 in ev:
            s0.record(stream)
            plan.decode(stream)
            e0.record(stream)
        torch.cuda.synchronize()
        plan_ms = sum(s0.elapsed_time(e0) for s0, e0 in ev) / args.steps
        log(f"{layout} layer: {tot_ms:.4f} ms as 7 op launches, {plan_ms:.4f} ms as one plan launch "
            f"({plan.info()['work_items']} work items)")
        results[layout] = {"layer_decode_ms": round(tot_ms, 4), "out_gbs": round(2 * elems / tot_ms / 1e6, 1),
                           "algorithmic_bytes": int(tot_alg), "achieved_gbs": round(tot_alg / tot_ms / 1e6, 1),
                           "plan_layer_ms": round(plan_ms, 4), "plan_out_gbs": round(2 * elems / plan_ms / 1e6, 1),
                           "plan_achieved_gbs": round(tot_alg / plan_ms / 1e6, 1),
                           "plan_work_items": plan.info()["work_items"], "per_tensor": per}
        plan.close()
    cpu = None
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        done = 0
        elapsed = 0.0
        while elapsed < args.cpu_seconds:
            for name, n, m, w, sc, _, _, _ in layouts["by_scale"]:
                hsc = {k: v.cpu().numpy() for k, v in sc.items()}
                q = w.int4_u8.cpu().numpy()
                t0 = time.perf_counter()
                got = oracle.awq_decode(hsc, q, n, m, nthreads=threads)
                elapsed += time.perf_counter() - t0
                if not np.array_equal(got, w.bf16.view(torch.uint16).cpu().numpy()):
                    raise RuntimeError(f"CPU baseline AWQ decode of {name} is not bit-exact")
                done += n * m
                if elapsed >= args.cpu_seconds:
                    break
        cpu = {"value": round(2 * done / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"oracle AWQ by-scale decode of layer-0 weights, {done / 1e6:.1f} M elements in "
                         f"{elapsed:.2f} s"}
    head = results["by_scale"]
    traffic, traffic_src = read_traffic("awq8b_by_scale", os.path.join(ROOT, "profiles", "awq_decode_layer8b.md"))
    result = {
        "metric": "AWQ int4 -> BF16 decompress GB/s (out); one Llama-3-8B layer in one plan launch",
        "value": head["plan_out_gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["plan_layer_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u16", "data": "synthetic: seeded N(0,0.02^2) BF16, AWQ-style int4 (group 128), sidecar built on "
                                "the GPU",
        "config": {"workload": WORKLOADS["awq8b"], "threads_per_block": args.awq_k, "layouts": results},
        "roofline": {"bound": "hbm", "achieved": head["plan_achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["plan_achieved_gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": head["algorithmic_bytes"], "kernel_ms": head["plan_layer_ms"],
                     "traffic_source": traffic_src},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def weight_list(workload: str):
    """(name, n, m, seed, sigma, outlier_p) of every weight of a workload."""
    from mpserve_amd.synthetic import config_weights

    return config_weights("layer8b" if workload == "gemm8b" else workload)


def data_note(workload: str) -> str:
    if workload == "layer70b":
        return ("synthetic: seeded N(0,0.015^2) BF16 with 0.1% outliers at +-8 sigma, per-channel FP8 e4m3, "
                "sidecar built on the GPU")
    return "synthetic: seeded N(0,0.02^2) BF16, per-channel FP8 e4m3, sidecar built on the GPU"


def time_per_tensor(entries, outs, stream, reps: int = 20):
    """Each tensor decoded alone, timed with events around each launch on its
    stream: through the drop-in op (one launch per tensor over its buckets, as
    the reference decodes), and through a plan of that tensor alone (which
    splits large buckets into row ranges when they are few for the CUs)."""
    import torch

    import MPServe_cuda
    from mpserve_amd.decode import DecodePlan, sidecar_decode_args

    def timed(launch):
        for _ in range(3):
            launch()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for s, e in ev:
            s.record(stream)
            launch()
            e.record(stream)
        torch.cuda.synchronize()
        return sum(s.elapsed_time(e) for s, e in ev) / reps

    rows = []
    for (name, fp8, sc, src), o in zip(entries, outs):
        n, m = int(fp8.shape[0]), int(fp8.shape[1])
        call = sidecar_decode_args(fp8, sc)
        alg = algorithmic_bytes(n, m, sc)
        row = {"tensor": name, "shape": [n, m], "buckets": int(sc["bucket_table_i32"].shape[0]),
               "esc_tables": int(((sc["decode_lens_u8"] & 0x88) != 0).any(dim=1).sum().item())}
        plan = DecodePlan([(fp8, sc, o)])
        row["plan_work_items"] = plan.info()["work_items"]
        for key, launch in (("op", lambda: MPServe_cuda.huffman_decode_fp8(*call, out=o)),
                            ("plan", lambda: plan.decode(stream))):
            o.zero_()
            ms = timed(launch)
            if not torch.equal(o.view(torch.uint16), src.view(torch.uint16)):
                raise RuntimeError(f"per-tensor decode ({key}) of {name} is not bit-exact")
            row[f"{key}_ms"] = round(ms, 4)
            row[f"{key}_rw_gbs"] = round(alg / ms / 1e6, 1)
            row[f"{key}_pct_hbm_peak_rw"] = round(100.0 * alg / ms / 1e6 / HBM_PEAK_GBS, 2)
        plan.close()
        rows.append(row)
        log(f"{name} {n}x{m}: op {row['op_ms']:.4f} ms ({row['op_pct_hbm_peak_rw']}%), plan of "
            f"{row['plan_work_items']} items {row['plan_ms']:.4f} ms ({row['plan_pct_hbm_peak_rw']}%)")
    return rows


def run_gemm(args, entries, outs, plan, dev) -> int:
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
    outs2 = [torch.empty_like(o) for o in outs]
    plan2 = DecodePlan((fp8, sc, o) for (_, fp8, sc, _), o in zip(entries, outs2))
    plans, bufs = (plan, plan2), (outs, outs2)
    for _ in range(max(1, args.warmup)):
        plan.decode(stream)
    plan2.decode(stream)
    torch.cuda.synchronize()
    for (name, _, _, src), o, o2 in zip(entries, outs, outs2):
        for buf in (o, o2):
            if not torch.equal(buf.view(torch.uint16), src.view(torch.uint16)):
                raise RuntimeError(f"decode of {name} is not bit-exact")
    log("decoded scratch bit-exact")
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

    results = []
    for T in (1, 16, 128, 1024):
        xs = [torch.randn((T, o.shape[1]), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
              for o in outs]

        def gemms(ws):
            for x, w in zip(xs, ws):
                F.linear(x, w)

        def sequential():
            plan.decode(stream)
            gemms(outs)

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

        t_gemm = timed(lambda: gemms(outs), 50)
        t_dec = timed(lambda: plan.decode(stream), 50)
        t_seq = timed(sequential, 50)
        t_ovl = timed(overlapped, 10) / chain
        results.append({"T": T, "gemm_ms": round(t_gemm, 4), "decode_ms": round(t_dec, 4),
                        "sequential_ms": round(t_seq, 4), "overlapped_ms": round(t_ovl, 4),
                        "decode_share_sequential": round((t_seq - t_gemm) / t_seq, 4),
                        "decode_share_overlapped": round(max(0.0, t_ovl - t_gemm) / t_ovl, 4)})
        log(f"T={T}: GEMMs {t_gemm:.4f} ms, decode {t_dec:.4f} ms, sequential {t_seq:.4f} ms, "
            f"overlapped {t_ovl:.4f} ms per layer")
    share16 = [r for r in results if r["T"] == 16][0]["decode_share_sequential"]
    result = {
        "metric": "cfg4: decode share of an 8B layer's latency (decode + 7 BF16 GEMMs), T=16",
        "value": round(100.0 * share16, 2), "unit": "%", "n_gpus": 1, "steps": 50, "warmup": args.warmup,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "u16+bf16",
        "data": data_note(args.workload),
        "config": {"workload": WORKLOADS[args.workload], "tensors": len(entries),
                   "elements": sum(o.numel() for o in outs), "overlap_chain_layers": chain, "results": results},
    }
    print(json.dumps(result), flush=True)
    return 0


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


# builder outputs the compress script does not persist (bucket_U/unique_gid/fp8_uidx)
_NOT_STORED = ("bucket_U_i32", "bucket_unique_gid_i32", "bucket_fp8_uidx_i16")


def sidecar_bytes(sc) -> int:
    """Bytes of the sidecar tensors a checkpoint stores next to the FP8 bytes."""
    return sum(t.numel() * t.element_size() for k, t in sc.items() if k not in _NOT_STORED)


def read_traffic(workload: str, path: str = TRAFFIC_PROFILE):
    """HBM bytes per decode launch from a committed rocprofv3 PMC summary, if it covers this workload."""
    try:
        text = open(path).read()
    except OSError:
        return None, None
    m = re.search(r"^traffic_bytes_per_launch\[%s\]\s*=\s*([0-9.eE+]+)" % re.escape(workload), text, re.M)
    if not m:
        return None, None
    return float(m.group(1)), os.path.relpath(path, ROOT)


def cpu_baseline(items, seconds: float, threads: int):
    """Oracle (CPU restatement) decode of layer-0 weights, repeated until ``seconds`` pass."""
    import numpy as np
    import oracle

    host = []
    for name, fp8, sc, src in items:
        n, m = fp8.shape
        host.append((name, fp8.cpu().numpy(), {k: v.cpu().numpy() for k, v in sc.items()},
                     src.view(__import__("torch").uint16).cpu().numpy(), n, m))
    done_elems = 0
    elapsed = 0.0
    names = []
    while elapsed < seconds:
        for name, q, sc, ref, n, m in host:
            out = np.empty((n, m), dtype=np.uint16)
            t0 = time.perf_counter()
            oracle.decode(sc, q, n, m, 7, oracle.MODE_LOSSLESS, threads, out)
            elapsed += time.perf_counter() - t0
            if not np.array_equal(out, ref):
                raise RuntimeError(f"CPU baseline decode of {name} is not bit-exact")
            done_elems += n * m
            names.append(name)
            if elapsed >= seconds:
                break
    gbs = 2.0 * done_elems / elapsed / 1e9
    sample = (f"{len(names)} decodes of layer-0 weights ({done_elems / 1e6:.1f} M elements, "
              f"{2 * done_elems / 1e9:.2f} GB BF16 out) in {elapsed:.2f} s")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port", "sample": sample}


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
    from mpserve_amd.encode import build_fp8_sidecar
    from mpserve_amd.decode import DecodePlan
    from mpserve_amd.synthetic import make_weight

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.workload == "awq8b":
        return run_awq(args, dev)
    weights = weight_list(args.workload)
    log(f"workload {args.workload}: {len(weights)} tensors, building inputs on {torch.cuda.get_device_name(dev)}")

    t_build = time.perf_counter()
    entries = []  # (name, fp8, sidecar, src)
    total_alg = 0
    total_side = 0
    for i, (name, n, m, seed, sigma, outlier_p) in enumerate(weights):
        w = make_weight(n, m, sigma=sigma, seed=seed, outlier_p=outlier_p, device=dev)
        sc = build_fp8_sidecar(w.bf16, w.fp8_u8, w.scale_u16, max_len=7, threads_per_block=1024)
        entries.append((name, w.fp8_u8, sc, w.bf16))
        total_alg += algorithmic_bytes(n, m, sc)
        total_side += sidecar_bytes(sc)
        del w
        if i % 7 == 6 or i == len(weights) - 1:
            log(f"built {i + 1}/{len(weights)} ({time.perf_counter() - t_build:.1f} s)")
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t_build

    outs = [torch.empty(src.shape, dtype=torch.bfloat16, device=dev) for _, _, _, src in entries]
    plan = DecodePlan((fp8, sc, o) for (_, fp8, sc, _), o in zip(entries, outs))
    elems = sum(o.numel() for o in outs)
    bf16_bytes = 2 * elems
    stream = torch.cuda.current_stream(dev)
    if args.workload == "gemm8b":
        return run_gemm(args, entries, outs, plan, dev)

    for _ in range(max(1, args.warmup)):
        plan.decode(stream)
    torch.cuda.synchronize()
    if not args.no_verify:
        for (name, _, _, src), o in zip(entries, outs):
            if not torch.equal(o.view(torch.uint16), src.view(torch.uint16)):
                raise RuntimeError(f"decode of {name} is not bit-exact")
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
        for (name, _, _, src), o in zip(entries, outs):
            if not torch.equal(o.view(torch.uint16), src.view(torch.uint16)):
                raise RuntimeError(f"timed decode of {name} is not bit-exact")
    per_tensor = time_per_tensor(entries, outs, stream) if args.workload != "model8b" else None

    if args.copy_calibration > 0:
        n32 = args.copy_calibration * (1 << 20) // 4
        src32 = torch.ones(n32, dtype=torch.int32, device=dev)
        dst32 = torch.empty_like(src32)
        for _ in range(3):
            torch.bitwise_not(src32, out=dst32)
        torch.cuda.synchronize()
        log(f"copy calibration: 3 x bitwise_not over {args.copy_calibration} MiB int32 "
            f"(reads and writes {n32 * 4} bytes each)")
        del src32, dst32

    value = bf16_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = total_alg / (kernel_ms * 1e-3) / 1e9
    traffic, traffic_src = read_traffic(args.workload)
    cpu = None
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        layer0 = [e for e in entries if e[0].startswith("layers.0.")]
        log(f"CPU baseline: oracle decode on {threads} threads, ~{args.cpu_seconds:.0f} s budget")
        cpu = cpu_baseline(layer0, args.cpu_seconds, threads)

    fp8_bytes = elems
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u16",
        "data": data_note(args.workload),
        "config": {
            "workload": WORKLOADS[args.workload],
            "tensors": len(entries),
            "elements": elems,
            "max_len": 7,
            "threads_per_block": 1024,
            "full_decode_ms": round(kernel_ms, 4),
            "pct_hbm_peak_out": round(100.0 * value / HBM_PEAK_GBS, 2),
            "pct_hbm_peak_rw": round(100.0 * achieved / HBM_PEAK_GBS, 2),
            "sidecar_over_bf16": round(total_side / bf16_bytes, 4),
            "sidecar_plus_fp8_over_bf16": round((total_side + fp8_bytes) / bf16_bytes, 4),
            "build_s": round(build_s, 2),
            "plan": plan.info(),
            # LDS per workgroup (the bucket's 256 expanded tables + the bitstream queues) and waves per CU
            "lds_occupancy": {"bytes_per_workgroup": plan.info()["lds_bytes"], "of_cu_lds": 163840,
                              "workgroups_per_cu": 1, "waves_per_cu": 16},
            "esc_tables": sum(int(((sc["decode_lens_u8"] & 0x88) != 0).any(dim=1).sum().item())
                              for _, _, sc, _ in entries),
            "per_tensor": per_tensor,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes": total_alg,
            "kernel_ms": round(kernel_ms, 4),
            "traffic_source": traffic_src,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
