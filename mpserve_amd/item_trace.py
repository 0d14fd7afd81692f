"""Work-item timelines of one decode plan launch, from an instrumented build.

Build the library with the trace compiled in (it is off in the product build),
then run one of the synthetic workloads through it::

    python -m mpserve_amd.build --define MPS_TRACE_ITEMS=1 --out /tmp/lib_trace.so
    python -m mpserve_amd.item_trace /tmp/lib_trace.so --workload layer8b --k 1024

FP8 workloads (model8b, layer8b, layer70b): every workgroup of the plan kernel
records, for its first 128 items, the real-time clock (100 MHz) at the item's
start, after its set-up's last barrier, when waves 0 and 15 finish their
decode, and after its end barrier. The summary gives the launch's span, when
the workgroups ended (the tail), a least-squares fit of an item's duration to
``a + b * (elements one work-item decodes)``, whose intercept is the per-item
overhead, and the mean of each phase: set-up (start to the set-up barrier),
decode (to the last of the two waves' ends) and drain (to the end barrier).
AWQ workload (awq8b, both layouts at ``--k``): one record per workgroup, its
duration by record kind.

The decoded outputs are checked bit-exact against the inputs (ESC collisions of
the AWQ row builder aside), so a trace comes from a correct launch.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
from typing import Dict, List

import numpy as np


def _fit(x: np.ndarray, y: np.ndarray) -> Dict[str, float]:
    a = np.vstack([np.ones_like(x, dtype=float), x.astype(float)]).T
    (c0, c1), *_ = np.linalg.lstsq(a, y, rcond=None)
    return {"setup_us": round(float(c0), 2), "ns_per_lane_element": round(float(c1) * 1000.0, 1)}


def _lib(path: str) -> ctypes.CDLL:
    lib = ctypes.CDLL(os.path.abspath(path))
    for name in ("mps_item_trace_clear", "mps_awq_trace_clear"):
        if not hasattr(lib, name):
            raise SystemExit(f"{path} has no {name}: build it with --define MPS_TRACE_ITEMS=1")
    return lib


def fp8_trace(lib_path: str, workload: str, k: int) -> Dict:
    import torch

    from . import _native
    from .decode import sidecar_decode_args
    from .encode import build_fp8_sidecar
    from .mpserve_cuda import _descriptor
    from .synthetic import config_weights, make_weight

    lib = _lib(lib_path)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.mps_fp8_plan_create.argtypes = [ctypes.POINTER(_native.MpsFp8Tensor), i64, vp, ctypes.POINTER(vp)]
    lib.mps_fp8_plan_decode.argtypes = [vp, vp]
    lib.mps_fp8_plan_destroy.argtypes = [vp]
    lib.mps_item_trace_read.argtypes = [ctypes.POINTER(ctypes.c_uint64), i64]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    entries = []
    for name, n, m, seed, sigma, outlier_p in config_weights(workload):
        w = make_weight(n, m, sigma=sigma, seed=seed, outlier_p=outlier_p, device=dev)
        sc = build_fp8_sidecar(w.bf16, w.fp8_u8, w.scale_u16, max_len=7, threads_per_block=k)
        entries.append((w.fp8_u8, sc, w.bf16, torch.empty((n, m), dtype=torch.bfloat16, device=dev)))
    descs = [_descriptor(*sidecar_decode_args(f, sc)[:13], o) for f, sc, _, o in entries]
    arr = (_native.MpsFp8Tensor * len(descs))(*descs)
    h = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    plan = ctypes.c_void_p()
    _native.check(lib.mps_fp8_plan_create(arr, len(descs), h, ctypes.byref(plan)))
    try:
        for _ in range(20):  # steady clocks
            _native.check(lib.mps_fp8_plan_decode(plan, h))
        torch.cuda.synchronize()
        exact = all(torch.equal(o.view(torch.uint16), s.view(torch.uint16)) for _, _, s, o in entries)
        if not exact:
            raise RuntimeError("the instrumented build's decode is not bit-exact")
        _native.check(lib.mps_item_trace_clear())
        torch.cuda.synchronize()
        _native.check(lib.mps_fp8_plan_decode(plan, h))
        torch.cuda.synchronize()
        words = 256 * 128 * 12
        buf = (ctypes.c_uint64 * words)()
        _native.check(lib.mps_item_trace_read(buf, words))
    finally:
        lib.mps_fp8_plan_destroy(plan)
    a = np.frombuffer(buf, dtype=np.uint64).reshape(256, 128, 12).astype(np.int64)
    valid = a[:, :, 1] > 0
    t0 = int(a[:, :, 0][valid].min())
    rec = a[valid]
    dur = (rec[:, 1] - rec[:, 0]) / 100.0  # us
    path, rows, k_eff, cl = rec[:, 2] >> 40, (rec[:, 2] >> 20) & 0xFFFFF, rec[:, 2] & 0xFFFFF, rec[:, 3]
    multi = (path & 0x10) != 0
    range_rows = np.where(multi, np.minimum((path >> 8) & 0xFF, rows), rows)
    per_lane = range_rows * (cl // np.maximum(k_eff, 1))
    ends = np.array([(a[g][valid[g]][:, 1].max() - t0) / 100.0 for g in range(256) if valid[g].any()])
    busy = np.array([(a[g][valid[g]][:, 1] - a[g][valid[g]][:, 0]).sum() / 100.0
                     for g in range(256) if valid[g].any()])
    truncated = int(valid.sum(axis=1).max()) >= 128
    out = {"workload": workload, "k": k, "items_traced": int(len(rec)), "workgroups": int(len(ends)),
           "trace_truncated": truncated, "span_us": round(float(ends.max()), 1),
           "wg_end_us": {"min": round(float(ends.min()), 1), "median": round(float(np.median(ends)), 1),
                         "max": round(float(ends.max()), 1)},
           "busy_mean_us": round(float(busy.mean()), 1),
           "idle_at_end_frac": round(float(1.0 - busy.mean() / ends.max()), 4),
           "fit_all": _fit(per_lane, dur)}
    setup = (rec[:, 4] - rec[:, 0]) / 100.0
    wave_end = np.maximum(rec[:, 5], rec[:, 6])
    decode = (wave_end - rec[:, 4]) / 100.0
    drain = (rec[:, 1] - wave_end) / 100.0
    skew = np.abs(rec[:, 5] - rec[:, 6]) / 100.0
    out["phases_us"] = {"setup_mean": round(float(setup.mean()), 2), "setup_median": round(float(np.median(setup)), 2),
                        "decode_mean": round(float(decode.mean()), 2), "drain_mean": round(float(drain.mean()), 2),
                        "drain_median": round(float(np.median(drain)), 2),
                        "wave0_wave15_skew_mean": round(float(skew.mean()), 2)}
    out["fit_decode_phase"] = _fit(per_lane, decode)
    lv = rec[:, 7]
    if (lv != 0).any():
        l1, l2 = (lv & 0xFFFFFFFF) / 100.0, (lv >> 32) / 100.0
        out["setup_levels_us"] = {"level1_mean": round(float(l1.mean()), 2),
                                  "level2_mean": round(float((l2 - l1).mean()), 2),
                                  "after_level2_mean": round(float((setup - l2).mean()), 2)}
        w8, w9 = rec[:, 8], rec[:, 9]
        if (w8 != 0).any():
            exp_end, b1 = (w8 & 0xFFFFFFFF) / 100.0, (w8 >> 32) / 100.0
            out["setup_levels_us"].update({
                "last_wave_tables_mean": round(float((w9 / 100.0).mean()), 2),
                "wave0_expansion_end_mean": round(float(exp_end.mean()), 2),
                "first_barrier_mean": round(float(b1.mean()), 2)})
    if multi.any():
        out["fit_side_by_side"] = _fit(per_lane[multi], dur[multi])
        out["items_side_by_side"] = int(multi.sum())
    return out


def awq_trace(lib_path: str, k: int) -> Dict:
    import torch

    from . import _native, awq
    from .awq import _sidecar_descriptor
    from .synthetic import LLAMA3_8B_LAYER, make_awq_weight

    lib = _lib(lib_path)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.mps_awq_plan_create.argtypes = [ctypes.POINTER(_native.MpsAwqTensor), i64, vp, ctypes.POINTER(vp)]
    lib.mps_awq_plan_decode.argtypes = [vp, vp]
    lib.mps_awq_plan_destroy.argtypes = [vp]
    lib.mps_awq_trace_read.argtypes = [ctypes.POINTER(ctypes.c_uint64), i64]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    h = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    kinds = {0: "per-lane run", 1: "slab bucket run", 2: "row range", 3: "ranges side by side"}
    result = {"workload": "awq8b", "k": k, "layouts": {}}
    for layout, group in (("by_scale", 128), ("row_buckets", None)):
        items = []
        for j, (_, n, m) in enumerate(LLAMA3_8B_LAYER):
            w = make_awq_weight(n, m, group, seed=300 + j, device=dev)
            sc, st = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, k, 1024, bool(group), with_stats=True)
            o = torch.empty((n, m), dtype=torch.bfloat16, device=dev)
            items.append((w, sc, o, st))
        arr = (_native.MpsAwqTensor * len(items))(*[_sidecar_descriptor(w.int4_u8, sc, o) for w, sc, o, _ in items])
        plan = ctypes.c_void_p()
        _native.check(lib.mps_awq_plan_create(arr, len(items), h, ctypes.byref(plan)))
        try:
            for _ in range(20):
                _native.check(lib.mps_awq_plan_decode(plan, h))
            torch.cuda.synchronize()
            for w, _, o, st in items:
                if st["esc_collisions"] == 0 and not torch.equal(o.view(torch.uint16), w.bf16.view(torch.uint16)):
                    raise RuntimeError("the instrumented build's AWQ decode is not bit-exact")
            _native.check(lib.mps_awq_trace_clear())
            torch.cuda.synchronize()
            _native.check(lib.mps_awq_plan_decode(plan, h))
            torch.cuda.synchronize()
            words = 8192 * 4
            buf = (ctypes.c_uint64 * words)()
            _native.check(lib.mps_awq_trace_read(buf, words))
        finally:
            lib.mps_awq_plan_destroy(plan)
        a = np.frombuffer(buf, dtype=np.uint64).reshape(8192, 4).astype(np.int64)
        a = a[a[:, 1] > 0]
        t0 = int(a[:, 0].min())
        dur = (a[:, 1] - a[:, 0]) / 100.0
        kind = a[:, 2] >> 32
        by_kind: Dict[str, Dict] = {}
        for kv in sorted(set(kind.tolist())):
            d = dur[kind == kv]
            by_kind[kinds.get(int(kv), str(kv))] = {"records": int(d.size), "mean_us": round(float(d.mean()), 1),
                                                    "max_us": round(float(d.max()), 1)}
        span = float((a[:, 1].max() - t0) / 100.0)
        ends = np.sort((a[:, 1] - t0) / 100.0)
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        result["layouts"][layout] = {"records_traced": int(len(a)),
                                     "span_us": round(span, 1),
                                     "record_us_mean": round(float(statistics.mean(dur.tolist())), 1),
                                     # records' time over the CUs' (one workgroup per CU)
                                     "busy_fraction": round(float(dur.sum()) / (span * cus), 3),
                                     "last_start_us": round(float((a[:, 0].max() - t0) / 100.0), 1),
                                     # when the last CUs' records end: the CUs-th latest end and the median of those
                                     "ends_us": {"cus_th_latest": round(float(ends[-min(cus, len(ends))]), 1),
                                                 "median_of_last_cus": round(float(np.median(ends[-cus:])), 1)},
                                     "by_kind": by_kind}
    return result


def main(argv: List[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("lib", help="a libmpserve_amd build with --define MPS_TRACE_ITEMS=1")
    p.add_argument("--workload", choices=("model8b", "layer8b", "layer70b", "awq8b"), default="layer8b")
    p.add_argument("--k", type=int, default=1024, help="substreams per bucket of the sidecars")
    args = p.parse_args(argv)
    res = awq_trace(args.lib, args.k) if args.workload == "awq8b" else fp8_trace(args.lib, args.workload, args.k)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
