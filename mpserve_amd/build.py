"""Compile libmpserve_amd.so (HIP, gfx950) in-tree.

``python -m mpserve_amd.build`` or ``mpserve_amd.build.build()``. The library is
placed next to this file so it travels with the source tree.

Tuning builds: ``python -m mpserve_amd.build --define MPS_SLAB_PREFETCH=12 --out
/tmp/lib_df12.so`` compiles the same sources with the decode kernel's
compile-time knobs set otherwise (``MPS_SLAB_PREFETCH``, ``MPS_PRIO_LEAD``,
``MPS_SLAB_RESERVE_BLOCKS``, ``MPS_SLAB_ALIGN``, ``MPS_SLAB_OUT_CPOL``,
``MPS_SLAB_FP8_CPOL``, ``MPS_SLAB_BS_CPOL``, and the plans' ``MPS_SPLIT_DIV``,
``MPS_TAIL_RATIO``; for AWQ ``MPS_AWQ_SLAB_PREFETCH``, ``MPS_AWQ_FEED_EVERY``,
``MPS_AWQ_PRIO``, ``MPS_AWQ_PRIO_LEAD``, ``MPS_AWQ_RUN_DIV``) into another file, for
``bench.py --compare-libs``. The product library is never built with defines.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmpserve_amd.so")
ARCH = os.environ.get("MPS_OFFLOAD_ARCH", "gfx950")

SOURCES = ["fp8_decode.hip", "fp8_encode.hip", "awq_decode.hip"]

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    # Packed FP32 VALU forms stay off (no float code here, but keep the rule global).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def build(verbose: bool = False, defines=(), out: str | None = None) -> str:
    """Compile every HIP source into libmpserve_amd.so (always recompiles), or,
    with ``defines`` (``NAME=VALUE`` strings), into the tuning library ``out``.
    The sources compile in parallel, one object each (in a temporary
    directory), and are then linked."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    if defines and (out is None or os.path.abspath(out) == LIB):
        raise ValueError("a build with --define needs --out: the product library keeps the default knobs")
    target = os.path.abspath(out) if out else LIB
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    incs = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    with tempfile.TemporaryDirectory(prefix="mps_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.basename(s) + ".o") for s in srcs]
        cmds = [[_hipcc(), *flags, *(f"-D{d}" for d in defines), *incs, "-c", s, "-o", o] for s, o in zip(srcs, objs)]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
            for f in [ex.submit(subprocess.run, c, check=True) for c in cmds]:
                f.result()
        tmp = target + ".tmp"
        link = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
        if verbose:
            print(" ".join(link), flush=True)
        subprocess.run(link, check=True)
    os.replace(tmp, target)
    return target


def main(argv=None) -> int:
    import argparse

    p = argparse.ArgumentParser(description="compile libmpserve_amd.so for gfx950")
    p.add_argument("-v", "--verbose", action="store_true")
    p.add_argument("--define", action="append", default=[], metavar="NAME=VALUE",
                   help="compile-time knob of a tuning build (needs --out)")
    p.add_argument("--out", default=None, help="output path of a tuning build")
    a = p.parse_args(argv)
    try:
        print(build(a.verbose, a.define, a.out))
    except ValueError as e:
        p.error(str(e))
    return 0


if __name__ == "__main__":
    sys.exit(main())
