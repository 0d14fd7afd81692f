"""Write the golden sidecar fixtures of tests/golden/ (run from the repository root).

Each fixture holds a small seeded input (BF16 bits, FP8 bytes, u16 scale keys)
and the 17 sidecar arrays the CPU oracle builds from it. The oracle itself is
pinned by hand-traced vectors, brute force and invariants
(tests/test_oracle_known_answers.py, tests/test_oracle_properties.py); the
reference ships no fixtures of its own. The cases are chosen to reach every
decode path and bucketing mode: per-row, scalar and block-2D scale keys; the
k = 1024 slab path with P = 4 and with P = 14 (rows straddle groups); k = 1024
with P < 4; tables with ESC codes on the slab path at P = 4 and P = 14; other
k; and col_len < k.

    python tests/golden/make_fixtures.py [name ...]   (default: every fixture)
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from mpserve_amd.synthetic import make_weight  # noqa: E402

# name: (n, m, k, seed, sigma, outlier_p, scale mode)
CASES = {
    "slab_p4": (8, 4096, 1024, 101, 0.02, 0.0, "row"),
    "slab_wrap_p14": (4, 14336, 1024, 102, 0.02, 0.0, "row"),
    "k1024_p2": (16, 2048, 1024, 103, 0.02, 0.0, "row"),
    "esc_k1024": (12, 4096, 1024, 104, 0.0, 0.0, "esc"),
    "esc_slab_p14": (6, 14336, 1024, 108, 0.0, 0.0, "esc"),
    "scalar_k256": (300, 513, 256, 105, 0.02, 0.0, "scalar"),
    "narrow_k1024": (40, 100, 1024, 106, 0.02, 0.0, "row"),
    "block2d": (256, 256, 64, 107, 0.02, 0.0, "block2d"),
}
MAX_LEN = 7


def inputs(n, m, seed, sigma, outlier_p, mode):
    if mode == "esc":
        # one (scale, fp8) key carrying 600 distinct BF16 symbols with a skewed
        # head (so the kept set is well defined): its rare symbols need ESC codes
        rng = np.random.default_rng(seed)
        bf = rng.integers(0x3C00, 0x3C00 + 600, size=(n, m)).astype(np.uint16)
        head = rng.random((n, m)) < 0.5
        bf[head] = (0x3C00 + rng.integers(0, 20, size=int(head.sum()))).astype(np.uint16)
        q = np.full((n, m), 0x38, dtype=np.uint8)
        q[:, ::7] = 0x39  # a second, small key
        return bf, q, np.array([0x1C00], dtype=np.uint16)
    w = make_weight(n, m, sigma=sigma, seed=seed, outlier_p=outlier_p)
    bf = w.bf16.view(__import__("torch").uint16).numpy()
    q = w.fp8_u8.numpy()
    key = w.scale_u16.numpy()
    if mode == "scalar":
        # one key for rows quantized with different scales: a valid input whose
        # keys collect many symbols, so some need ESC codes
        sc = key[:1].copy()
    elif mode == "block2d":
        # one key per 128 x 128 block: the row key of the block's first row,
        # bumped by the block column so that column blocks differ
        sc = np.array([[key[r] + c for c in range(0, m, 128)] for r in range(0, n, 128)], dtype=np.uint16)
    else:
        sc = key
    return bf, q, sc


def main(names=None) -> int:
    path = os.path.join(HERE, "manifest.json")
    manifest = {}
    if names and os.path.exists(path):
        with open(path) as f:
            manifest = json.load(f)
    for name, (n, m, k, seed, sigma, outlier_p, mode) in CASES.items():
        if names and name not in names:
            continue
        bf, q, sc = inputs(n, m, seed, sigma, outlier_p, mode)
        side, stats = oracle.encode(bf, q, sc, MAX_LEN, k, with_stats=True)
        arrays = {"in_bf16": bf, "in_fp8": q, "in_scales": sc}
        arrays.update({"sc_" + key: v for key, v in side.items()})
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        manifest[name] = {"n": n, "m": m, "threads_per_block": k, "max_len": MAX_LEN, "seed": seed,
                          "sigma": sigma, "outlier_p": outlier_p, "scale_mode": mode,
                          "buckets": int(side["bucket_col_len_i32"].shape[0]),
                          "tables": int(side["decode_syms_u16"].shape[0]),
                          "bitstream_words": int(side["bitstream_u64"].shape[0]), **stats}
        print(name, manifest[name])
    with open(path, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
