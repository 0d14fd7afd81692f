"""Write the AWQ int4 golden sidecar fixtures of tests/golden/ (run from the repository root).

Each fixture holds a small seeded input (BF16 bits, int4 values, u16 BF16-bit
scales) and the sidecar arrays the CPU oracle builds from it with one of the
reference's two AWQ int4 builders (row buckets, build_huffman.cu:1583-2126;
by scale, build_huffman.cu:1075-1580). The oracle is pinned by
tests/test_awq_oracle.py; the reference ships no fixtures. Scales are coarsened
(low bits cleared) so that few keys, and so few 2048-entry tables, are stored.
The cases reach: per-row and block-2D scales, k below and above the column
count, by-scale group buckets cut at a small group cap, ESC keys in both
layouts, and the row builder's ESC collision (a rare symbol equal to esc_sym).

    python tests/golden/make_awq_fixtures.py
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
from mpserve_amd.synthetic import make_awq_weight  # noqa: E402
from tests.test_awq_oracle import esc_inputs  # noqa: E402

# name: (n, m, group (None: per row), k, group_cap, by_scale, seed, mode)
CASES = {
    "awq_row_per_row_k256": (64, 512, None, 256, 1, False, 401, "synthetic"),
    "awq_row_block2d_k1024": (64, 256, 64, 1024, 1, False, 402, "synthetic"),
    "awq_by_scale_g128_cap16": (64, 512, 128, 256, 16, True, 403, "synthetic"),
    "awq_esc_by_scale": (32, 1024, None, 256, 1024, True, 404, "esc"),
    "awq_esc_row_collision": (32, 1024, None, 1024, 1, False, 405, "esc_zero"),
}
MAX_LEN = 11


def inputs(n, m, group, seed, mode):
    if mode.startswith("esc"):
        return esc_inputs(n, m, distinct=3000, seed=seed, with_zero=(mode == "esc_zero"))
    import torch

    w = make_awq_weight(n, m, group, seed=seed)
    sc = (w.scale_u16.numpy() & 0xFFE0).astype(np.uint16)  # few distinct scales -> few tables
    return w.bf16.view(torch.uint16).numpy(), w.int4_u8.numpy(), sc


def main() -> int:
    manifest = {}
    for name, (n, m, group, k, cap, by_scale, seed, mode) in CASES.items():
        bf, q, sc = inputs(n, m, group, seed, mode)
        side, stats = oracle.awq_encode(bf, q, sc, MAX_LEN, k, cap, by_scale, with_stats=True)
        arrays = {"in_bf16": bf, "in_int4": q, "in_scales": sc}
        arrays.update({"sc_" + key: v for key, v in side.items()})
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        manifest[name] = {"n": n, "m": m, "threads": k, "group_cap": cap, "by_scale": by_scale,
                          "max_len": MAX_LEN, "seed": seed, "mode": mode, "keys": list(side),
                          "buckets": int(side["bucket_table_i32"].shape[0]),
                          "tables": int(side["decode_syms_u16"].shape[0]),
                          "bitstream_words": int(side["bitstream_u64"].shape[0]), **stats}
        print(name, {k: v for k, v in manifest[name].items() if k != "keys"})
    with open(os.path.join(HERE, "awq_manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
