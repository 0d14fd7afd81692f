"""The committed AWQ int4 golden sidecars (written by tests/golden/make_awq_fixtures.py).

CPU: the oracle still builds every fixture byte for byte, and decodes it back to
the input (except the elements of the row builder's ESC collision, which the
reference's own stream cannot carry). GPU: the HIP builders give the same
arrays, and the HIP decoders give the oracle's output. Integer work: the bar is
equality.
"""
import json
import os

import numpy as np
import pytest
import torch

import MPServe_cuda
import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "awq_manifest.json")))
NAMES = sorted(MANIFEST)
DEV = "cuda:0"


def _load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as z:
        arrays = {k: z[k] for k in z.files}
    side = {k: arrays["sc_" + k] for k in MANIFEST[name]["keys"]}  # the reference's key order
    return arrays["in_bf16"], arrays["in_int4"], arrays["in_scales"], side


def _build_oracle(name, bf, q, sc):
    c = MANIFEST[name]
    return oracle.awq_encode(bf, q, sc, c["max_len"], c["threads"], c["group_cap"], c["by_scale"])


def test_fixture_set_covers_the_cases():
    modes = {(c["by_scale"], c["esc_keys"] > 0, c["esc_collisions"] > 0) for c in MANIFEST.values()}
    assert (True, True, False) in modes and (False, True, True) in modes and (True, False, False) in modes
    assert any(c["threads"] > c["m"] // 4 for c in MANIFEST.values() if not c["by_scale"])


@pytest.mark.parametrize("name", NAMES)
def test_oracle_rebuilds_fixture(name):
    bf, q, sc, want = _load(name)
    got = _build_oracle(name, bf, q, sc)
    assert list(got) == list(want)
    for key in want:
        assert got[key].dtype == want[key].dtype and np.array_equal(got[key], want[key]), key
    out = oracle.awq_decode(want, q, bf.shape[0], bf.shape[1])
    bad = int((out != bf).sum())
    assert (bad == 0) == (MANIFEST[name]["esc_collisions"] == 0)


def _decode_gpu(side, q, n, m, by_scale):
    t = {k: torch.from_numpy(v).to(DEV) for k, v in side.items()}
    t["bitstream_u64"] = torch.from_numpy(side["bitstream_u64"].view(np.int64)).to(DEV).view(torch.uint64)
    t["decode_syms_u16"] = torch.from_numpy(side["decode_syms_u16"].view(np.int16)).to(DEV).view(torch.uint16)
    t["bucket_thread_startbit_u32"] = torch.from_numpy(
        side["bucket_thread_startbit_u32"].view(np.int32)).to(DEV).view(torch.uint32)
    qd = torch.from_numpy(q).to(DEV)
    if by_scale:
        out = MPServe_cuda.huffman_decode_awq_int4_bucket_by_scale(
            qd, t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"], t["bucket_table_i32"],
            t["bucket_group_offsets_i32"], t["group_rows_i32"], t["group_col_start_i32"],
            t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], n, m, 11, int(side["shape_nmkg_i64"][3]))
    else:
        out = MPServe_cuda.huffman_decode_awq_int4_bucket(
            qd, t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"], t["bucket_table_i32"],
            t["bucket_col_start_i32"], t["bucket_col_len_i32"], t["bucket_row_offsets_i32"], t["row_indices_i32"],
            t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], n, m, 11)
    torch.cuda.synchronize()
    return out.view(torch.uint16).cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_gpu_build_and_decode_match_fixture(name):
    print(f"[awq golden] {name}", flush=True)
    c = MANIFEST[name]
    bf, q, sc, want = _load(name)
    bft = torch.from_numpy(bf.view(np.int16)).view(torch.bfloat16)
    qt = torch.from_numpy(q)
    st = torch.from_numpy(sc.view(np.int16)).view(torch.uint16)
    if c["by_scale"]:
        got = MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables_by_scale(
            bft, qt, st, c["max_len"], c["threads"], c["group_cap"])
    else:
        got = MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables(bft, qt, st, c["max_len"], c["threads"])
    assert list(got) == list(want)
    for key in want:
        g = got[key].numpy()
        assert np.array_equal(g.view(want[key].dtype) if g.dtype != want[key].dtype else g, want[key]), key
    out = _decode_gpu(want, q, bf.shape[0], bf.shape[1], c["by_scale"])
    ref = oracle.awq_decode(want, q, bf.shape[0], bf.shape[1])
    if c["esc_collisions"] == 0:
        assert np.array_equal(out, bf) and np.array_equal(out, ref)
    else:
        # a bare ESC code desynchronises its lane: every other lane still matches
        k = c["threads"]
        e = np.arange(bf.size).reshape(bf.shape) % k  # lane of each element (one bucket, col_len == m)
        bad_lanes = np.unique(e[ref != bf])
        ok = ~np.isin(e, bad_lanes)
        assert np.array_equal(out[ok], bf[ok])
