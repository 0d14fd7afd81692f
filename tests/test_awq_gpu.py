"""AWQ int4 path on the GPU: builders byte for byte against the oracle, decoders
bit for bit against the input (and the oracle's decode), through MPServe_cuda.

Integer work: the bar is equality.
"""
import ctypes

import numpy as np
import pytest
import torch

import MPServe_cuda
import oracle
from mpserve_amd import awq
from mpserve_amd.mpserve_cuda import read_status
from mpserve_amd.synthetic import make_awq_weight
from tests.test_awq_oracle import esc_inputs

DEV = "cuda:0"
pytestmark = pytest.mark.gpu

CASES = [
    # name, n, m, group (None: per row), k, by_scale, group_cap
    ("row_per_row_k256", 192, 512, None, 256, False, 1024),
    ("row_block2d_g128_k256", 64, 512, 128, 256, False, 1024),
    ("row_block2d_g64_k1024", 96, 256, 64, 1024, False, 1024),
    ("row_per_row_k1", 8, 64, None, 1, False, 1024),
    ("by_scale_g128_k256", 128, 512, 128, 256, True, 1024),
    ("by_scale_g128_k1024_cap16", 128, 512, 128, 1024, True, 16),
    ("by_scale_per_row_k100", 96, 384, None, 100, True, 1024),
    ("by_scale_g32_k7", 32, 256, 32, 7, True, 5),
]


def _inputs(name, n, m, group):
    w = make_awq_weight(n, m, group, seed=sum(map(ord, name)))
    return w.bf16, w.int4_u8, w.scale_u16


def _build(bf16, q, sc, k, by_scale, cap):
    if by_scale:
        return MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables_by_scale(bf16, q, sc, 11, k, cap)
    return MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables(bf16, q, sc, 11, k)


def _same(got, want):
    assert list(got) == list(want)
    for key, v in want.items():
        g = got[key].numpy()
        assert g.shape == v.shape, (key, g.shape, v.shape)
        assert np.array_equal(g.view(v.dtype) if g.dtype != v.dtype else g, v), \
            f"{key}: {(g != v).sum()} entries differ"


def _decode(d, q, n, m, by_scale):
    t = {k: v.to(DEV) for k, v in d.items()}
    qd = q.to(DEV)
    if by_scale:
        out = MPServe_cuda.huffman_decode_awq_int4_bucket_by_scale(
            qd, t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"], t["bucket_table_i32"],
            t["bucket_group_offsets_i32"], t["group_rows_i32"], t["group_col_start_i32"],
            t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], n, m, 11, int(d["shape_nmkg_i64"][3]))
    else:
        out = MPServe_cuda.huffman_decode_awq_int4_bucket(
            qd, t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"], t["bucket_table_i32"],
            t["bucket_col_start_i32"], t["bucket_col_len_i32"], t["bucket_row_offsets_i32"], t["row_indices_i32"],
            t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], n, m, 11)
    torch.cuda.synchronize()
    return out.view(torch.uint16).cpu().numpy()


@pytest.mark.parametrize("name,n,m,group,k,by_scale,cap", CASES, ids=[c[0] for c in CASES])
def test_build_matches_oracle_and_decode_round_trips(name, n, m, group, k, by_scale, cap):
    print(f"[awq] {name}", flush=True)
    bf16, q, sc = _inputs(name, n, m, group)
    bits = bf16.view(torch.uint16).numpy()
    got = _build(bf16, q, sc, k, by_scale, cap)
    want = oracle.awq_encode(bits, q.numpy(), sc.numpy(), 11, k, cap, by_scale)
    _same(got, want)
    read_status(torch.device(DEV))
    out = _decode(got, q, n, m, by_scale)
    assert np.array_equal(out, bits)
    assert np.array_equal(out, oracle.awq_decode(want, q.numpy(), n, m))
    assert read_status(torch.device(DEV)) == 0


@pytest.mark.parametrize("by_scale", [False, True])
def test_esc_keys(by_scale):
    print(f"[awq] esc by_scale={by_scale}", flush=True)
    bits, q, sc = esc_inputs(with_zero=not by_scale)
    bf16 = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    qt, st = torch.from_numpy(q), torch.from_numpy(sc.view(np.int16)).view(torch.uint16)
    got = _build(bf16, qt, st, 256, by_scale, 1024)
    want, stats = oracle.awq_encode(bits, q, sc, 11, 256, 1024, by_scale, with_stats=True)
    assert stats["esc_keys"] == 1
    _same(got, want)  # row buckets: includes the reference's ESC collisions (bare ESC codes)
    if by_scale:
        read_status(torch.device(DEV))
        assert np.array_equal(_decode(got, qt, 64, 1024, True), bits)
        assert read_status(torch.device(DEV)) == 0


def test_esc_round_trip_row_buckets():
    print("[awq] esc row buckets, no collision", flush=True)
    bits, q, sc = esc_inputs(with_zero=False)
    bf16 = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    qt, st = torch.from_numpy(q), torch.from_numpy(sc.view(np.int16)).view(torch.uint16)
    got = _build(bf16, qt, st, 1024, False, 1024)
    assert np.array_equal(_decode(got, qt, 64, 1024, False), bits)


def test_cuda_inputs_give_cuda_outputs_and_same_bytes():
    bf16, q, sc = _inputs("cuda_in", 64, 256, 64)
    host = _build(bf16, q, sc, 256, True, 1024)
    dev = _build(bf16.to(DEV), q.to(DEV), sc.to(DEV), 256, True, 1024)
    for key in host:
        assert dev[key].is_cuda
        assert torch.equal(dev[key].cpu(), host[key])


@pytest.mark.parametrize("by_scale", [False, True])
def test_full_size_round_trip(by_scale):
    """Llama-3-8B q_proj, group 128: GPU build, GPU decode, equality with the input."""
    print(f"[awq] 4096x4096 by_scale={by_scale}", flush=True)
    w = make_awq_weight(4096, 4096, 128 if by_scale else None, seed=21, device=DEV)
    d = _build(w.bf16, w.int4_u8, w.scale_u16, 1024, by_scale, 1024)
    read_status(torch.device(DEV))
    t = {k: v for k, v in d.items()}
    if by_scale:
        out = awq.huffman_decode_awq_int4_bucket_by_scale(
            w.int4_u8, t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"], t["bucket_table_i32"],
            t["bucket_group_offsets_i32"], t["group_rows_i32"], t["group_col_start_i32"],
            t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], 4096, 4096, 11, 128)
    else:
        out = awq.huffman_decode_awq_int4_bucket(
            w.int4_u8, t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"], t["bucket_table_i32"],
            t["bucket_col_start_i32"], t["bucket_col_len_i32"], t["bucket_row_offsets_i32"], t["row_indices_i32"],
            t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], 4096, 4096, 11)
    assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16))
    assert read_status(torch.device(DEV)) == 0


def test_decode_argument_checks():
    bf16, q, sc = _inputs("checks", 32, 256, 128)
    d = {k: v.to(DEV) for k, v in _build(bf16, q, sc, 256, False, 1024).items()}
    qd = q.to(DEV)
    args = [qd, d["bitstream_u64"], d["decode_syms_u16"], d["decode_lens_u8"], d["bucket_table_i32"],
            d["bucket_col_start_i32"], d["bucket_col_len_i32"], d["bucket_row_offsets_i32"], d["row_indices_i32"],
            d["bucket_thread_startbit_u32"], d["bucket_bit_base_i64"], 32, 256]
    with pytest.raises(ValueError, match="max_len must be 11"):
        MPServe_cuda.huffman_decode_awq_int4_bucket(*args, 7)
    with pytest.raises(ValueError, match="int4_values_u8 numel must equal n\\*m"):
        MPServe_cuda.huffman_decode_awq_int4_bucket(*args[:-2], 31, 256)
    bad = list(args)
    bad[4] = d["bucket_table_i32"][:, :8].contiguous()
    with pytest.raises(ValueError, match=r"bucket_table_i32 must be int32 CUDA \[B,16\]"):
        MPServe_cuda.huffman_decode_awq_int4_bucket(*bad)


def _tiny_sidecar(values, table_ids, rows, n, m):
    """One row bucket, k = 1, every element coded through `table_ids` (all -1:
    the reference decodes each element as ESC, 11 bits then 16 raw bits)."""
    bits = []
    for v in values:
        bits += [0] * 11 + [(v >> (15 - i)) & 1 for i in range(16)]
    bits += [0] * (-len(bits) % 64)
    words = np.array([int("".join(map(str, bits[i:i + 64])), 2) for i in range(0, len(bits), 64)], dtype=np.uint64)
    total = len(values)
    return {
        "bitstream_u64": words, "decode_syms_u16": np.zeros((1, 2048), np.uint16),
        "decode_lens_u8": np.zeros((1, 1024), np.uint8),
        "bucket_table_i32": np.array([table_ids], dtype=np.int32),
        "bucket_col_start_i32": np.array([0], np.int32), "bucket_col_len_i32": np.array([m], np.int32),
        "bucket_row_offsets_i32": np.array([0, len(rows)], np.int32), "row_indices_i32": np.array(rows, np.int32),
        "bucket_thread_startbit_u32": np.array([[0, 27 * total]], np.uint32),
        "bucket_bit_base_i64": np.array([0, 27 * total], np.int64),
    }


def _tiny_decode(sc, q, n, m, out=None):
    t = {k: torch.from_numpy(v.view(np.int64) if v.dtype == np.uint64 else
                             v.view(np.int16) if v.dtype == np.uint16 else
                             v.view(np.int32) if v.dtype == np.uint32 else v).to(DEV) for k, v in sc.items()}
    t["bitstream_u64"] = t["bitstream_u64"].view(torch.uint64)
    t["decode_syms_u16"] = t["decode_syms_u16"].view(torch.uint16)
    t["bucket_thread_startbit_u32"] = t["bucket_thread_startbit_u32"].view(torch.uint32)
    o = MPServe_cuda.huffman_decode_awq_int4_bucket(
        torch.from_numpy(q).to(DEV), t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"],
        t["bucket_table_i32"], t["bucket_col_start_i32"], t["bucket_col_len_i32"], t["bucket_row_offsets_i32"],
        t["row_indices_i32"], t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], n, m, 11, out=out)
    torch.cuda.synchronize()
    return o.view(torch.uint16).cpu().numpy()


def test_missing_table_decodes_as_esc_like_the_reference():
    """decode_huffman.cu:448-460: bucket_table -1 -> consume L bits, then 16 raw bits."""
    vals = [0x3F80, 0xBF80, 0x0001, 0xFFFF, 0x1234, 0x8000]
    n, m = 2, 3
    sc = _tiny_sidecar(vals, [-1] * 16, [0, 1], n, m)
    q = np.array([[0, 5, 15], [3, 8, 12]], np.uint8)
    read_status(torch.device(DEV))
    out = _tiny_decode(sc, q, n, m)
    assert out.reshape(-1).tolist() == vals
    assert np.array_equal(out, oracle.awq_decode(sc, q, n, m))
    assert read_status(torch.device(DEV)) == 0


def test_integrity_flags_bad_row_and_bad_table():
    from mpserve_amd._native import MPS_STATUS_BAD_ROW, MPS_STATUS_BAD_TABLE

    vals = [0x3F80, 0xBF80, 0x0001]
    q = np.zeros((2, 3), np.uint8)
    read_status(torch.device(DEV))
    sc = _tiny_sidecar(vals, [-1] * 16, [7], 2, 3)  # row 7 of a 2-row tensor
    _tiny_decode(sc, q, 2, 3, out=torch.zeros((2, 3), dtype=torch.bfloat16, device=DEV))
    assert read_status(torch.device(DEV)) & MPS_STATUS_BAD_ROW
    sc = _tiny_sidecar(vals, [5] + [-1] * 15, [0], 2, 3)  # table id 5 of a 1-table sidecar
    _tiny_decode(sc, q, 2, 3)
    assert read_status(torch.device(DEV)) & MPS_STATUS_BAD_TABLE


def test_no_buckets_is_a_no_op():
    bf16, q, sc = _inputs("empty", 8, 64, None)
    d = {k: v.to(DEV) for k, v in _build(bf16, q, sc, 64, False, 1024).items()}
    empty = {k: v[:0] if k in ("bucket_table_i32", "bucket_col_start_i32", "bucket_col_len_i32",
                               "bucket_thread_startbit_u32") else v for k, v in d.items()}
    empty["bucket_row_offsets_i32"] = d["bucket_row_offsets_i32"][:1]
    empty["bucket_bit_base_i64"] = d["bucket_bit_base_i64"][:1]
    out = torch.full((8, 64), 7.0, dtype=torch.bfloat16, device=DEV)
    MPServe_cuda.huffman_decode_awq_int4_bucket(
        q.to(DEV), empty["bitstream_u64"], empty["decode_syms_u16"], empty["decode_lens_u8"],
        empty["bucket_table_i32"], empty["bucket_col_start_i32"], empty["bucket_col_len_i32"],
        empty["bucket_row_offsets_i32"], empty["row_indices_i32"], empty["bucket_thread_startbit_u32"],
        empty["bucket_bit_base_i64"], 8, 64, 11, out=out)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_plan_decodes_mixed_layouts_in_one_launch():
    """AwqDecodePlan: every bucket of four tensors (both layouts, k 256 and 1024) in one launch."""
    print("[awq] plan over mixed layouts", flush=True)
    items, srcs = [], []
    for j, (n, m, group, by_scale) in enumerate([(256, 512, 128, True), (128, 1024, None, False),
                                                 (64, 256, 64, False), (512, 256, 128, True)]):
        w = make_awq_weight(n, m, group, seed=500 + j, device=DEV)
        sc = _build(w.bf16, w.int4_u8, w.scale_u16, 1024 if j % 2 else 256, by_scale, 16)
        items.append((w.int4_u8, sc, torch.empty((n, m), dtype=torch.bfloat16, device=DEV)))
        srcs.append(w.bf16)
    plan = awq.AwqDecodePlan(items)
    # k = 256 tensors: runs of same-scale buckets share a workgroup, so fewer records than buckets
    assert 0 < plan.info()["work_items"] < sum(sc["bucket_table_i32"].shape[0] for _, sc, _ in items)
    read_status(torch.device(DEV))
    for _ in range(2):  # replays give the same outputs
        for o in plan.outputs:
            o.zero_()
        plan.decode()
        torch.cuda.synchronize()
        for o, s in zip(plan.outputs, srcs):
            assert torch.equal(o.view(torch.uint16), s.view(torch.uint16))
    assert plan.read_status() == 0
    plan.close()
    assert awq.AwqDecodePlan([]).decode() == []


def test_truncated_bitstream_and_wild_start_bits_flag_desync_without_faults():
    """A bitstream cut short, or start bits past its end, must only raise the
    desync flag: every read stays inside the bitstream and every store inside out."""
    from mpserve_amd._native import MPS_STATUS_DESYNC

    bf16, q, sc = _inputs("trunc", 64, 512, 128)
    d = {k: v.to(DEV) for k, v in _build(bf16, q, sc, 256, True, 16).items()}
    for what in ("truncate", "wild_start"):
        t = dict(d)
        if what == "truncate":
            t["bitstream_u64"] = d["bitstream_u64"][: d["bitstream_u64"].numel() // 2].clone()
        else:
            sb = d["bucket_thread_startbit_u32"].clone()
            sb.view(torch.int32)[:, 5] = -16  # 0xFFFFFFF0: far past the end
            t["bucket_thread_startbit_u32"] = sb
        read_status(torch.device(DEV))
        out = MPServe_cuda.huffman_decode_awq_int4_bucket_by_scale(
            q.to(DEV), t["bitstream_u64"], t["decode_syms_u16"], t["decode_lens_u8"], t["bucket_table_i32"],
            t["bucket_group_offsets_i32"], t["group_rows_i32"], t["group_col_start_i32"],
            t["bucket_thread_startbit_u32"], t["bucket_bit_base_i64"], 64, 512, 11, 128)
        torch.cuda.synchronize()
        assert out.shape == (64, 512)
        assert read_status(torch.device(DEV)) & MPS_STATUS_DESYNC, what


def _slab_counts(sc):
    """Per-lane element counts of the buckets the plan sends down the slab path:
    by-scale buckets of 8..1024 groups (one count per wave pair), row buckets of
    1..128 rows over P >= 4 blocks of 1024 columns (rows x P)."""
    if "bucket_group_offsets_i32" in sc:
        g = np.diff(sc["bucket_group_offsets_i32"].cpu().numpy().astype(np.int64))
        g = g[(g >= 8) & (g <= 1024)]
        return np.concatenate([g // 8 + (j < g % 8) for j in range(8)]) if g.size else g
    rows = np.diff(sc["bucket_row_offsets_i32"].cpu().numpy().astype(np.int64))
    cl = sc["bucket_col_len_i32"].cpu().numpy().astype(np.int64)
    ok = (rows >= 1) & (rows <= 128) & (cl % 1024 == 0) & (cl >= 4096)
    return (rows * (cl // 1024))[ok]


@pytest.mark.parametrize(
    "by_scale,n,m,cap,seed",
    [(True, 4096, 4096, 1024, 700), (True, 1024, 4096, 1024, 701), (True, 2048, 4096, 12, 702),
     (True, 14336, 4096, 1024, 703), (False, 2048, 4096, 1024, 721), (False, 512, 14336, 1024, 722),
     (False, 1024, 14336, 1024, 724)],
    ids=["q_4096", "kv_1024x4096", "cap12_partial_slabs", "gate_14336x4096", "rows_p4", "rows_p14_wrap",
         "rows_p14_1024"])
def test_plan_slab_path_matches_input_and_the_lane_path(by_scale, n, m, cap, seed, monkeypatch):
    """Sidecars with k = 1024 decode on the slab path (dword int4 loads, register
    transposes, 8-byte stores): by-scale with 128-column groups, and row buckets
    over P >= 4 blocks of 1024 columns (P % 4 == 0, or a step straddling two rows).
    Bit-exact to the input, equal to the per-lane path's output, status clean. The
    cases hold ESC keys, partial last slabs (by-scale group counts not a multiple
    of 8) and partial last steps (per-lane counts not a multiple of 4); the row
    buckets of a lone tensor are split into row ranges started from lane
    checkpoints."""
    print(f"[awq] slab path {'by-scale' if by_scale else 'rows'} {n}x{m} cap {cap}", flush=True)
    w = make_awq_weight(n, m, 128 if by_scale else None, seed=seed, device=DEV)
    sc, st = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, 1024, cap, by_scale, with_stats=True)
    assert st["esc_collisions"] == 0
    counts = _slab_counts(sc)
    assert counts.size > 0
    if by_scale and cap == 12:
        assert (counts % 4 != 0).any()
    if not by_scale and m % 4096 != 0:
        assert (counts % 4 != 0).any()  # rows x 14: partial last steps
    if not by_scale or n * m >= 4096 * 4096:  # every row case here has ESC keys (6, 10 and 23)
        assert st["esc_keys"] > 0
    outs = {}
    for slab in ("1", "0"):
        monkeypatch.setenv("MPSERVE_AWQ_SLAB", slab)
        out = torch.empty((n, m), dtype=torch.bfloat16, device=DEV)
        plan = awq.AwqDecodePlan([(w.int4_u8, sc, out)])
        if slab == "1" and not by_scale:
            # a lone tensor's row buckets exceed total / (2 CUs): split into row ranges
            assert plan.info()["work_items"] > sc["bucket_table_i32"].shape[0]
        if slab == "1" and by_scale and cap == 12:
            # 12-group buckets of one scale are far below total / (2 CUs): runs of
            # them with identical table ids share a record and its tables
            assert plan.info()["work_items"] < sc["bucket_table_i32"].shape[0]
        plan.read_status()
        for _ in range(2):
            out.zero_()
            plan.decode()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16)), slab
        assert plan.read_status() == 0
        plan.close()
        outs[slab] = out
    assert torch.equal(outs["1"].view(torch.uint16), outs["0"].view(torch.uint16))


@pytest.mark.parametrize(
    "k,n,m,seed",
    [(256, 2048, 4096, 730), (512, 512, 14336, 731), (256, 512, 14336, 732), (256, 300, 1024, 733),
     (512, 96, 2048, 734)],
    ids=["k256_p16", "k512_p28", "k256_p56", "k256_p4", "k512_p4"])
def test_plan_rows_k256_k512_ranges_side_by_side(k, n, m, seed, monkeypatch):
    """Row buckets with k = 256 or 512 and P = col_len / k a multiple of 4 decode on
    the slab path at stride k, 1024 / k row ranges side by side in a record (from
    a full set of lane checkpoints; a last record may hold fewer ranges than
    groups). Bit-exact to the input and equal to the per-lane path's output."""
    print(f"[awq] rows side by side k {k} {n}x{m}", flush=True)
    w = make_awq_weight(n, m, None, seed=seed, device=DEV)
    sc, st = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, k, 1024, False, with_stats=True)
    assert st["esc_collisions"] == 0
    outs = {}
    for slab in ("1", "0"):
        monkeypatch.setenv("MPSERVE_AWQ_SLAB", slab)
        out = torch.empty((n, m), dtype=torch.bfloat16, device=DEV)
        plan = awq.AwqDecodePlan([(w.int4_u8, sc, out)])
        plan.read_status()
        for _ in range(2):
            out.zero_()
            plan.decode()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16)), slab
        assert plan.read_status() == 0
        plan.close()
        outs[slab] = out
    assert torch.equal(outs["1"].view(torch.uint16), outs["0"].view(torch.uint16))
    # the op: whole buckets on the first call, the sidecar's cached plan from the second
    monkeypatch.setenv("MPSERVE_AWQ_SLAB", "1")
    read_status(torch.device(DEV))
    for _ in range(3):
        got = _op_call(sc, w, n, m, None)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.uint16), w.bf16.view(torch.uint16))
    assert read_status(torch.device(DEV)) == 0


@pytest.mark.parametrize(
    "k,n,m,cap,seed",
    [(256, 4096, 4096, 1024, 750), (512, 1024, 4096, 1024, 751), (256, 2048, 4096, 201, 752),
     (512, 4096, 14336, 1024, 753), (256, 512, 4096, 12, 754)],
    ids=["k256_q", "k512_kv", "k256_cap201", "k512_down", "k256_cap12_runs"])
def test_plan_by_scale_k256_k512_slab_ranges(k, n, m, cap, seed, monkeypatch):
    """By-scale buckets with k = 256 or 512 (and at least 32 slabs) decode on the slab
    path in ranges of at most 128 slabs (k / 128 groups each), 1024 / k ranges side
    by side in a record, from a full set of lane checkpoints. Group counts that are
    not a multiple of k / 128 leave partial last slabs (cap 201); small buckets (cap
    12) stay on the per-lane path in same-scale runs. Bit-exact to the input, equal
    to the per-lane path's output."""
    print(f"[awq] by-scale slab ranges k {k} {n}x{m} cap {cap}", flush=True)
    w = make_awq_weight(n, m, 128, seed=seed, device=DEV)
    sc = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, k, cap, True)
    outs = {}
    for slab in ("1", "0"):
        monkeypatch.setenv("MPSERVE_AWQ_SLAB", slab)
        out = torch.empty((n, m), dtype=torch.bfloat16, device=DEV)
        plan = awq.AwqDecodePlan([(w.int4_u8, sc, out)])
        plan.read_status()
        for _ in range(2):
            out.zero_()
            plan.decode()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16)), slab
        assert plan.read_status() == 0
        plan.close()
        outs[slab] = out
    assert torch.equal(outs["1"].view(torch.uint16), outs["0"].view(torch.uint16))
    # the op: whole buckets on the first call, the sidecar's cached plan from the second
    monkeypatch.setenv("MPSERVE_AWQ_SLAB", "1")
    read_status(torch.device(DEV))
    for _ in range(3):
        got = _op_call(sc, w, n, m, 128)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.uint16), w.bf16.view(torch.uint16))
    assert read_status(torch.device(DEV)) == 0


@pytest.mark.parametrize("by_scale", [False, True])
def test_side_by_side_ranges_with_corrupt_sidecars(by_scale, monkeypatch):
    """k = 256 plans whose buckets would run ranges side by side, over corrupt
    sidecars: a row index out of range (the checkpoint walk stops and the bucket
    keeps its per-lane record), a table id out of range, shifted start bits. The
    flags are raised and nothing is written outside the output."""
    monkeypatch.setenv("MPSERVE_AWQ_SLAB", "1")
    n, m = (512, 4096) if by_scale else (256, 4096)
    w = make_awq_weight(n, m, 128 if by_scale else None, seed=760 + by_scale, device=DEV)
    sc = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, 256, 1024, by_scale)
    rows_key = "group_rows_i32" if by_scale else "row_indices_i32"
    guard = 4096
    for what, flag_bit in (("row", 0x2), ("table", 0x4), ("start", 0x8)):
        bad = {key: v.clone() for key, v in sc.items()}
        if what == "row":
            bad[rows_key][3] = n + 1000
        elif what == "table":
            bad["bucket_table_i32"][0, 5] = 10 ** 8
        else:
            bad["bucket_thread_startbit_u32"].view(torch.int32)[0, 7] += 3  # (no uint32 add on the GPU)
        buf = torch.zeros(n * m + 2 * guard, dtype=torch.bfloat16, device=DEV)
        out = buf[guard:guard + n * m].view(n, m)
        plan = awq.AwqDecodePlan([(w.int4_u8, bad, out)])
        plan.read_status()
        plan.decode()
        st = plan.read_status()
        plan.close()
        torch.cuda.synchronize()
        assert st & flag_bit, (what, st)
        g = buf.view(torch.uint16)
        assert int((g[:guard] != 0).sum()) == 0 and int((g[guard + n * m:] != 0).sum()) == 0, what


def test_plan_mixes_both_range_kinds(monkeypatch):
    """One plan over a k = 1024 row tensor (its buckets split into row ranges) and
    a k = 256 row tensor (ranges side by side) launches the kernel with both
    range paths; both decode bit-exact."""
    monkeypatch.setenv("MPSERVE_AWQ_SLAB", "1")
    a = make_awq_weight(1024, 4096, None, seed=740, device=DEV)
    b = make_awq_weight(512, 4096, None, seed=741, device=DEV)
    sa = awq.build_awq_sidecar(a.bf16, a.int4_u8, a.scale_u16, 11, 1024, 1024, False)
    sb = awq.build_awq_sidecar(b.bf16, b.int4_u8, b.scale_u16, 11, 256, 1024, False)
    oa = torch.empty((1024, 4096), dtype=torch.bfloat16, device=DEV)
    ob = torch.empty((512, 4096), dtype=torch.bfloat16, device=DEV)
    plan = awq.AwqDecodePlan([(a.int4_u8, sa, oa), (b.int4_u8, sb, ob)])
    plan.read_status()
    plan.decode()
    torch.cuda.synchronize()
    assert torch.equal(oa.view(torch.uint16), a.bf16.view(torch.uint16))
    assert torch.equal(ob.view(torch.uint16), b.bf16.view(torch.uint16))
    assert plan.read_status() == 0
    plan.close()


def _op_call(sc, w, n, m, group, out=None):
    if "bucket_group_offsets_i32" in sc:
        return MPServe_cuda.huffman_decode_awq_int4_bucket_by_scale(
            w.int4_u8, sc["bitstream_u64"], sc["decode_syms_u16"], sc["decode_lens_u8"], sc["bucket_table_i32"],
            sc["bucket_group_offsets_i32"], sc["group_rows_i32"], sc["group_col_start_i32"],
            sc["bucket_thread_startbit_u32"], sc["bucket_bit_base_i64"], n, m, 11, group, out=out)
    return MPServe_cuda.huffman_decode_awq_int4_bucket(
        w.int4_u8, sc["bitstream_u64"], sc["decode_syms_u16"], sc["decode_lens_u8"], sc["bucket_table_i32"],
        sc["bucket_col_start_i32"], sc["bucket_col_len_i32"], sc["bucket_row_offsets_i32"], sc["row_indices_i32"],
        sc["bucket_thread_startbit_u32"], sc["bucket_bit_base_i64"], n, m, 11, out=out)


def test_plan_run_with_a_bad_group_row():
    """A by-scale plan takes a run of buckets with identical table ids into one
    record, and the run's later buckets set up wave by wave. A group row out of
    range in such a bucket flags MPS_STATUS_BAD_ROW, no write leaves the output
    (guards on both sides), and every element outside that bucket decodes exactly."""
    from mpserve_amd._native import MPS_STATUS_BAD_ROW

    n, m = 2048, 4096
    w = make_awq_weight(n, m, 128, seed=702, device=DEV)
    sc = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, 1024, 12, True)
    tab = sc["bucket_table_i32"].cpu().numpy()
    goff = sc["bucket_group_offsets_i32"].cpu().numpy().astype(np.int64)
    ng = np.diff(goff)
    same = np.concatenate([[False], (tab[1:] == tab[:-1]).all(1)])
    # the second bucket of a run: same tables as the one before it, which starts the run
    second = [b for b in range(2, len(tab)) if same[b] and not same[b - 1] and ng[b] >= 8 and ng[b - 1] >= 8]
    assert second, "no same-table runs"
    b = second[len(second) // 2]
    bad = dict(sc)
    rows = sc["group_rows_i32"].clone()
    rows[int(goff[b]) + 3] = n + 1000
    bad["group_rows_i32"] = rows
    guard = 4096
    buf = torch.zeros(n * m + 2 * guard, dtype=torch.bfloat16, device=DEV)
    out = buf[guard:guard + n * m].view(n, m)
    plan = awq.AwqDecodePlan([(w.int4_u8, bad, out)])
    assert plan.info()["work_items"] < len(tab)  # runs share records
    plan.read_status()
    plan.decode()
    torch.cuda.synchronize()
    assert plan.read_status() & MPS_STATUS_BAD_ROW
    assert bool((buf[:guard] == 0).all()) and bool((buf[guard + n * m:] == 0).all())
    keep = torch.ones((n, m), dtype=torch.bool, device=DEV)
    for r, c in zip(sc["group_rows_i32"][goff[b]:goff[b + 1]].tolist(),
                    sc["group_col_start_i32"][goff[b]:goff[b + 1]].tolist()):
        keep[r, c:c + 128] = False
    assert torch.equal(out.view(torch.int16)[keep], w.bf16.view(torch.int16)[keep])


def test_op_plan_cache_alternating_sidecars():
    """The AWQ decode ops keep one plan per sidecar with k = 1024 (by-scale with
    128-column groups, or row buckets) from their second call on, so its buckets take
    the slab path: sidecars of both layouts
    alternated through the ops decode bit-exact on every call; an output that is
    not 8-byte aligned takes the direct kernel; an in-place rewrite of a tensor
    drops its sidecar's plan until it is seen twice again."""
    from mpserve_amd import awq as awq_mod
    from mpserve_amd import mpserve_cuda as mc

    print("[awq] op plan cache", flush=True)
    mc.clear_decode_plans()
    cases = []
    for n, m, group, by_scale, seed in ((2048, 4096, 128, True, 710), (512, 4096, None, False, 711)):
        w = make_awq_weight(n, m, group, seed=seed, device=DEV)
        sc = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, 1024, 1024, by_scale)
        cases.append((sc, w, n, m, group or m))
    read_status(torch.device(DEV))
    for call in range(4):
        for sc, w, n, m, group in cases:
            out = _op_call(sc, w, n, m, group)
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16)), f"call {call}"
        assert read_status(torch.device(DEV)) == 0
    cache = awq_mod._plan_cache()
    assert len(cache) == 2 and all(e.plan is not None for e in cache._entries.values())
    sc, w, n, m, group = cases[0]
    buf = torch.zeros(n * m + 1, dtype=torch.bfloat16, device=DEV)
    out = _op_call(sc, w, n, m, group, out=buf[1:])  # 2-byte offset: the direct kernel
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16).reshape(-1))
    w.int4_u8.copy_(w.int4_u8.clone())  # same bytes, new version
    out = _op_call(sc, w, n, m, group)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16))
    assert sum(e.plan is None for e in cache._entries.values()) == 1
    assert read_status(torch.device(DEV)) == 0
    mc.clear_decode_plans()
    assert len(cache) == 0


def test_plan_queue_every_record_on_every_launch_replay_and_two_streams():
    """An AWQ plan's workgroups take their records from a work queue in the plan's
    memory, which each launch's last workgroup resets. Every launch, every replay of
    a graph that captured one, and two launches of the plan on two streams at once
    (each stream with its own queue) decode every record."""
    from mpserve_amd import _native

    print("[awq] plan queue: launches, graph replays, two streams", flush=True)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    shapes = [(4096, 4096, 1024), (4096, 4096, 1024), (1024, 4096, 256), (4096, 4096, 256)]
    srcs, descs, sizes = [], [], []
    for j, (n, m, k) in enumerate(shapes):
        w = make_awq_weight(n, m, 128, seed=720 + j, device=DEV)
        sc = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, k, 1024, True)
        srcs.append(w)
        descs.append(sc)
        sizes.append(n * m)
    total = sum(sizes)
    flat = [torch.empty(total, dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    outs, off = [], 0
    for (n, m, _), sz in zip(shapes, sizes):
        outs.append(flat[0][off:off + sz].view(n, m))
        off += sz
    plan = awq.AwqDecodePlan([(w.int4_u8, sc, o) for w, sc, o in zip(srcs, descs, outs)])
    assert plan.info()["work_items"] > 2 * cus

    def check(buf, tag):
        torch.cuda.synchronize()
        o = 0
        for j, (w, sz) in enumerate(zip(srcs, sizes)):
            assert torch.equal(buf[o:o + sz].view(torch.uint16), w.bf16.view(torch.uint16).reshape(-1)), \
                f"{tag}: tensor {j}"
            o += sz

    plan.read_status()
    for rep in range(3):
        flat[0].fill_(float("nan"))
        plan.decode()
        check(flat[0], f"launch {rep}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.decode()
    for rep in range(3):
        flat[0].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        check(flat[0], f"replay {rep}")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rnd in range(3):
        for f in flat:
            f.fill_(float("nan"))
        for st in streams:
            st.wait_stream(torch.cuda.current_stream())
        for f, st in zip(flat, streams):
            _native.check(_native.lib().mps_awq_plan_decode_into(plan._plan, ctypes.c_void_p(f.data_ptr()),
                                                                 ctypes.c_void_p(st.cuda_stream)))
        for st in streams:
            torch.cuda.current_stream().wait_stream(st)
        for s_i, f in enumerate(flat):
            check(f, f"round {rnd}, stream {s_i}")
    assert plan.read_status() == 0
    assert read_status(torch.device(DEV)) == 0
    plan.close()


@pytest.mark.parametrize("n,m,k,cap,by_scale,seed", [
    (256, 1024, 1024, 3, True, 730),    # every bucket <= 3 groups: at most 384 elements for 1024 lanes
    (512, 512, 1024, 2, True, 731),     # buckets of 1-2 groups; many tensors' worth of tiny records
    (8, 96, 1024, 1024, False, 732),    # a row-bucket tensor of 768 elements
])
def test_plan_tiny_buckets_look_codes_up_in_the_global_tables(n, m, k, cap, by_scale, seed):
    """Buckets with no more elements than lanes (k = 1024) code one element a lane:
    the plan decodes them without staging their tables in LDS. Bit-exact to the
    input, status clear; a group row out of range in one tiny bucket is flagged,
    nothing is written outside the output, and every other element decodes."""
    from mpserve_amd._native import MPS_STATUS_BAD_ROW

    print(f"[awq] tiny buckets n={n} m={m} k={k} cap={cap} by_scale={by_scale}", flush=True)
    w = make_awq_weight(n, m, 128 if by_scale else None, seed=seed, device=DEV)
    sc, st = awq.build_awq_sidecar(w.bf16, w.int4_u8, w.scale_u16, 11, k, cap, by_scale, with_stats=True)
    assert st["esc_collisions"] == 0
    offs = (sc["bucket_group_offsets_i32"] if by_scale else sc["bucket_row_offsets_i32"]).cpu().numpy().astype(np.int64)
    cols = 128 if by_scale else sc["bucket_col_len_i32"].cpu().numpy().astype(np.int64)
    elems = np.diff(offs) * cols
    assert (elems <= k).mean() > 0.5, "the case should be mostly tiny buckets"
    out = torch.empty((n, m), dtype=torch.bfloat16, device=DEV)
    plan = awq.AwqDecodePlan([(w.int4_u8, sc, out)])
    plan.read_status()
    for _ in range(2):
        out.fill_(float("nan"))
        plan.decode()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16))
    assert plan.read_status() == 0
    plan.close()
    if not by_scale:
        return
    # a group row out of range in the first tiny bucket with two or more groups
    b = int(next(i for i in range(len(elems)) if elems[i] <= k and offs[i + 1] - offs[i] >= 2))
    bad = dict(sc)
    rows = sc["group_rows_i32"].clone()
    rows[int(offs[b]) + 1] = n + 77
    bad["group_rows_i32"] = rows
    guard = 4096
    buf = torch.zeros(n * m + 2 * guard, dtype=torch.bfloat16, device=DEV)
    out = buf[guard:guard + n * m].view(n, m)
    plan = awq.AwqDecodePlan([(w.int4_u8, bad, out)])
    plan.read_status()
    plan.decode()
    torch.cuda.synchronize()
    assert plan.read_status() & MPS_STATUS_BAD_ROW
    assert bool((buf[:guard] == 0).all()) and bool((buf[guard + n * m:] == 0).all())
    keep = torch.ones((n, m), dtype=torch.bool, device=DEV)
    r, c = int(sc["group_rows_i32"][int(offs[b]) + 1]), int(sc["group_col_start_i32"][int(offs[b]) + 1])
    keep[r, c:c + 128] = False
    assert torch.equal(out.view(torch.int16)[keep], w.bf16.view(torch.int16)[keep])
    plan.close()
