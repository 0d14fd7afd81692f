"""HIP decode parity: MPServe_cuda.huffman_decode_fp8 vs the CPU oracle and the input weights.

Integer path, so the bar is bit-exact equality of the BF16 bit patterns.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.helpers import decode_args, synth, to_torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _gpu_decode(sc, q):
    import MPServe_cuda

    sc_t = to_torch(sc, DEV)
    q_t = torch.from_numpy(np.ascontiguousarray(q)).to(DEV)
    out = MPServe_cuda.huffman_decode_fp8(*decode_args(sc_t, q_t))
    torch.cuda.synchronize()
    return out.view(torch.uint16).cpu().numpy()


def _status():
    from mpserve_amd.mpserve_cuda import read_status

    return read_status(torch.device(DEV))


@pytest.mark.parametrize("n,m,k,seed", [
    (4096, 4096, 1024, 0),   # config 1 shape, compress default k
    (1, 1, 1, 1),
    (3, 5, 7, 2),
    (7, 100, 1024, 3),       # col_len < k_eff: lanes wrap several rows per step
    (64, 256, 64, 4),
    (300, 513, 1024, 5),
    (129, 1000, 256, 6),
    (40, 3000, 1000, 7),
    (1024, 4096, 1024, 8),   # k_proj / v_proj shape of the 8B layer
    (256, 14336, 1024, 9),   # down_proj row length
])
def test_decode_roundtrip_per_row(n, m, k, seed):
    bf, q, sc_u16 = synth(n, m, seed=seed)
    sc = oracle.encode(bf, q, sc_u16, 7, k)
    _status()
    got = _gpu_decode(sc, q)
    ref = oracle.decode(sc, q, n, m, 7, nthreads=8)
    assert np.array_equal(ref, bf)
    assert np.array_equal(got, bf), f"mismatches: {(got != bf).sum()}"
    assert _status() == 0


@pytest.mark.parametrize("n,m,seed", [
    (130, 1024, 100),    # P = 1 column block per row -> G = 1
    (96, 2048, 101),     # P = 2 -> G = 2
    (70, 3072, 102),     # P = 3 -> G = 1
    (200, 4096, 103),    # P = 4 -> G = 4
    (40, 7168, 104),     # P = 7 -> G = 7
    (33, 8192, 105),     # P = 8 -> G = 8
    (20, 14336, 106),    # P = 14 -> G = 7 (down_proj rows)
    (9, 16384, 107),     # P = 16 -> G = 8
    (3, 28672, 108),     # P = 28 -> G = 7 (70B down_proj rows)
])
def test_decode_k1024_block_sizes(n, m, seed):
    """The k = 1024 path walks a row in blocks of G | P elements; every G it picks."""
    bf, q, sc_u16 = synth(n, m, seed=seed)
    sc = oracle.encode(bf, q, sc_u16, 7, 1024)
    _status()
    got = _gpu_decode(sc, q)
    assert np.array_equal(got, bf), f"mismatches: {(got != bf).sum()}"
    assert _status() == 0


@pytest.mark.parametrize("n,m,seed", [(40, 2048, 110), (48, 4096, 111), (30, 7168, 112), (17, 8192, 113),
                                      (12, 3072, 114)])
def test_decode_k1024_esc(n, m, seed):
    """ESC buckets on the k = 1024 path: lossless, and the lane ends where the next begins."""
    bf, q, scales = _esc_inputs(n, m, seed)
    sc, stats = oracle.encode(bf, q, scales, 7, 1024, with_stats=True)
    assert stats["esc_keys"] >= 1 and stats["esc_elements"] > 0 and stats["esc_collisions"] == 0
    _status()
    got = _gpu_decode(sc, q)
    assert np.array_equal(got, bf), f"mismatches: {(got != bf).sum()}"
    assert _status() == 0


@pytest.mark.parametrize("n,m,seed,esc", [
    (1, 1024, 140, False),     # P = 1, one row: one partial group
    (5, 1024, 141, False),     # P = 1: a group spans four rows, the last holds one
    (3, 2048, 142, False),     # P = 2: six slabs, the last group half full
    (66, 2048, 143, False),
    (7, 3072, 144, False),     # P = 3: groups straddle rows at every block offset, tail of one
    (127, 3072, 145, False),
    (128, 1024, 146, False),   # the most rows a k = 1024 bucket takes
    (9, 1024, 147, True),      # ESC codes with P = 1
    (11, 3072, 148, True),     # ESC codes with P = 3, tail of one
])
def test_decode_k1024_small_p_slab(n, m, seed, esc):
    """k = 1024 buckets with P = col_len / 1024 < 4 take the slab path with a
    per-lane row walk (slab i is row i / P, block i % P): one scale key, so a
    bucket holds every row (up to 128) and its last group is partial unless
    4 | rows * P. Bit-exact through the op and through a plan, which splits the
    larger buckets into row ranges; the status word stays clear."""
    if esc:
        bf, q, scales = _esc_inputs(n, m, seed)
    else:
        bf, q, sc_u16 = synth(n, m, seed=seed)
        scales = sc_u16[:1].copy()
    sc, stats = oracle.encode(bf, q, scales, 7, 1024, with_stats=True)
    assert (stats["esc_keys"] >= 1) == esc
    _status()
    got = _gpu_decode(sc, q)
    assert np.array_equal(got, bf), f"mismatches: {(got != bf).sum()}"
    assert _status() == 0
    outs, info, status = _plan_decode([(bf, q, sc)])
    assert np.array_equal(outs[0], bf), f"plan mismatches: {(outs[0] != bf).sum()}"
    assert status == 0
    if n >= 66:
        assert info["work_items"] > sc["bucket_table_i32"].shape[0]  # row ranges from lane checkpoints


@pytest.mark.parametrize("n,m,k,seed,esc", [
    (200, 4096, 256, 120, False),   # P = 16, per-row scales
    (100, 1536, 256, 121, False),   # P = 6: groups straddle rows
    (64, 3584, 512, 122, False),    # P = 7
    (130, 2048, 512, 123, False),   # P = 4
    (40, 2048, 256, 124, True),     # ESC entries, P = 8
    (30, 1792, 256, 125, True),     # ESC entries, P = 7
    (50, 768, 256, 126, False),     # P = 3: groups span two rows
    (33, 1024, 512, 127, False),    # P = 2
    (9, 512, 512, 128, False),      # P = 1: groups span four rows
    (120, 1280, 256, 129, "one_key"),  # P = 5, one 120-row bucket: ranges side by side
    (128, 768, 256, 130, "one_key"),   # P = 3, ranges side by side
    (101, 512, 512, 131, "one_key"),   # P = 1, two ranges an item
    (26, 512, 256, 132, True),      # ESC entries, P = 2
    (13, 768, 512, 133, True),      # ESC entries, P = 1.5 -> k_eff 512 does not divide: not the slab path
])
def test_decode_slab_k256_k512(n, m, k, seed, esc):
    """Buckets with k = 256 or 512 substreams take the slab path (groups of four
    elements across 4 x 4 lane transposes) for every P = col_len / k: groups in one
    row (4 | P), straddling two rows (P > 4), or spanning two to four rows (P < 4);
    as the single op and inside a plan (whole buckets and row ranges side by side)."""
    if esc is True:
        bf, q, scales = _esc_inputs(n, m, seed)
        sc, stats = oracle.encode(bf, q, scales, 7, k, with_stats=True)
        assert stats["esc_keys"] >= 1 and stats["esc_elements"] > 0
    else:
        bf, q, scales = synth(n, m, seed=seed)
        sc = oracle.encode(bf, q, scales[:1].copy() if esc == "one_key" else scales, 7, k)
    _status()
    got = _gpu_decode(sc, q)
    assert np.array_equal(got, bf), f"mismatches: {(got != bf).sum()}"
    assert _status() == 0
    outs, _, status = _plan_decode([(bf, q, sc)])
    assert np.array_equal(outs[0], bf), f"plan mismatches: {(outs[0] != bf).sum()}"
    assert status == 0


def test_decode_scalar_scale_many_buckets():
    n, m = 1000, 640
    bf, q, sc_u16 = synth(n, m, seed=11)
    sc = oracle.encode(bf, q, sc_u16[:1].copy(), 7, 512)
    assert sc["bucket_table_i32"].shape[0] == 8  # ceil(1000/128) buckets of one scale
    assert np.array_equal(_gpu_decode(sc, q), bf)


def test_decode_block2d_scales():
    n, m = 256, 384
    bf, q, _ = synth(n, m, seed=12)
    rng = np.random.default_rng(12)
    scales = rng.integers(0x2000, 0x2010, size=(4, 3), dtype=np.uint16)  # 64x128 blocks
    sc = oracle.encode(bf, q, scales, 7, 1024)
    assert (sc["bucket_col_len_i32"] == 128).all() and sc["row_indices_i32"].size == n * 3
    got = _gpu_decode(sc, q)
    assert np.array_equal(got, bf)


def _esc_inputs(n, m, seed, with_collision=False):
    """One (scale, fp8) key carrying > 128 distinct BF16 symbols -> ESC codes."""
    rng = np.random.default_rng(seed)
    bf = rng.integers(0x3C00, 0x3C00 + 600, size=(n, m)).astype(np.uint16)
    # a skewed head so that the kept set is well defined
    head = rng.random((n, m)) < 0.5
    bf[head] = (0x3C00 + rng.integers(0, 20, size=int(head.sum()))).astype(np.uint16)
    if with_collision:
        bf.flat[rng.choice(bf.size, 3, replace=False)] = 0  # esc_sym will be 0x0000
    q = np.full((n, m), 0x38, dtype=np.uint8)
    q[:, ::7] = 0x39  # a second, small key
    return bf, q, np.array([0x1C00], dtype=np.uint16)


def test_decode_esc_lossless():
    n, m = 200, 512
    bf, q, scales = _esc_inputs(n, m, 21)
    sc, stats = oracle.encode(bf, q, scales, 7, 1024, with_stats=True)
    assert stats["esc_keys"] >= 1 and stats["esc_elements"] > 0 and stats["esc_collisions"] == 0
    got = _gpu_decode(sc, q)
    assert np.array_equal(got, bf)
    # the reference kernel ignores ESC (decode_huffman.cu:348-353): it loses those elements
    ref_kernel = oracle.decode(sc, q, n, m, 7, mode=oracle.MODE_REFERENCE_KERNEL)
    assert not np.array_equal(ref_kernel, bf)


def test_decode_esc_collision_matches_oracle():
    """esc_sym equal to a rare data symbol: the builder emits an ESC code without
    raw bits (build_huffman.cu:850-864). Both decoders read 16 raw bits there;
    the GPU must still agree with the oracle element for element."""
    n, m = 120, 600
    bf, q, scales = _esc_inputs(n, m, 22, with_collision=True)
    sc, stats = oracle.encode(bf, q, scales, 7, 1024, with_stats=True)
    assert stats["esc_collisions"] > 0
    got = _gpu_decode(sc, q)
    ref = oracle.decode(sc, q, n, m, 7)
    assert np.array_equal(got, ref)
    # the ambiguous code loses those elements (the lane usually re-synchronises
    # within a few codes, so the lane-end check need not fire)
    assert not np.array_equal(got, bf)
    _status()


def test_decode_reference_kernel_equivalence_on_wellformed():
    """Where the reference kernel is well defined (no ESC, col_len >= k), the
    lossless decode and the reference kernel's walk give the same output."""
    n, m = 512, 2048
    bf, q, sc_u16 = synth(n, m, seed=31)
    sc = oracle.encode(bf, q, sc_u16, 7, 1024)
    ref_kernel = oracle.decode(sc, q, n, m, 7, mode=oracle.MODE_REFERENCE_KERNEL)
    assert np.array_equal(ref_kernel, bf)
    assert np.array_equal(_gpu_decode(sc, q), ref_kernel)


def test_decode_safetensors_dtype_views():
    """Sidecar as stored by the compress script (int64/int16/int32 casts) and
    viewed back the way apply() does (mpserve_vllm_fp8_huffman.py:457-472)."""
    import MPServe_cuda

    n, m = 333, 1024
    bf, q, sc_u16 = synth(n, m, seed=41)
    sc = oracle.encode(bf, q, sc_u16, 7, 1024)
    st = to_torch(sc, DEV)
    stored = {
        "bitstream": st["bitstream_u64"].to(torch.int64), "syms": st["decode_syms_u16"].to(torch.int16),
        "sb": st["bucket_thread_startbit_u32"].to(torch.int32),
    }
    q_t = torch.from_numpy(q).to(DEV)
    out = MPServe_cuda.huffman_decode_fp8(
        q_t, stored["bitstream"].view(torch.uint64), stored["syms"].view(torch.uint16), st["decode_lens_u8"],
        st["bucket_table_i32"], st["bucket_col_start_i32"], st["bucket_col_len_i32"],
        st["bucket_row_offsets_i32"], st["row_indices_i32"], stored["sb"].view(torch.uint32),
        st["bucket_bit_base_i64"], n, m, 7)
    assert np.array_equal(out.view(torch.uint16).cpu().numpy(), bf)


def test_decode_on_side_stream_and_out_buffer():
    import MPServe_cuda

    n, m = 700, 2048
    bf, q, sc_u16 = synth(n, m, seed=51)
    sc_t = to_torch(oracle.encode(bf, q, sc_u16, 7, 1024), DEV)
    q_t = torch.from_numpy(q).to(DEV)
    side = torch.cuda.Stream()
    buf = torch.full((n * m,), float("nan"), dtype=torch.bfloat16, device=DEV)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        MPServe_cuda.huffman_decode_fp8(*decode_args(sc_t, q_t), out=buf)
    torch.cuda.current_stream().wait_stream(side)
    assert np.array_equal(buf.view(torch.uint16).cpu().numpy().reshape(n, m), bf)


def test_plan_decodes_many_tensors():
    from mpserve_amd.decode import DecodePlan

    shapes = [(256, 1024, 1024), (64, 4096, 1024), (300, 700, 512), (5, 9, 3)]
    items, refs = [], []
    for i, (n, m, k) in enumerate(shapes):
        bf, q, sc_u16 = synth(n, m, seed=60 + i)
        sc_t = to_torch(oracle.encode(bf, q, sc_u16, 7, k), DEV)
        items.append((torch.from_numpy(q).to(DEV), sc_t))
        refs.append(bf)
    outs = [torch.empty((q.shape[0], q.shape[1]), dtype=torch.bfloat16, device=DEV) for q, _ in items]
    plan = DecodePlan([(q, sc, o) for (q, sc), o in zip(items, outs)])
    for _ in range(2):
        plan.decode()
        torch.cuda.synchronize()
        for o, r in zip(outs, refs):
            assert np.array_equal(o.view(torch.uint16).cpu().numpy(), r)
    assert plan.read_status() == 0


def test_plan_queue_hands_out_every_item_on_every_launch():
    """A plan with more work items than twice the CUs: each launch takes the items
    from a queue in the plan's memory, which the launch's last workgroup resets.
    Every launch, and every replay of a graph that captured one, decodes all items."""
    from mpserve_amd.decode import DecodePlan

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    shapes = [(512, 4096, 1024)] * 6 + [(64, 1024, 256)] * 8 + [(300, 700, 512)]
    items, refs = [], []
    for i, (n, m, k) in enumerate(shapes):
        bf, q, sc_u16 = synth(n, m, seed=90 + i)
        items.append((torch.from_numpy(q).to(DEV), to_torch(oracle.encode(bf, q, sc_u16, 7, k), DEV)))
        refs.append(bf)
    outs = [torch.empty((q.shape[0], q.shape[1]), dtype=torch.bfloat16, device=DEV) for q, _ in items]
    plan = DecodePlan([(q, sc, o) for (q, sc), o in zip(items, outs)])
    assert plan.info()["work_items"] > 2 * cus

    def check(tag):
        torch.cuda.synchronize()
        for j, (o, r) in enumerate(zip(outs, refs)):
            got = o.view(torch.uint16).cpu().numpy()
            assert np.array_equal(got, r), f"{tag}: tensor {j}, {(got != r).sum()} mismatches"

    for rep in range(3):
        for o in outs:
            o.zero_()
        plan.decode()
        check(f"launch {rep}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.decode()
    for rep in range(3):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        check(f"replay {rep}")
    assert plan.read_status() == 0


def test_integrity_flags_on_corrupt_sidecar():
    """Corrupt lane starts / row indices / table ids are flagged (writes are checked
    against the output's bounds in test_corrupt_sidecar_writes_stay_inside_out)."""
    import MPServe_cuda

    n, m = 256, 1024
    bf, q, sc_u16 = synth(n, m, seed=71)
    sc = oracle.encode(bf, q, sc_u16, 7, 1024)
    q_t = torch.from_numpy(q).to(DEV)

    bad = {k: v.copy() for k, v in sc.items()}
    bad["bucket_thread_startbit_u32"][0, 5] += 3
    out = MPServe_cuda.huffman_decode_fp8(*decode_args(to_torch(bad, DEV), q_t))
    assert _status() & 0x8

    bad = {k: v.copy() for k, v in sc.items()}
    bad["row_indices_i32"][3] = n + 1000
    MPServe_cuda.huffman_decode_fp8(*decode_args(to_torch(bad, DEV), q_t))
    assert _status() & 0x2

    bad = {k: v.copy() for k, v in sc.items()}
    bad["bucket_table_i32"][0, 10] = 10 ** 8
    MPServe_cuda.huffman_decode_fp8(*decode_args(to_torch(bad, DEV), q_t))
    assert _status() & 0x4
    assert out.shape == (n, m)


def _plan_decode(items):
    """Decode [(bf16 ref or None, fp8 u8 numpy, oracle sidecar)] in one plan;
    (outputs, plan info, the plan's status flags)."""
    from mpserve_amd.decode import DecodePlan

    dev_items = []
    for _, q, sc in items:
        q_t = torch.from_numpy(np.ascontiguousarray(q)).to(DEV)
        dev_items.append((q_t, to_torch(sc, DEV), torch.zeros(q.shape, dtype=torch.bfloat16, device=DEV)))
    plan = DecodePlan(dev_items)
    plan.decode()
    torch.cuda.synchronize()
    return [o.view(torch.uint16).cpu().numpy() for _, _, o in dev_items], plan.info(), plan.read_status()


@pytest.mark.parametrize("case", ["slab_p8", "slab_wrap_p14", "esc_k1024", "fast_k256", "fast_k512", "fast_k256_ragged",
                                  "mixed", "mixed_multi"])
def test_plan_splits_buckets_into_row_ranges(case):
    """A plan with few large buckets splits them into row ranges started from lane
    checkpoints; every range decodes bit-exact and ends where the next begins. A
    fast-path bucket with k = 256 or 512 runs 1024 / k of its ranges side by side
    in one work item (its other work-items would idle): fewer items than ranges,
    and with ragged rows the last item has fewer ranges than work-item groups."""
    if case == "slab_p8":       # 2 buckets of 128 rows x 8192 columns (one scale key)
        bf, q, sc = synth(256, 8192, seed=81)
        items = [(bf, q, oracle.encode(bf, q, sc[:1].copy(), 7, 1024))]
    elif case == "slab_wrap_p14":  # P = 14: groups straddle rows
        bf, q, sc = synth(128, 14336, seed=82)
        items = [(bf, q, oracle.encode(bf, q, sc[:1].copy(), 7, 1024))]
    elif case == "esc_k1024":
        bf, q, scales = _esc_inputs(48, 4096, 83)
        side, stats = oracle.encode(bf, q, scales, 7, 1024, with_stats=True)
        assert stats["esc_keys"] >= 1
        items = [(bf, q, side)]
    elif case == "fast_k256":   # k = 256 substreams, P = 8
        bf, q, sc = synth(300, 2048, seed=84)
        items = [(bf, q, oracle.encode(bf, q, sc[:1].copy(), 7, 256))]
    elif case == "fast_k512":   # k = 512, P = 8: two ranges an item
        bf, q, sc = synth(256, 4096, seed=89)
        items = [(bf, q, oracle.encode(bf, q, sc[:1].copy(), 7, 512))]
    elif case == "fast_k256_ragged":  # 10 rows, P = 128: five ranges of 2 rows, the second item holds one
        bf, q, sc = synth(10, 32768, seed=90)
        items = [(bf, q, oracle.encode(bf, q, sc[:1].copy(), 7, 256))]
    elif case == "mixed_multi":  # a multi-range bucket beside k = 1024 slab buckets
        a = synth(256, 8192, seed=91)
        b = synth(200, 2048, seed=92)
        items = [(a[0], a[1], oracle.encode(a[0], a[1], a[2][:1].copy(), 7, 1024)),
                 (b[0], b[1], oracle.encode(b[0], b[1], b[2][:1].copy(), 7, 256))]
    else:                       # a split tensor next to whole buckets and a generic-path tensor
        a = synth(256, 8192, seed=85)
        b = synth(64, 4096, seed=86)
        c = synth(40, 100, seed=87)
        items = [(a[0], a[1], oracle.encode(a[0], a[1], a[2][:1].copy(), 7, 1024)),
                 (b[0], b[1], oracle.encode(b[0], b[1], b[2], 7, 1024)),
                 (c[0], c[1], oracle.encode(c[0], c[1], c[2], 7, 1024))]
    buckets = sum(sc["bucket_table_i32"].shape[0] for _, _, sc in items)
    outs, info, status = _plan_decode(items)
    if case.startswith("fast_k"):
        assert info["work_items"] >= buckets  # ranges run side by side: items, not ranges
    else:
        assert info["work_items"] > buckets
    for (bf, _, _), got in zip(items, outs):
        assert np.array_equal(got, bf), f"mismatches: {(got != bf).sum()}"
    assert status == 0


def test_plan_small_buckets_of_k1024_tensors_on_the_k256_slab_path():
    """In a plan that also holds a k = 256 tensor (so its kernel has the k = 256 /
    512 slab instances), k = 1024 buckets of one short row have k_eff = 256 or
    512 substreams (a row of 256 or 512 columns) and take that slab path with
    P = 1; bit-exact, and so through the op, whose kernel walks them per element."""
    a = synth(64, 1024, seed=150)
    b = synth(5, 256, seed=151)     # one row a bucket: k_eff 256
    c = synth(3, 512, seed=152)     # k_eff 512
    items = [(a[0], a[1], oracle.encode(a[0], a[1], a[2][:1].copy(), 7, 256)),
             (b[0], b[1], oracle.encode(b[0], b[1], b[2], 7, 1024)),
             (c[0], c[1], oracle.encode(c[0], c[1], c[2], 7, 1024))]
    assert (items[1][2]["bucket_row_offsets_i32"][1:] - items[1][2]["bucket_row_offsets_i32"][:-1] == 1).all()
    outs, _, status = _plan_decode(items)
    for (bf, _, _), got in zip(items, outs):
        assert np.array_equal(got, bf), f"mismatches: {(got != bf).sum()}"
    assert status == 0
    for bf, q, sc in items[1:]:
        _status()
        assert np.array_equal(_gpu_decode(sc, q), bf)
        assert _status() == 0


def test_plan_split_with_bad_row_keeps_bucket_whole():
    """A row index out of range in a bucket the plan would split: the checkpoint
    walk stops, the bucket stays whole, and its decode reports the bad row."""
    bf, q, sc = synth(256, 8192, seed=88)
    side = oracle.encode(bf, q, sc[:1].copy(), 7, 1024)
    bad = {k: v.copy() for k, v in side.items()}
    bad["row_indices_i32"][130] = 10 ** 6
    _status()
    outs, info, status = _plan_decode([(None, q, bad)])
    assert status & 0x2
    assert _status() == 0  # a plan's flags go to its own word, not the device's


def test_op_plan_cache_alternating_sidecars():
    """huffman_decode_fp8 keeps one plan per sidecar from its second call on: two
    sidecars alternated through the op (fresh dtype views each call, as the
    reference's apply() passes them) decode bit-exact on every call, and an
    in-place rewrite of one sidecar's tensor (its version changes) drops that
    sidecar's plan until it is seen twice again."""
    import MPServe_cuda
    from mpserve_amd import mpserve_cuda as mc

    mc.clear_decode_plans()
    cases = []
    for n, m, scalar, seed in ((256, 8192, True, 90), (1024, 4096, False, 91)):
        bf, q, sc_u16 = synth(n, m, seed=seed)
        sc = oracle.encode(bf, q, sc_u16[:1].copy() if scalar else sc_u16, 7, 1024)
        stored = to_torch(sc, DEV)
        stored["bitstream_u64"] = stored["bitstream_u64"].view(torch.int64)  # stored signed, like safetensors
        cases.append((stored, torch.from_numpy(q).to(DEV), bf))
    _status()
    for call in range(4):
        for stored, q_t, bf in cases:
            args = list(decode_args(stored, q_t))
            args[1] = stored["bitstream_u64"].view(torch.uint64)  # a new view object every call
            out = MPServe_cuda.huffman_decode_fp8(*args)
            torch.cuda.synchronize()
            assert np.array_equal(out.view(torch.uint16).cpu().numpy(), bf), f"call {call}"
        assert _status() == 0
    entries = list(mc._PLANS._entries.values())
    assert len(entries) == 2 and all(e.plan is not None for e in entries)
    # the few-bucket sidecar's plan splits its 2 buckets into row ranges
    wi = ctypes_work_items(entries[0].plan)
    assert wi > 2
    stored, q_t, bf = cases[1]
    q_t.copy_(q_t.clone())  # same bytes, new version
    out = MPServe_cuda.huffman_decode_fp8(*decode_args(stored, q_t)[:1], stored["bitstream_u64"].view(torch.uint64),
                                          *decode_args(stored, q_t)[2:])
    torch.cuda.synchronize()
    assert np.array_equal(out.view(torch.uint16).cpu().numpy(), bf)
    assert sum(e.plan is None for e in mc._PLANS._entries.values()) == 1
    mc.clear_decode_plans()
    assert len(mc._PLANS) == 0


def ctypes_work_items(plan) -> int:
    import ctypes

    from mpserve_amd import _native

    wi, lds = ctypes.c_int64(0), ctypes.c_int64(0)
    _native.check(_native.lib().mps_fp8_plan_info(plan.handle, ctypes.byref(wi), ctypes.byref(lds)))
    return int(wi.value)


@pytest.mark.parametrize("k", [1024, 256])
def test_corrupt_sidecar_writes_stay_inside_out(k):
    """Decoding corrupt sidecars into the middle of a larger buffer (op, then a
    plan): the flags are raised and the words around the output stay zero. At
    k = 256 (one scale: two 128-row buckets) the plan runs the buckets' row
    ranges side by side on the slab path, from lane checkpoints walked over the
    corrupt sidecar."""
    import MPServe_cuda
    from mpserve_amd.decode import DecodePlan

    n, m = 256, 1024
    bf, q, sc_u16 = synth(n, m, seed=72)
    sc = oracle.encode(bf, q, sc_u16 if k == 1024 else sc_u16[:1].copy(), 7, k)
    q_t = torch.from_numpy(q).to(DEV)
    guard = 4096
    corruptions = [
        ("start bit", 0x8, lambda b: b["bucket_thread_startbit_u32"].__setitem__((0, 5), b["bucket_thread_startbit_u32"][0, 5] + 3)),
        ("row index", 0x2, lambda b: b["row_indices_i32"].__setitem__(3, n + 1000)),
        ("table id", 0x4, lambda b: b["bucket_table_i32"].__setitem__((0, 10), 10 ** 8)),
        ("bit base", 0x8, lambda b: b["bucket_bit_base_i64"].__setitem__(1, b["bucket_bit_base_i64"][1] + 64 * 5000)),
    ]
    for what, flag_bit, corrupt in corruptions:
        bad = {k: v.copy() for k, v in sc.items()}
        corrupt(bad)
        bad_t = to_torch(bad, DEV)
        for via in ("op", "plan"):
            buf = torch.zeros(n * m + 2 * guard, dtype=torch.bfloat16, device=DEV)
            out = buf[guard:guard + n * m]
            _status()
            if via == "op":
                MPServe_cuda.huffman_decode_fp8(*decode_args(bad_t, q_t), out=out)
                st = _status()
            else:
                plan = DecodePlan([(q_t, bad_t, out)])
                plan.decode()
                st = plan.read_status()
                plan.close()
            torch.cuda.synchronize()
            assert st & flag_bit, (what, via, st)
            g = buf.view(torch.uint16)
            assert int((g[:guard] != 0).sum()) == 0 and int((g[guard + n * m:] != 0).sum()) == 0, (what, via)


def test_plan_creation_waits_for_the_stream_writing_the_sidecar():
    """A plan built on the stream that is still writing its sidecar (behind a long
    kernel) reads the finished sidecar: creation synchronises that stream."""
    from mpserve_amd.decode import DecodePlan

    n, m = 128, 8192
    bf, q, sc_u16 = synth(n, m, seed=73)
    good = to_torch(oracle.encode(bf, q, sc_u16[:1].copy(), 7, 1024), DEV)
    dst = {k: torch.zeros_like(v) for k, v in good.items()}
    q_t = torch.from_numpy(q).to(DEV)
    out = torch.zeros((n, m), dtype=torch.bfloat16, device=DEV)
    busy = torch.randn((2048, 2048), device=DEV)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for _ in range(30):
            busy = torch.tanh(busy @ busy)
        for k in dst:
            dst[k].copy_(good[k])
    plan = DecodePlan([(q_t, dst, out)], stream=side)
    plan.decode(side)
    side.synchronize()
    assert plan.info()["work_items"] > 1
    assert np.array_equal(out.view(torch.uint16).cpu().numpy(), bf)
    assert plan.read_status(side) == 0


def test_cuda_clock_rate_khz():
    import MPServe_cuda

    khz = MPServe_cuda.cuda_clock_rate_khz()
    assert isinstance(khz, int) and khz > 0


def test_op_alternates_two_sidecars_on_two_streams():
    """huffman_decode_fp8 on two sidecars, each called on two streams in turn with
    no synchronisation between the calls: from the second sighting each sidecar's
    cached plan launches on both streams, every stream with its own work queue.
    Every output is bit-exact."""
    import MPServe_cuda
    from mpserve_amd.mpserve_cuda import _PLANS, read_status

    MPServe_cuda.clear_decode_plans()
    sides = []
    for i, (n, m) in enumerate(((256, 8192), (384, 4096))):
        bf, q, sc_u16 = synth(n, m, seed=260 + i)
        sides.append((to_torch(oracle.encode(bf, q, sc_u16, 7, 1024), DEV), torch.from_numpy(q).to(DEV), bf))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    outs = []
    for rnd in range(4):
        for j in range(4):
            sc_t, q_t, _ = sides[j % 2]
            st = streams[(j // 2 + rnd) % 2]
            with torch.cuda.stream(st):
                o = torch.full(q_t.shape, float("nan"), dtype=torch.bfloat16, device=DEV)
                MPServe_cuda.huffman_decode_fp8(*decode_args(sc_t, q_t), out=o)
            outs.append((o, j % 2, rnd, st))
    torch.cuda.synchronize()
    assert len(_PLANS) == 2 and all(e.plan is not None for e in _PLANS._entries.values())
    for o, which, rnd, _ in outs:
        got = o.view(torch.uint16).cpu().numpy()
        assert np.array_equal(got, sides[which][2]), f"round {rnd}, sidecar {which}"
    assert read_status(torch.device(DEV)) == 0


def test_one_plan_on_two_streams_at_once():
    """Launches of one plan on two streams overlap (each takes its items from its
    stream's queue) and both decode every item, round after round."""
    from mpserve_amd.decode import DecodePlan

    shapes = [(512, 4096, 1024)] * 4 + [(64, 1024, 256)] * 4
    items, refs = [], []
    for i, (n, m, k) in enumerate(shapes):
        bf, q, sc_u16 = synth(n, m, seed=270 + i)
        items.append((torch.from_numpy(q).to(DEV), to_torch(oracle.encode(bf, q, sc_u16, 7, k), DEV)))
        refs.append(bf)
    total = sum(q.numel() for q, _ in items)
    flat = [torch.empty(total, dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    outs, off = [], 0
    for q, _ in items:
        outs.append(flat[0][off:off + q.numel()])
        off += q.numel()
    plan = DecodePlan([(q, sc, o) for (q, sc), o in zip(items, outs)])
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rnd in range(3):
        for f in flat:
            f.fill_(float("nan"))
        for st in streams:
            st.wait_stream(torch.cuda.current_stream())
        for f, st in zip(flat, streams):
            plan.decode_into(f, st)
        for st in streams:
            torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        for s_i, f in enumerate(flat):
            off = 0
            for j, r in enumerate(refs):
                got = f[off:off + r.size].view(torch.uint16).cpu().numpy().reshape(r.shape)
                off += r.size
                assert np.array_equal(got, r), f"round {rnd}, stream {s_i}, tensor {j}"
    from mpserve_amd.mpserve_cuda import read_status

    assert read_status(torch.device(DEV)) == 0


@pytest.mark.parametrize("n,m,scalar,outlier_p,seed", [
    (256, 8192, True, 0.0, 280),     # 2 buckets: 16 workgroups each, one wave apiece
    (1024, 8192, True, 0.0, 281),    # 8 buckets (a 70B k_proj's count)
    (300, 14336, False, 0.0, 282),   # per-row scales, P = 14: groups straddle rows
    (128, 2048, True, 0.0, 283),     # P = 2: groups span rows
    (512, 8192, True, 1e-3, 284),    # ESC codes (one scale key with outliers)
    (4096, 1024, False, 0.0, 285),   # many buckets: no sharing
])
def test_op_whole_buckets_shared_by_workgroups(monkeypatch, n, m, scalar, outlier_p, seed):
    """With plans off, huffman_decode_fp8 launches whole buckets; a k = 1024
    tensor with fewer buckets than CUs has each bucket shared by several
    workgroups, each decoding some of its waves' substreams. Bit-exact,
    status clear, every path of the slab decode."""
    import MPServe_cuda

    monkeypatch.setenv("MPSERVE_DECODE_PLANS", "0")
    bf, q, sc_u16 = synth(n, m, seed=seed, outlier_p=outlier_p)
    sc = oracle.encode(bf, q, sc_u16[:1].copy() if scalar else sc_u16, 7, 1024)
    sc_t = to_torch(sc, DEV)
    q_t = torch.from_numpy(q).to(DEV)
    _status()
    for _ in range(2):
        out = torch.full((n, m), float("nan"), dtype=torch.bfloat16, device=DEV)
        MPServe_cuda.huffman_decode_fp8(*decode_args(sc_t, q_t), out=out)
        torch.cuda.synchronize()
        assert np.array_equal(out.view(torch.uint16).cpu().numpy(), bf)
    assert _status() == 0
