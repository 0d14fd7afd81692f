"""Pins the AWQ int4 oracle (oracle/awq_huffman_oracle.c) on the CPU.

The reference ships no tests or vectors for these builders either, so each part
is pinned by what the mathematics or the reference's own structure fixes:

* round trip: decode(encode(x)) == x bit for bit, for both layouts, every scale
  mode, k below and above the bucket's column count, and keys with ESC codes;
* tables and buckets: closed forms recomputed with numpy (np.unique of the
  (scale, qv) keys, the row / group order and chunking);
* code books: Kraft sums, LUT coverage, the ESC entry (nibble 15, length L,
  one entry); with ESC the 2^L codes all have length L, so the LUT lists the
  symbols in hand-out order, which differs between the builders: (count asc,
  sym asc) with ESC placed by its weight for row buckets, (count desc, sym asc)
  with ESC last by scale - a mistake in either ordering fails that test;
* hypothesis: random small shapes, layouts, k and group caps round-trip, with
  64-bit aligned bucket bases and monotone start bits;
* ESC symbol choice: smallest u16 outside the kept set (row buckets, where a
  data symbol can collide with it) or outside all of the key's symbols (by
  scale), checked against a brute-force scan.
"""
import numpy as np
import pytest
import torch

import oracle
from mpserve_amd.synthetic import make_awq_weight

L = 11


def _np(w):
    return (w.bf16.view(torch.uint16).numpy(), w.int4_u8.numpy(), w.scale_u16.numpy())


def esc_inputs(n=64, m=1024, distinct=3000, seed=0, with_zero=True):
    """One key (scalar scale, one int4 value) with more than 2^11 distinct symbols."""
    rng = np.random.default_rng(seed)
    syms = np.arange(0x3C00, 0x3C00 + distinct, dtype=np.uint16)  # no 0x0000 / 0x0001 among them
    p = 1.0 / np.arange(1, distinct + 1) ** 0.7
    bits = rng.choice(syms, size=n * m, p=p / p.sum()).astype(np.uint16)
    if with_zero:
        bits[rng.choice(n * m, size=3, replace=False)] = 0  # rare symbol 0: never kept
    q = np.full(n * m, 5, dtype=np.uint8)
    return bits.reshape(n, m), q.reshape(n, m), np.array([0x3F80], dtype=np.uint16)


CASES = [
    ("per_row", 64, 256, None, 256, False),
    ("block2d_sb0_1", 64, 256, 128, 256, False),
    ("by_scale_group128", 64, 256, 128, 256, True),
    ("by_scale_per_row", 48, 384, None, 100, True),
    ("by_scale_k_gt_group", 32, 512, 64, 1024, True),
    ("block2d_k1", 16, 64, 32, 1, False),
]


@pytest.mark.parametrize("name,n,m,group,k,by_scale", CASES, ids=[c[0] for c in CASES])
def test_round_trip(name, n, m, group, k, by_scale):
    bits, q, sc = _np(make_awq_weight(n, m, group, seed=hash(name) & 0xFFFF))
    d = oracle.awq_encode(bits, q, sc, L, k, 16, by_scale)
    assert np.array_equal(oracle.awq_decode(d, q, n, m), bits)


def test_round_trip_block2d_rows_and_columns():
    # block-2D with sb0 > 1 and k above the column block
    w = make_awq_weight(64, 256, 64, seed=3)
    bits, q, _ = _np(w)
    sc = w.scale_u16.numpy()[::4].copy()  # [16, 4]: 4 rows x 64 columns share a scale
    for by_scale in (False, True):
        d = oracle.awq_encode(bits, q, sc, L, 512, 8, by_scale)
        assert np.array_equal(oracle.awq_decode(d, q, 64, 256), bits)


def _key_of_elements(q, sc, n, m):
    if sc.size == 1:
        s = np.full((n, m), sc.reshape(-1)[0], np.uint32)
    elif sc.ndim == 1:
        s = np.repeat(sc.astype(np.uint32)[:, None], m, axis=1)
    else:
        s = np.kron(sc.astype(np.uint32), np.ones((n // sc.shape[0], m // sc.shape[1]), np.uint32))
    return (s << 16) | (q.astype(np.uint32) & 0xF)


@pytest.mark.parametrize("by_scale", [False, True])
def test_tables_and_bucket_table_closed_form(by_scale):
    w = make_awq_weight(64, 256, 64, seed=7)
    bits, q, sc = _np(w)
    d = oracle.awq_encode(bits, q, sc, L, 256, 8, by_scale)
    keys = np.unique(_key_of_elements(q, sc, 64, 256))
    assert np.array_equal(d["table_scale_u16"], (keys >> 16).astype(np.uint16))
    assert np.array_equal(d["table_qv_u16"], (keys & 0xFFFF).astype(np.uint16))
    bkey = (d["bucket_scale_u16"].astype(np.uint32)[:, None] << 16) | np.arange(16, dtype=np.uint32)[None]
    pos = np.searchsorted(keys, bkey)
    want = np.where((pos < keys.size) & (keys[np.minimum(pos, keys.size - 1)] == bkey), pos, -1)
    assert np.array_equal(d["bucket_table_i32"], want.astype(np.int32))


def test_by_scale_groups_closed_form():
    w = make_awq_weight(40, 256, 32, seed=11)
    bits, q, sc = _np(w)
    cap = 7
    d = oracle.awq_encode(bits, q, sc, L, 64, cap, True)
    rows, cols = np.meshgrid(np.arange(40), np.arange(0, 256, 32), indexing="ij")
    gsc = sc.reshape(-1)
    order = np.lexsort((cols.reshape(-1), rows.reshape(-1), gsc))  # scale, then (row, col)
    assert np.array_equal(d["group_rows_i32"], rows.reshape(-1)[order])
    assert np.array_equal(d["group_col_start_i32"], cols.reshape(-1)[order])
    # buckets: runs of one scale, cut every `cap` groups
    offs, bsc = [0], []
    s_sorted = gsc[order]
    i = 0
    while i < s_sorted.size:
        j = i
        while j < s_sorted.size and s_sorted[j] == s_sorted[i]:
            j += 1
        for off in range(i, j, cap):
            offs.append(min(off + cap, j))
            bsc.append(s_sorted[i])
        i = j
    assert np.array_equal(d["bucket_group_offsets_i32"], offs)
    assert np.array_equal(d["bucket_scale_u16"], bsc)
    assert list(d["shape_nmkg_i64"]) == [40, 256, 64, 32]


def test_row_buckets_closed_form():
    w = make_awq_weight(300, 64, None, seed=12)
    bits, q, sc = _np(w)
    sc = (sc & 0xFFF0).astype(np.uint16)  # fewer distinct scales: several rows share one
    d = oracle.awq_encode(bits, q, sc, L, 32, 1, False)
    order = np.lexsort((np.arange(300), sc))
    assert np.array_equal(d["row_indices_i32"], order)
    assert np.all(np.diff(d["bucket_row_offsets_i32"]) <= 128)
    assert np.all(d["bucket_col_start_i32"] == 0) and np.all(d["bucket_col_len_i32"] == 64)
    assert list(d["shape_nmk_i64"]) == [300, 64, 32]


def _lengths(lens_row):
    nib = np.empty(lens_row.size * 2, np.uint8)
    nib[0::2] = lens_row & 0xF
    nib[1::2] = lens_row >> 4
    return nib


def _code_table(d, g):
    """{sym: (length, number of LUT entries)} of table g, and the ESC entry indices."""
    syms, nib = d["decode_syms_u16"][g], _lengths(d["decode_lens_u8"][g])
    out, esc = {}, np.nonzero(nib == 15)[0]
    for s in np.unique(syms[nib != 0]):
        idx = np.nonzero((syms == s) & (nib != 0))[0]
        ln = int(nib[idx[0]])
        out[int(s)] = (L if ln == 15 else ln, idx.size)
    return out, esc


@pytest.mark.parametrize("by_scale", [False, True])
def test_code_tables_kraft_and_coverage(by_scale):
    bits, q, sc = _np(make_awq_weight(64, 256, 128, seed=5))
    d = oracle.awq_encode(bits, q, sc, L, 256, 16, by_scale)
    for g in range(d["decode_syms_u16"].shape[0]):
        codes, esc = _code_table(d, g)
        assert esc.size == 0
        kraft = sum(2.0 ** -ln for ln, _ in codes.values())
        assert kraft <= 1.0 + 1e-12
        if len(codes) == 1:
            # one symbol: every entry, length 1 (build_huffman.cu:1731-1737)
            assert list(codes.values()) == [(1, 2 ** L)]
            continue
        assert kraft == pytest.approx(1.0)
        for ln, cnt in codes.values():
            assert cnt == 2 ** (L - ln)  # each code fills its whole LUT range


def _esc_case(by_scale, with_zero=True):
    bits, q, sc = esc_inputs(with_zero=with_zero)
    d, st = oracle.awq_encode(bits, q, sc, L, 256, 1024, by_scale, with_stats=True)
    assert st["esc_keys"] == 1
    codes, esc = _code_table(d, 0)
    return bits, q, d, st, codes, esc


@pytest.mark.parametrize("by_scale", [False, True])
def test_esc_entry_is_one_L_bit_code(by_scale):
    _, _, d, _, codes, esc = _esc_case(by_scale)
    assert esc.size == 1  # length L: exactly one LUT entry, nibble 15
    assert len(codes) == 2 ** L  # 2^L - 1 kept symbols + ESC


def test_esc_symbol_row_buckets_smallest_not_kept_and_collision():
    bits, q, d, st, codes, esc = _esc_case(False)
    esc_sym = int(d["decode_syms_u16"][0][esc[0]])
    kept = set(codes) - {esc_sym}
    assert esc_sym == min(set(range(65536)) - kept)  # brute force
    assert esc_sym == 0  # symbol 0 is present but rare: not kept, so it collides
    assert st["esc_collisions"] == 3
    # the colliding elements are coded as bare ESC codes: the round trip breaks
    # exactly as the reference's stream does
    assert not np.array_equal(oracle.awq_decode(d, q, 64, 1024), bits)


def test_esc_symbol_by_scale_absent_from_all_symbols():
    bits, q, d, st, codes, esc = _esc_case(True)
    esc_sym = int(d["decode_syms_u16"][0][esc[0]])
    present = set(np.unique(bits).tolist())
    assert esc_sym == min(set(range(65536)) - present)
    assert st["esc_collisions"] == 0
    assert np.array_equal(oracle.awq_decode(d, q, 64, 1024), bits)


def test_esc_round_trip_row_buckets_without_collision():
    bits, q, d, st, _, _ = _esc_case(False, with_zero=False)
    assert st["esc_collisions"] == 0 and st["esc_elements"] > 0
    assert np.array_equal(oracle.awq_decode(d, q, 64, 1024), bits)


def test_esc_code_order_row_buckets_vs_by_scale():
    """With ESC the 2^L codes all have length L (Kraft), so the LUT lists the
    symbols in hand-out order: (count asc, sym asc) with ESC placed by its
    weight for row buckets; (count desc, sym asc) with ESC last by scale."""
    for by_scale in (False, True):
        bits, _, d, _, _, esc = _esc_case(by_scale, with_zero=False)
        lut = d["decode_syms_u16"][0].astype(np.int64)
        esc_sym = int(lut[esc[0]])
        vals, counts = np.unique(bits, return_counts=True)
        freq = dict(zip(vals.tolist(), counts.tolist()))
        kept = sorted(freq, key=lambda s: (-freq[s], s))[: 2 ** L - 1]
        esc_w = sum(freq.values()) - sum(freq[s] for s in kept)
        if by_scale:
            want = kept + [esc_sym]
        else:
            w = dict(freq)
            w[esc_sym] = esc_w
            want = sorted(kept + [esc_sym], key=lambda s: (w[s], s))
        assert lut.tolist() == want
        if by_scale:
            assert esc[0] == 2 ** L - 1


def test_validation_messages():
    bits, q, sc = _np(make_awq_weight(8, 32, None, seed=1))
    with pytest.raises(ValueError, match=r"max_len must be in \(0,15\]"):
        oracle.awq_encode(bits, q, sc, 16)
    with pytest.raises(ValueError, match=r"threads_per_block must be in \[1,1024\]"):
        oracle.awq_encode(bits, q, sc, 11, 0)
    with pytest.raises(ValueError, match="group_cap must be > 0"):
        oracle.awq_encode(bits, q, sc, 11, 256, 0, True)
    with pytest.raises(ValueError, match="unsupported scales_u16 shape"):
        oracle.awq_encode(bits, q, np.zeros(5, np.uint16), 11)


from hypothesis import HealthCheck, assume, example, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402


def test_make_awq_weight_rejects_group_not_dividing_columns():
    with pytest.raises(ValueError, match="must divide the column count"):
        make_awq_weight(1, 8, 16, seed=0)


@settings(max_examples=25, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(n=st.integers(1, 24), mcols=st.sampled_from([8, 16, 48, 64]), group=st.sampled_from([None, 8, 16]),
       k=st.sampled_from([1, 3, 64, 256, 1024]), cap=st.integers(1, 9), by_scale=st.booleans(),
       seed=st.integers(0, 1 << 16))
@example(n=1, mcols=16, group=16, k=1, cap=1, by_scale=True, seed=0)
@example(n=1, mcols=8, group=8, k=1, cap=1, by_scale=False, seed=0)
def test_round_trip_property(n, mcols, group, k, cap, by_scale, seed):
    """Any small shape, scale layout, k (below and above the column count) and
    group cap: decode(encode(x)) == x, and per-bucket bit counts sum up. The
    group width must divide the column count (a quantisation group never
    straddles rows)."""
    assume(group is None or mcols % group == 0)
    w = make_awq_weight(n, mcols, group, seed=seed)
    bits, q, sc = _np(w)
    d = oracle.awq_encode(bits, q, sc, L, k, cap, by_scale)
    assert np.array_equal(oracle.awq_decode(d, q, n, mcols), bits)
    base, sb = d["bucket_bit_base_i64"], d["bucket_thread_startbit_u32"]
    assert np.all(base[:-1] % 64 == 0) and np.all(np.diff(sb.astype(np.int64), axis=1) >= 0)
    assert np.all(base[:-1] + sb[:, -1] <= np.append(base[1:-1], base[-1]))
