"""Parity of the benchmark configurations at their full shapes, on the GPU.

Configuration 2 (one Llama-3-8B layer) and configuration 3 (one Llama-3-70B
layer with outliers, so ESC codes; all seven tensors, the 235 M-element
gate/up/down included, about a minute of oracle time each) compare the GPU
sidecar builder with the CPU oracle byte for byte and the GPU decode with the
input bit for bit. Each 70B tensor's ESC keys and ESC-coded elements also
match the oracle's counts, the latter counted on the GPU from the sidecar's
tables and the input. Configuration 4 drives the vLLM
method's apply() at the 8B layer's merged shapes for T in {1, 16, 128, 1024};
configuration 5 decodes all 225 weights of the 8B model in one plan launch.

Reference: kernel/build_huffman.cu:292-969 (builder), kernel/decode_huffman.cu:188-372
(decoder), scripts/mpserve_vllm_fp8_huffman.py:389-665 (apply).
"""
import os
import sys

import numpy as np
import pytest
import torch

import oracle
from mpserve_amd.synthetic import config_weights, make_weight
from tests.helpers import NP_DTYPES, decode_args

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
CFG2 = config_weights("layer8b")
CFG3 = config_weights("layer70b")
# every 70B tensor is compared with the oracle (k/v 8 M, q/o 67 M, gate/up/down 235 M elements)
CFG3_ORACLE = tuple(c[0] for c in CFG3)


def _status():
    from mpserve_amd.mpserve_cuda import read_status

    return read_status(torch.device(DEV))


def _weight(n, m, seed, sigma, outlier_p):
    print(f"[cfg] weight {n}x{m} seed {seed} sigma {sigma} outliers {outlier_p}", flush=True)
    return make_weight(n, m, sigma=sigma, seed=seed, outlier_p=outlier_p, device=DEV)


def _gpu_build(w, k=1024):
    from mpserve_amd.encode import build_fp8_sidecar

    return build_fp8_sidecar(w.bf16, w.fp8_u8, w.scale_u16, max_len=7, threads_per_block=k, with_stats=True)


def _assert_same_as_oracle(side, w):
    bf = w.bf16.view(torch.uint16).cpu().numpy()
    q = w.fp8_u8.cpu().numpy()
    ref, stats = oracle.encode(bf, q, w.scale_u16.cpu().numpy(), 7, 1024, with_stats=True)
    assert list(side.keys()) == list(ref.keys())
    for key, r in ref.items():
        g = side[key].cpu().numpy()
        assert g.dtype == NP_DTYPES[key] and g.shape == r.shape, (key, g.dtype, g.shape, r.shape)
        assert np.array_equal(g, r), f"{key}: {(g != r).sum()} differing entries"
    return stats


def _esc_elements(side, w) -> int:
    """Elements coded as ESC: those of a key with ESC entries whose symbol is not
    one its table keeps (build_huffman.cu:485-535, :850-864), counted on the GPU
    from the sidecar and the input alone."""
    lens = side["decode_lens_u8"]
    esc_gids = torch.nonzero(((lens & 0x88) != 0).any(dim=1)).flatten().tolist()
    if not esc_gids:
        return 0
    n, m = w.fp8_u8.shape
    ro = side["bucket_row_offsets_i32"].long()
    bucket_of_pos = torch.repeat_interleave(torch.arange(ro.numel() - 1, device=DEV), ro[1:] - ro[:-1])
    row_bucket = torch.empty(n, dtype=torch.long, device=DEV)
    row_bucket[side["row_indices_i32"].long()] = bucket_of_pos
    table = side["bucket_table_i32"]
    syms = side["decode_syms_u16"].view(torch.int16).to(torch.int32) & 0xFFFF
    nib = torch.stack([lens & 0xF, lens >> 4], dim=2).reshape(lens.shape[0], -1)  # entry p's nibble
    count = 0
    for r0 in range(0, n, 1024):  # row chunks keep the gathered ids small
        r1 = min(n, r0 + 1024)
        gid = table[row_bucket[r0:r1, None], w.fp8_u8[r0:r1].long()]
        sym = w.bf16[r0:r1].view(torch.int16).to(torch.int32) & 0xFFFF
        for g in esc_gids:
            kept = torch.unique(syms[g][((nib[g] & 8) == 0) & ((nib[g] & 7) != 0)])
            sel = gid == g
            count += int((~torch.isin(sym[sel], kept)).sum().item())
    return count


def _assert_invariants(side, n, m):
    """Structure every well-formed sidecar has (build_huffman.cu:786-925)."""
    base = side["bucket_bit_base_i64"].cpu().numpy()
    sb = side["bucket_thread_startbit_u32"].cpu().numpy().astype(np.int64)
    ro = side["bucket_row_offsets_i32"].cpu().numpy()
    rows = np.sort(side["row_indices_i32"].cpu().numpy())
    assert np.array_equal(rows, np.arange(n)), "every row in exactly one bucket"
    assert ro[0] == 0 and np.all(np.diff(ro) >= 1) and np.all(np.diff(ro) <= 128)
    assert np.all(base[:-1] % 64 == 0) and np.all(np.diff(base) >= 0)
    assert np.all(sb[:, 0] == 0) and np.all(np.diff(sb, axis=1) >= 0)
    assert np.all(base[:-1] + sb[:, -1] <= base[1:]), "a bucket's lanes end before the next bucket"
    assert base[-1] == base[-2] + sb[-1, -1]
    assert side["bitstream_u64"].numel() == (int(base[-1]) + 63) // 64
    assert (side["bucket_col_len_i32"] == m).all() and (side["bucket_col_start_i32"] == 0).all()


def _decode_op_and_plan(side, w):
    import MPServe_cuda
    from mpserve_amd.decode import DecodePlan

    _status()
    ref = w.bf16.view(torch.uint16)
    out = MPServe_cuda.huffman_decode_fp8(*decode_args(side, w.fp8_u8))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.uint16), ref), f"op: {(out.view(torch.uint16) != ref).sum().item()} mismatches"
    assert _status() == 0
    plan_out = torch.zeros_like(w.bf16)
    plan = DecodePlan([(w.fp8_u8, side, plan_out)])
    plan.decode()
    torch.cuda.synchronize()
    assert torch.equal(plan_out.view(torch.uint16), ref)
    assert plan.read_status() == 0
    plan.close()


@pytest.mark.parametrize("name,n,m,seed,sigma,outlier_p", CFG2, ids=[c[0].split(".")[-1] for c in CFG2])
def test_cfg2_layer8b(name, n, m, seed, sigma, outlier_p):
    """Config 2: GPU build == oracle (17 arrays), GPU decode == input, per 8B linear."""
    w = _weight(n, m, seed, sigma, outlier_p)
    side, _ = _gpu_build(w)
    _assert_same_as_oracle(side, w)
    _assert_invariants(side, n, m)
    _decode_op_and_plan(side, w)


@pytest.mark.parametrize("name,n,m,seed,sigma,outlier_p", CFG3, ids=[c[0].split(".")[-1] for c in CFG3])
def test_cfg3_layer70b(name, n, m, seed, sigma, outlier_p):
    """Config 3: outliers put every row on one scale key, so the keys of the
    large tensors (64 M elements and more) exceed 128 symbols and their
    sidecars carry ESC codes; the decode stays lossless. (k/v, 8 M elements,
    stay below 128 symbols per key.)"""
    w = _weight(n, m, seed, sigma, outlier_p)
    side, stats = _gpu_build(w)
    assert stats["esc_collisions"] == 0
    if n * m >= 8192 * 8192:
        assert stats["esc_keys"] > 0
    assert int(((side["decode_lens_u8"] & 0x88) != 0).any(dim=1).sum().item()) == stats["esc_keys"]
    # rows group by scale key in runs of <= 128 (build_huffman.cu:611-656); a row
    # with no +-8 sigma outlier (~e^-8 of them) has a key of its own
    _, per_key = torch.unique(w.scale_u16, return_counts=True)
    assert int(per_key.max()) >= 0.99 * n
    assert side["bucket_table_i32"].shape[0] == int(((per_key + 127) // 128).sum())
    if name in CFG3_ORACLE:
        print(f"[cfg3] {name}: oracle build of {n}x{m}", flush=True)
        ostats = _assert_same_as_oracle(side, w)
        assert ostats["esc_keys"] == stats["esc_keys"]
        assert ostats["esc_collisions"] == stats["esc_collisions"] == 0
        assert ostats["esc_elements"] == _esc_elements(side, w)
        assert (ostats["esc_elements"] > 0) == (stats["esc_keys"] > 0)
    _assert_invariants(side, n, m)
    _decode_op_and_plan(side, w)


@pytest.mark.parametrize("k", [256, 512])
def test_cfg2_layer8b_k256_k512_one_plan_and_op(k):
    """Config 2 with sidecars of k = 256 / 512 substreams (the reference builder's
    default is 256): all seven 8B linears in one plan launch, where their buckets
    run 1024 / k row ranges side by side on the slab path at stride k, and each
    through the op (whole buckets, then the sidecar's cached plan). Bit-exact, status
    clean. A 70B q_proj with outliers adds ESC tables at this k."""
    import MPServe_cuda
    from mpserve_amd.decode import DecodePlan

    items = []
    for name, n, m, seed, sigma, outlier_p in list(CFG2) + [c for c in CFG3 if c[0] == "layers.0.q_proj"]:
        w = _weight(n, m, seed, sigma, outlier_p)
        side, stats = _gpu_build(w, k)
        assert stats["esc_collisions"] == 0
        if outlier_p > 0:
            assert stats["esc_keys"] > 0
        items.append((w, side))
    _status()
    outs = [torch.zeros_like(w.bf16) for w, _ in items]
    plan = DecodePlan([(w.fp8_u8, side, o) for (w, side), o in zip(items, outs)])
    plan.decode()
    torch.cuda.synchronize()
    for (w, _), o in zip(items, outs):
        assert torch.equal(o.view(torch.uint16), w.bf16.view(torch.uint16))
    assert plan.read_status() == 0
    plan.close()
    for w, side in items:
        for _ in range(2):
            out = MPServe_cuda.huffman_decode_fp8(*decode_args(side, w.fp8_u8))
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.uint16), w.bf16.view(torch.uint16))
    assert _status() == 0


def test_cfg5_model8b_all_weights_one_plan():
    """Config 5: all 225 weights (32 layers x 7 + lm_head) built on the GPU and
    decoded in one plan launch, each equal to its input."""
    from mpserve_amd.decode import DecodePlan

    weights = config_weights("model8b")
    assert len(weights) == 225
    items, srcs = [], []
    for i, (name, n, m, seed, sigma, outlier_p) in enumerate(weights):
        w = make_weight(n, m, sigma=sigma, seed=seed, outlier_p=outlier_p, device=DEV)
        side, _ = _gpu_build(w)
        items.append((w.fp8_u8, side, torch.empty_like(w.bf16)))
        srcs.append(w.bf16)
        if i % 32 == 31:
            print(f"[cfg5] built {i + 1}/225", flush=True)
    _status()
    plan = DecodePlan(items)
    assert plan.info()["work_items"] >= sum(int(s["bucket_table_i32"].shape[0]) for _, s, _ in items)
    for rep in range(2):
        for _, _, o in items:
            o.fill_(float("nan"))
        plan.decode()
        torch.cuda.synchronize()
        for (name, *_), (_, _, o), src in zip(weights, items, srcs):
            assert torch.equal(o.view(torch.uint16), src.view(torch.uint16)), f"{name} (pass {rep})"
    assert plan.read_status() == 0
    plan.close()


# --------------------------------------------------------------------- config 4
FAKES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fakes")


def _stored(side, fp8):
    """GPU-built sidecar in the compress script's stored form (huff_ names, signed dtypes)."""
    t = {"huff_fp8_u8": fp8}
    for key in ("bitstream_u64", "decode_syms_u16", "decode_lens_u8", "bucket_table_i32", "bucket_col_start_i32",
                "bucket_col_len_i32", "bucket_row_offsets_i32", "row_indices_i32", "bucket_thread_startbit_u32",
                "bucket_bit_base_i64"):
        v = side[key]
        signed = {torch.uint64: torch.int64, torch.uint16: torch.int16, torch.uint32: torch.int32}.get(v.dtype)
        t["huff_" + key] = v.view(signed) if signed is not None else v
    t["huff_attn_block_row_start_i32"] = torch.empty((0,), dtype=torch.int32, device=fp8.device)
    t["huff_attn_block_row_len_i32"] = torch.empty((0,), dtype=torch.int32, device=fp8.device)
    return t


# merged linears of one 8B layer: (prefix, [(shard id, config-2 weight name)])
_CFG4_LAYERS = [
    ("model.layers.0.self_attn.qkv_proj", [("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj")]),
    ("model.layers.0.self_attn.o_proj", [(None, "o_proj")]),
    ("model.layers.0.mlp.gate_up_proj", [("gate", "gate_proj"), ("up", "up_proj")]),
    ("model.layers.0.mlp.down_proj", [(None, "down_proj")]),
]


@pytest.mark.parametrize("prefix,shards", _CFG4_LAYERS, ids=[p.split(".")[-1] for p, _ in _CFG4_LAYERS])
def test_cfg4_apply_8b_shapes(prefix, shards, monkeypatch):
    """Config 4: apply() on the 8B layer's linears (merged qkv and gate_up as
    vLLM loads them) rebuilds the exact BF16 weight, and its output equals
    x @ W^T on that weight for T in {1, 16, 128, 1024}. Tolerance: both sides run
    the same BF16 GEMM on identical operands, so they agree to BF16 rounding of
    the accumulation (rtol 1e-2, atol 2e-2 at |out| ~ 1.3)."""
    if FAKES not in sys.path:
        sys.path.insert(0, FAKES)
    monkeypatch.setenv("MPSERVE_ENABLE_FP8_HUFFMAN", "1")
    vfh = pytest.importorskip("mpserve_amd.vllm_fp8_huffman")
    from vllm.model_executor.layers.linear import LinearBase

    spec = {c[0].split(".")[-1]: c for c in CFG2}
    ws = []
    for _, wname in shards:
        _, n, m, seed, sigma, outlier_p = spec[wname]
        ws.append(_weight(n, m, seed, sigma, outlier_p))
    k = int(ws[0].bf16.shape[1])
    out_sizes = [int(w.bf16.shape[0]) for w in ws]
    layer = LinearBase(prefix)
    method = vfh.FP8HuffmanConfig.from_config({"max_len": 7}).get_quant_method(layer, prefix)
    assert isinstance(method, vfh.FP8HuffmanLinearMethod)
    method.create_weights(layer, k, out_sizes, k, sum(out_sizes), torch.bfloat16)
    layer.quant_method = method
    for (sid, _), w in zip(shards, ws):
        side, _ = _gpu_build(w)
        for pname, t in _stored(side, w.fp8_u8).items():
            p = getattr(layer, pname)
            if sid is None:
                p.weight_loader(p, t)
            else:
                p.weight_loader(p, t, sid)
    method.process_weights_after_loading(layer)
    w_exact = torch.cat([w.bf16 for w in ws], dim=0)
    got_w = method.decoded_weight(layer, k)
    torch.cuda.synchronize()
    assert torch.equal(got_w.view(torch.uint16), w_exact.view(torch.uint16))
    g = torch.Generator(device=DEV).manual_seed(4)
    for t in (1, 16, 128, 1024):
        x = torch.randn((t, k), generator=g, device=DEV, dtype=torch.float32).to(torch.bfloat16)
        out = method.apply(layer, x)
        ref = torch.matmul(x, w_exact.t())
        assert out.shape == (t, sum(out_sizes))
        assert torch.allclose(out.float(), ref.float(), rtol=1e-2, atol=2e-2), f"T={t}"
    assert _status() == 0
