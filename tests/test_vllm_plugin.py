"""The vLLM fp8_huffman surface, driven through a stand-in vLLM (tests/fakes/vllm).

Covers the reference plugin's contract (scripts/mpserve_vllm_fp8_huffman.py):
config keys, defaults and the env gate (:95-148), the thirteen huff_* params
and their loaders with the shard map (:155-360), and apply() (:389-665) on the
GPU, where a merged qkv layer must reproduce x @ W.T for the exact BF16 weights.
"""
import os
import sys

import numpy as np
import pytest
import torch

FAKES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fakes")
if FAKES not in sys.path:
    sys.path.insert(0, FAKES)

import oracle  # noqa: E402
from tests.helpers import synth  # noqa: E402

vfh = pytest.importorskip("mpserve_amd.vllm_fp8_huffman")
from vllm.model_executor.layers.linear import LinearBase, UnquantizedLinearMethod  # noqa: E402
from vllm.model_executor.layers.quantization import REGISTRY  # noqa: E402


def stored_sidecar(bf, q, sc, k=1024):
    """Sidecar tensors as the compress script stores them (signed dtypes, huff_ names)."""
    s = oracle.encode(bf, q, sc, 7, k)
    t = {
        "huff_fp8_u8": torch.from_numpy(np.ascontiguousarray(q)),
        "huff_bitstream_u64": torch.from_numpy(s["bitstream_u64"].view(np.int64)),
        "huff_decode_syms_u16": torch.from_numpy(s["decode_syms_u16"].view(np.int16)),
        "huff_decode_lens_u8": torch.from_numpy(s["decode_lens_u8"]),
        "huff_bucket_table_i32": torch.from_numpy(s["bucket_table_i32"]),
        "huff_bucket_col_start_i32": torch.from_numpy(s["bucket_col_start_i32"]),
        "huff_bucket_col_len_i32": torch.from_numpy(s["bucket_col_len_i32"]),
        "huff_bucket_row_offsets_i32": torch.from_numpy(s["bucket_row_offsets_i32"]),
        "huff_row_indices_i32": torch.from_numpy(s["row_indices_i32"]),
        "huff_bucket_thread_startbit_u32": torch.from_numpy(s["bucket_thread_startbit_u32"].view(np.int32)),
        "huff_bucket_bit_base_i64": torch.from_numpy(s["bucket_bit_base_i64"]),
        "huff_attn_block_row_start_i32": torch.empty((0,), dtype=torch.int32),
        "huff_attn_block_row_len_i32": torch.empty((0,), dtype=torch.int32),
    }
    return t


def make_layer(prefix, out_sizes, k):
    layer = LinearBase(prefix)
    cfg = vfh.FP8HuffmanConfig.from_config({"max_len": 7})
    cfg._enabled = True
    method = cfg.get_quant_method(layer, prefix)
    assert isinstance(method, vfh.FP8HuffmanLinearMethod)
    method.create_weights(layer, k, list(out_sizes), k, sum(out_sizes), torch.bfloat16)
    layer.quant_method = method
    return layer, method


def load(layer, tensors, shard_id=None):
    for name, t in tensors.items():
        p = getattr(layer, name)
        if shard_id is None:
            p.weight_loader(p, t)
        else:
            p.weight_loader(p, t, shard_id)


# ---------------------------------------------------------------------------- CPU
def test_config_surface(monkeypatch):
    assert REGISTRY["fp8_huffman"] is vfh.FP8HuffmanConfig
    cfg = vfh.FP8HuffmanConfig.from_config({"max_len": 7, "include_regex": r"self_attn"})
    assert cfg.get_name() == "fp8_huffman"
    assert cfg.get_supported_act_dtypes() == [torch.half, torch.bfloat16]
    assert vfh.FP8HuffmanConfig.get_min_capability() == 90
    assert vfh.FP8HuffmanConfig.get_config_filenames() == []
    with pytest.raises(ValueError, match="requires max_len=7"):
        vfh.FP8HuffmanConfig(max_len=12)
    # from_config leaves ignore_regex None unless given; the constructor default ignores lm_head & co
    assert vfh.FP8HuffmanConfig().ignore_regex == vfh.DEFAULT_IGNORE


def test_env_gate_and_regex_filters(monkeypatch):
    lin = LinearBase("model.layers.0.self_attn.qkv_proj")
    monkeypatch.delenv("MPSERVE_ENABLE_FP8_HUFFMAN", raising=False)
    assert isinstance(vfh.FP8HuffmanConfig().get_quant_method(lin, lin.prefix), UnquantizedLinearMethod)
    monkeypatch.setenv("MPSERVE_ENABLE_FP8_HUFFMAN", "1")
    cfg = vfh.FP8HuffmanConfig(include_regex=r"self_attn")
    assert isinstance(cfg.get_quant_method(lin, lin.prefix), vfh.FP8HuffmanLinearMethod)
    mlp = LinearBase("model.layers.0.mlp.gate_up_proj")
    assert isinstance(cfg.get_quant_method(mlp, mlp.prefix), UnquantizedLinearMethod)
    head = LinearBase("lm_head")
    assert isinstance(vfh.FP8HuffmanConfig().get_quant_method(head, "lm_head"), UnquantizedLinearMethod)
    assert vfh.FP8HuffmanConfig().get_quant_method(torch.nn.Linear(2, 2), "x") is None


def test_create_weights_registers_reference_params():
    layer, _ = make_layer("model.layers.0.self_attn.o_proj", [64], 32)
    names = dict(layer.named_parameters())
    for name, dt in vfh.HUFF_PARAMS:
        assert names[name].dtype == dt, name
    assert names["huff_attn_block_row_start_i32"].numel() == 0
    assert names["weight"].dtype == torch.uint8
    assert names["weight_scale_inv"].dtype == torch.float16 and names["weight_scale"].dtype == torch.float16
    assert int(layer.huff_max_len) == 7 and int(layer.huff_in_features_i32) == 32
    assert int(layer.huff_out_features_i32) == 64
    assert "huff_max_len" not in layer.state_dict()  # non-persistent buffers


def test_tp_greater_than_one_is_rejected():
    layer = LinearBase("x")
    layer.tp_size = 2
    m = vfh.FP8HuffmanLinearMethod(vfh.FP8HuffmanParams())
    with pytest.raises(NotImplementedError, match="tp_size=1"):
        m.create_weights(layer, 8, [8], 8, 8, torch.bfloat16)


def test_loaders_unsharded_and_sharded():
    bf, q, sc = synth(40, 64, seed=1)
    t = stored_sidecar(bf, q, sc, 64)
    layer, method = make_layer("model.layers.0.self_attn.o_proj", [40], 64)
    load(layer, t)
    assert torch.equal(layer.huff_fp8_u8.data.cpu(), t["huff_fp8_u8"])
    layer.weight.weight_loader(layer.weight, torch.ones(3))  # discarded
    assert layer.weight.numel() == 1

    merged, _ = make_layer("model.layers.0.self_attn.qkv_proj", [40, 8, 8], 64)
    for sid in ("q", "k", "v"):
        load(merged, t, sid)
    assert sorted(merged._fp8_huff_shards) == [0, 1, 2]
    assert set(merged._fp8_huff_shards[1]) == set(t)  # every huff_* array of the k shard
    with pytest.raises(ValueError, match="Unknown shard_id"):
        merged.huff_fp8_u8.weight_loader(merged.huff_fp8_u8, t["huff_fp8_u8"], "o")
    method.process_weights_after_loading(layer)
    assert isinstance(layer.huff_fp8_u8, torch.nn.Parameter)
    assert vfh._LAYERS_BY_PREFIX["model.layers.0.self_attn.o_proj"] is layer


def _pack(start, rows):
    return {"huff_attn_block_row_start_i32": torch.tensor([start], dtype=torch.int32),
            "huff_attn_block_row_len_i32": torch.tensor([rows], dtype=torch.int32)}


def test_packed_leader_with_its_own_rows_does_not_recurse():
    """A block leader (<block>.self_attn.o_proj) that carries pack rows itself
    slices its own decoded weight (reference :628-655). Without a GPU its weight
    cannot be decoded: that is reported, for the leader and for its members."""
    bf, q, sc = synth(96, 64, seed=3)
    leader, lm = make_layer("model.layers.5.self_attn.o_proj", [96], 64)
    load(leader, stored_sidecar(bf, q, sc, 64))
    load(leader, _pack(0, 32))
    lm.process_weights_after_loading(leader)
    st = leader._fp8_huff
    assert st.pack == (0, 32) and st.leader == "model.layers.5.self_attn.o_proj"
    with pytest.raises(RuntimeError, match="not on a GPU"):
        lm._weight_for_apply(leader)
    member, mm = make_layer("model.layers.5.mlp.gate_up_proj", [64], 64)
    load(member, _pack(32, 64))
    mm.process_weights_after_loading(member)
    assert member._fp8_huff.plan is None and member._fp8_huff.leader == "model.layers.5.self_attn.o_proj"
    with pytest.raises(RuntimeError, match="layer-pack leader"):
        mm._weight_for_apply(member)
    with pytest.raises(RuntimeError, match="leader's"):
        mm.decoded_weight(member)
    orphan, om = make_layer("model.layers.9.mlp.down_proj", [8], 64)
    load(orphan, _pack(0, 8))
    om.process_weights_after_loading(orphan)
    with pytest.raises(RuntimeError, match="cannot find layer-pack leader"):
        om._weight_for_apply(orphan)


def test_pack_rows_outside_a_block_are_ignored():
    """Pack rows of a layer that is in no attention or MLP block do not apply:
    the reference then decodes the layer's own sidecar (:609-629)."""
    bf, q, sc = synth(16, 64, seed=4)
    layer, method = make_layer("model.embed_proj", [16], 64)
    load(layer, stored_sidecar(bf, q, sc, 64))
    load(layer, _pack(0, 8))
    method.process_weights_after_loading(layer)
    assert layer._fp8_huff.pack is None and layer._fp8_huff.leader is None
    assert vfh._leader_prefix("model.layers.2.self_attn.qkv_proj") == "model.layers.2.self_attn.o_proj"
    assert vfh._leader_prefix("model.layers.2.mlp.down_proj") == "model.layers.2.self_attn.o_proj"
    assert vfh._leader_prefix("lm_head") is None and vfh._leader_prefix("") is None


def test_scratch_tokens_separate_layers_captures_and_forward_passes():
    """A buffer's token names the layer state, the capture id and the forward
    context of the last decode enqueued into it; a packed block reuses its
    leader's weight only under the same three."""
    pool = vfh.ScratchPool()
    buf = torch.empty(4, dtype=torch.bfloat16)
    a, b = object(), object()
    fwd1, fwd2 = object(), object()
    assert not pool.holds(buf, (a, 0, None))
    pool.mark(buf, (a, 0, fwd1))
    assert pool.holds(buf, (a, 0, fwd1))
    assert not pool.holds(buf, (b, 0, fwd1))      # another layer decoded since
    assert not pool.holds(buf, (a, 7, fwd1))      # inside a capture: eager contents are not the graph's
    assert not pool.holds(buf, (a, 0, fwd2))      # the next forward pass
    pool.mark(buf, (a, 7, None))
    assert pool.holds(buf, (a, 7, None)) and not pool.holds(buf, (a, 8, None))  # another capture
    pool.clear()
    assert not pool.holds(buf, (a, 7, None))


def test_apply_rejects_cpu_and_bad_dtypes():
    layer, method = make_layer("p", [8], 8)
    with pytest.raises(ValueError, match="requires CUDA tensors"):
        method.apply(layer, torch.zeros(2, 8, dtype=torch.bfloat16))


# ---------------------------------------------------------------------------- GPU
DEV = "cuda:0"


def _to(tensors, dev):
    return {k: v.to(dev) for k, v in tensors.items()}


@pytest.mark.gpu
def test_apply_merged_qkv_matches_exact_weights():
    k = 2048
    parts = [synth(256, k, seed=200), synth(64, k, seed=201), synth(64, k, seed=202)]
    layer, method = make_layer("model.layers.3.self_attn.qkv_proj", [256, 64, 64], k)
    for sid, (bf, q, sc) in zip(("q", "k", "v"), parts):
        load(layer, _to(stored_sidecar(bf, q, sc), DEV), sid)
    method.process_weights_after_loading(layer)
    w = torch.from_numpy(np.concatenate([p[0] for p in parts])).view(torch.bfloat16).to(DEV)
    got_w = method.decoded_weight(layer, k)
    torch.cuda.synchronize()
    assert torch.equal(got_w.view(torch.uint16), w.view(torch.uint16))
    g = torch.Generator(device="cpu").manual_seed(5)
    for t in (1, 16, 128):
        x = torch.randn((t, k), generator=g).to(torch.bfloat16).to(DEV)
        bias = torch.randn(384, generator=g).to(torch.bfloat16).to(DEV)
        out = method.apply(layer, x, bias)
        ref = torch.matmul(x, w.t()) + bias
        assert out.shape == (t, 384)
        assert torch.allclose(out.float(), ref.float(), rtol=1e-2, atol=1e-2)
    x16 = torch.randn((4, k), generator=g).to(torch.float16).to(DEV)
    out16 = method.apply(layer, x16)
    assert out16.dtype == torch.float16
    assert torch.allclose(out16.float(), torch.matmul(x16, w.to(torch.float16).t()).float(), rtol=1e-2, atol=1e-2)
    empty = method.apply(layer, torch.empty((0, k), dtype=torch.bfloat16, device=DEV))
    assert empty.shape == (0, 384)


@pytest.mark.gpu
def test_prefetch_on_side_stream():
    k = 1024
    bf, q, sc = synth(512, k, seed=210)
    layer, method = make_layer("model.layers.0.self_attn.o_proj", [512], k)
    load(layer, _to(stored_sidecar(bf, q, sc), DEV))
    method.process_weights_after_loading(layer)
    w = torch.from_numpy(bf).view(torch.bfloat16).to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    method.prefetch(layer, k, side, slot=1)
    x = torch.randn((8, k), device=DEV).to(torch.bfloat16)
    out = method.apply(layer, x)
    torch.cuda.synchronize()
    assert torch.allclose(out.float(), torch.matmul(x, w.t()).float(), rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_plans_built_at_load_and_reused_by_apply(monkeypatch):
    """process_weights_after_loading builds the layer's plan; apply() and
    prefetch() (into the relocated slot 1) launch it without building another."""
    k = 1024
    parts = [synth(128, k, seed=220), synth(64, k, seed=221)]
    layer, method = make_layer("model.layers.1.mlp.gate_up_proj", [128, 64], k)
    for sid, (bf, q, sc) in zip(("gate", "up"), parts):
        load(layer, _to(stored_sidecar(bf, q, sc), DEV), sid)
    method.process_weights_after_loading(layer)
    st = layer._fp8_huff
    plan = st.plan
    assert plan is not None and st.weight.shape == (192, k)
    w = torch.from_numpy(np.concatenate([p[0] for p in parts])).view(torch.bfloat16).to(DEV)
    x = torch.randn((4, k), device=DEV).to(torch.bfloat16)
    for _ in range(2):
        out = method.apply(layer, x)
        assert layer._fp8_huff.plan is plan
        assert torch.allclose(out.float(), torch.matmul(x, w.t()).float(), rtol=1e-2, atol=1e-2)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    method.prefetch(layer, k, side, slot=1)
    slot1 = layer._fp8_huff.pending[1]
    assert slot1.data_ptr() != st.weight.data_ptr()
    out = method.apply(layer, x)
    torch.cuda.synchronize()
    assert torch.equal(slot1.view(torch.uint16), w.view(torch.uint16))
    assert torch.allclose(out.float(), torch.matmul(x, w.t()).float(), rtol=1e-2, atol=1e-2)
    from mpserve_amd.mpserve_cuda import read_status

    assert read_status(torch.device(DEV)) == 0


@pytest.mark.gpu
def test_launches_on_two_streams_are_ordered():
    """A layer decoded on the current stream and, right after, on a side stream
    (a prefetch into slot 1) launches its plan on two streams; the plan's work
    queue is shared, so the second launch waits for the first. Both results are
    exact every round, with no synchronisation between the two launches."""
    k = 4096
    bf, q, sc = synth(2048, k, seed=230)
    layer, method = make_layer("model.layers.2.self_attn.o_proj", [2048], k)
    load(layer, _to(stored_sidecar(bf, q, sc), DEV))
    method.process_weights_after_loading(layer)
    w = torch.from_numpy(bf).view(torch.bfloat16).to(DEV)
    side = torch.cuda.Stream()
    w1 = method.decoded_weight(layer, slot=1, stream=side)
    torch.cuda.synchronize()
    for rnd in range(4):
        layer._fp8_huff.weight.zero_()
        w1.zero_()
        torch.cuda.synchronize()
        w0 = method.decoded_weight(layer)                      # current stream
        assert method.decoded_weight(layer, slot=1, stream=side).data_ptr() == w1.data_ptr()  # side stream
        method.decoded_weight(layer)                           # and back
        torch.cuda.synchronize()
        assert torch.equal(w0.view(torch.uint16), w.view(torch.uint16)), rnd
        assert torch.equal(w1.view(torch.uint16), w.view(torch.uint16)), rnd
    assert layer._fp8_huff.plan.read_status() == 0


@pytest.mark.gpu
def test_cache_mode_decodes_once_at_load(monkeypatch):
    monkeypatch.setenv("MPSERVE_FP8_HUFFMAN_CACHE", "1")
    k = 512
    bf, q, sc = synth(96, k, seed=230)
    layer, method = make_layer("model.layers.2.self_attn.o_proj", [96], k)
    load(layer, _to(stored_sidecar(bf, q, sc), DEV))
    method.process_weights_after_loading(layer)
    torch.cuda.synchronize()
    st = layer._fp8_huff
    assert st.cached and torch.equal(st.weight.view(torch.uint16).cpu(), torch.from_numpy(bf))
    st.weight.view(torch.int16)[0, 0] = 12345  # a marker: apply() must not decode again
    x = torch.randn((2, k), device=DEV).to(torch.bfloat16)
    method.apply(layer, x)
    torch.cuda.synchronize()
    assert int(st.weight.view(torch.int16)[0, 0]) == 12345


@pytest.mark.gpu
def test_packed_block_layers_use_the_leaders_rows():
    """A layer with huff_attn_block_row_* multiplies by its rows of the block
    leader's (o_proj) decoded weight (reference :559-655)."""
    k = 1024
    bf, q, sc = synth(384, k, seed=240)  # the leader's packed weight: qkv rows 0..255, gate rows 256..383
    leader, lm = make_layer("model.layers.5.self_attn.o_proj", [384], k)
    load(leader, _to(stored_sidecar(bf, q, sc), DEV))
    leader.quant_method = lm
    lm.process_weights_after_loading(leader)
    w = torch.from_numpy(bf).view(torch.bfloat16).to(DEV)
    packed = []
    for prefix, start, rows in (("model.layers.5.self_attn.qkv_proj", 0, 256), ("model.layers.5.mlp.gate_proj", 256, 128)):
        layer, method = make_layer(prefix, [rows], k)
        t = {"huff_attn_block_row_start_i32": torch.tensor([start], dtype=torch.int32),
             "huff_attn_block_row_len_i32": torch.tensor([rows], dtype=torch.int32)}
        load(layer, _to(t, DEV))
        method.process_weights_after_loading(layer)
        assert layer._fp8_huff.pack == (start, rows) and layer._fp8_huff.plan is None
        packed.append((layer, method, start, rows))
    x = torch.randn((3, k), device=DEV).to(torch.bfloat16)
    for layer, method, start, rows in packed:
        out = method.apply(layer, x)
        assert out.shape == (3, rows)
        assert torch.allclose(out.float(), torch.matmul(x, w[start:start + rows].t()).float(), rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_packed_leader_with_its_own_rows_decodes_once_per_forward():
    """o_proj leads a packed block and carries pack rows itself: it multiplies by
    its own rows, qkv and gate by theirs, all of the leader's exact decoded
    weight; the leader's plan launches once per forward pass of the block
    (reference :559-587, :628-655), again after another layer of the same size
    has been decoded into the shared scratch buffer."""
    k = 1024
    bf, q, sc = synth(512, k, seed=250)  # qkv rows 0..255, o_proj 256..383, gate 384..511
    leader, lm = make_layer("model.layers.6.self_attn.o_proj", [128], k)
    load(leader, _to(stored_sidecar(bf, q, sc), DEV))
    load(leader, _to(_pack(256, 128), DEV))
    lm.process_weights_after_loading(leader)
    st = leader._fp8_huff
    assert st.plan is not None and st.pack == (256, 128) and st.weight.shape == (512, k)
    launches = {"n": 0}
    real_decode = st.plan.decode

    def counted(stream=None):
        launches["n"] += 1
        return real_decode(stream)

    st.plan.decode = counted
    w = torch.from_numpy(bf).view(torch.bfloat16).to(DEV)
    members = []
    for prefix, start, rows in (("model.layers.6.self_attn.qkv_proj", 0, 256), ("model.layers.6.mlp.gate_proj", 384, 128)):
        layer, method = make_layer(prefix, [rows], k)
        load(layer, _to(_pack(start, rows), DEV))
        method.process_weights_after_loading(layer)
        members.append((layer, method, start, rows))
    order = [members[0], (leader, lm, 256, 128), members[1]]
    # another layer of the same size shares the leader's scratch buffer
    other_bf, other_q, other_sc = synth(512, k, seed=251)
    other, om = make_layer("model.layers.7.self_attn.o_proj", [512], k)
    load(other, _to(stored_sidecar(other_bf, other_q, other_sc), DEV))
    om.process_weights_after_loading(other)
    assert other._fp8_huff.weight.data_ptr() == st.weight.data_ptr()
    x = torch.randn((5, k), device=DEV).to(torch.bfloat16)
    for fwd in range(3):
        launches["n"] = 0
        for layer, method, start, rows in order:
            got_w = method._weight_for_apply(layer)
            assert torch.equal(got_w.view(torch.uint16), w[start:start + rows].view(torch.uint16)), (fwd, layer.prefix)
            out = method.apply(layer, x)
            assert out.shape == (5, rows)
            ref = torch.matmul(x.float(), w[start:start + rows].float().t())
            assert torch.allclose(out.float(), ref, rtol=2e-2, atol=2e-2), (fwd, layer.prefix)
        assert launches["n"] == 1, f"forward {fwd}: the leader decoded {launches['n']} times"
        om.apply(other, x)  # the next layer of this size overwrites the scratch buffer
    torch.cuda.synchronize()
    assert st.plan.read_status() == 0
