"""The committed golden sidecars of tests/golden/ (written by tests/golden/make_fixtures.py).

CPU: the oracle still builds every fixture byte for byte, and decodes it back
to the input. GPU: the HIP builder gives the same 17 arrays, and the HIP
decoder (one call per tensor, and one plan over all of them) gives the input
BF16 bits. Integer work, so the bar is equality.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import NP_DTYPES, decode_args, to_torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))
NAMES = sorted(MANIFEST)
DEV = "cuda:0"


def _load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as z:
        arrays = {k: z[k] for k in z.files}
    side = {k[3:]: v for k, v in arrays.items() if k.startswith("sc_")}
    side = {k: side[k] for k in NP_DTYPES}  # the reference's key order
    return arrays["in_bf16"], arrays["in_fp8"], arrays["in_scales"], side


def _same(got, ref):
    assert list(got) == list(ref)
    for key in ref:
        assert got[key].dtype == NP_DTYPES[key], (key, got[key].dtype)
        assert got[key].shape == ref[key].shape, (key, got[key].shape, ref[key].shape)
        assert np.array_equal(got[key], ref[key]), f"{key}: {(got[key] != ref[key]).sum()} entries differ"


def test_fixture_set_covers_the_paths():
    m = MANIFEST
    assert any(v["esc_keys"] > 0 for v in m.values())
    assert {v["scale_mode"] for v in m.values()} >= {"row", "scalar", "block2d"}
    assert any(v["m"] < v["threads_per_block"] for v in m.values())          # col_len < k
    ps = {v["m"] // 1024 for v in m.values() if v["threads_per_block"] == 1024 and v["m"] % 1024 == 0}
    assert {2, 4, 14} <= ps                                                   # k = 1024: P < 4, slab, wrap


@pytest.mark.parametrize("name", NAMES)
def test_oracle_rebuilds_fixture(name):
    bf, q, sc, ref = _load(name)
    info = MANIFEST[name]
    got, stats = oracle.encode(bf, q, sc, info["max_len"], info["threads_per_block"], with_stats=True)
    _same(got, ref)
    assert stats["esc_keys"] == info["esc_keys"] and stats["esc_elements"] == info["esc_elements"]
    assert np.array_equal(oracle.decode(ref, q, info["n"], info["m"], info["max_len"]), bf)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_gpu_build_matches_fixture(name):
    import MPServe_cuda

    bf, q, sc, ref = _load(name)
    info = MANIFEST[name]
    out = MPServe_cuda.huffman_build_fp8_decode_tables(
        torch.from_numpy(bf).view(torch.bfloat16), torch.from_numpy(q), torch.from_numpy(sc),
        max_len=info["max_len"], threads_per_block=info["threads_per_block"])
    _same({k: v.cpu().numpy() for k, v in out.items()}, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_gpu_decode_matches_fixture(name):
    import MPServe_cuda
    from mpserve_amd.mpserve_cuda import read_status

    bf, q, _, ref = _load(name)
    read_status(torch.device(DEV))
    q_t = torch.from_numpy(q).to(DEV)
    out = MPServe_cuda.huffman_decode_fp8(*decode_args(to_torch(ref, DEV), q_t))
    torch.cuda.synchronize()
    assert np.array_equal(out.view(torch.uint16).cpu().numpy(), bf)
    assert read_status(torch.device(DEV)) == 0


@pytest.mark.gpu
def test_gpu_plan_decodes_all_fixtures():
    from mpserve_amd.decode import DecodePlan
    from mpserve_amd.mpserve_cuda import read_status

    items, refs = [], []
    for name in NAMES:
        bf, q, _, ref = _load(name)
        q_t = torch.from_numpy(q).to(DEV)
        items.append((q_t, to_torch(ref, DEV), torch.empty(q.shape, dtype=torch.bfloat16, device=DEV)))
        refs.append(bf)
    read_status(torch.device(DEV))
    plan = DecodePlan(items)
    for _ in range(2):
        for _, _, o in items:
            o.zero_()
        plan.decode()
        torch.cuda.synchronize()
        for (_, _, o), bf in zip(items, refs):
            assert np.array_equal(o.view(torch.uint16).cpu().numpy(), bf)
    assert plan.read_status() == 0
    assert read_status(torch.device(DEV)) == 0  # plans flag into their own word
