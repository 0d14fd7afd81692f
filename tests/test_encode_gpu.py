"""GPU sidecar builder: byte-identical to the CPU oracle on every output, and
round-trips through the GPU decoder."""
import numpy as np
import pytest
import torch

import oracle
from tests.helpers import NP_DTYPES, decode_args, synth, to_torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _gpu_build(bf, q, scales, L=7, k=1024, on_device=False):
    import MPServe_cuda

    bf_t = torch.from_numpy(np.ascontiguousarray(bf)).view(torch.bfloat16)
    q_t = torch.from_numpy(np.ascontiguousarray(q))
    sc_t = torch.from_numpy(np.ascontiguousarray(scales))
    if on_device:
        bf_t, q_t, sc_t = bf_t.to(DEV), q_t.to(DEV), sc_t.to(DEV)
    out = MPServe_cuda.huffman_build_fp8_decode_tables(bf_t, q_t, sc_t, max_len=L, threads_per_block=k)
    return {k2: v.cpu().numpy() for k2, v in out.items()}


def _assert_same(got, ref):
    assert list(got.keys()) == list(ref.keys())
    for key in ref:
        g, r = got[key], ref[key]
        assert g.dtype == NP_DTYPES[key], (key, g.dtype)
        assert g.shape == r.shape, (key, g.shape, r.shape)
        assert np.array_equal(g, r), f"{key}: {(g != r).sum()} differing entries"


@pytest.mark.parametrize("n,m,k,seed", [
    (1, 1, 1, 0), (3, 5, 7, 1), (7, 100, 1024, 2), (64, 256, 64, 3), (300, 513, 1024, 4),
    (129, 1000, 256, 5), (1024, 4096, 1024, 6),
])
def test_build_matches_oracle_per_row(n, m, k, seed):
    bf, q, sc = synth(n, m, seed=seed)
    _assert_same(_gpu_build(bf, q, sc, 7, k), oracle.encode(bf, q, sc, 7, k))


def test_build_matches_oracle_full_size_cfg1():
    bf, q, sc = synth(4096, 4096, seed=0)
    got = _gpu_build(bf, q, sc, 7, 1024, on_device=True)
    _assert_same(got, oracle.encode(bf, q, sc, 7, 1024))


@pytest.mark.parametrize("L", [1, 2, 3, 5, 7, 9, 12, 15])
def test_build_all_max_len(L):
    bf, q, sc = synth(40, 300, seed=10 + L)
    _assert_same(_gpu_build(bf, q, sc, L, 128), oracle.encode(bf, q, sc, L, 128))


def test_build_scalar_and_block2d_scales():
    bf, q, sc = synth(300, 640, seed=20)
    _assert_same(_gpu_build(bf, q, sc[:1].copy(), 7, 512), oracle.encode(bf, q, sc[:1].copy(), 7, 512))
    rng = np.random.default_rng(21)
    blocks = rng.integers(0x2000, 0x2008, size=(3, 5), dtype=np.uint16)
    bf2, q2, _ = synth(192, 640, seed=22)
    _assert_same(_gpu_build(bf2, q2, blocks, 7, 1024), oracle.encode(bf2, q2, blocks, 7, 1024))


def _esc_inputs(n, m, seed, collision=False):
    rng = np.random.default_rng(seed)
    bf = rng.integers(0x3C00, 0x3C00 + 700, size=(n, m)).astype(np.uint16)
    head = rng.random((n, m)) < 0.4
    bf[head] = (0x3C00 + rng.integers(0, 25, size=int(head.sum()))).astype(np.uint16)
    if collision:
        bf.flat[rng.choice(bf.size, 5, replace=False)] = 0
    q = np.full((n, m), 0x40, dtype=np.uint8)
    q[:, ::5] = 0x41
    return bf, q, np.array([0x1C00], dtype=np.uint16)


@pytest.mark.parametrize("collision", [False, True])
def test_build_esc_keys(collision):
    bf, q, sc = _esc_inputs(150, 700, 30 + collision, collision)
    ref, st = oracle.encode(bf, q, sc, 7, 1024, with_stats=True)
    assert st["esc_keys"] >= 1
    _assert_same(_gpu_build(bf, q, sc, 7, 1024), ref)


def test_gpu_build_then_gpu_decode_roundtrip():
    import MPServe_cuda

    n, m = 2048, 4096
    bf, q, sc = synth(n, m, seed=40)
    bf_t = torch.from_numpy(bf).view(torch.bfloat16).to(DEV)
    q_t = torch.from_numpy(q).to(DEV)
    side = MPServe_cuda.huffman_build_fp8_decode_tables(bf_t, q_t, torch.from_numpy(sc).to(DEV), max_len=7,
                                                        threads_per_block=1024)
    assert all(v.is_cuda for v in side.values())
    out = MPServe_cuda.huffman_decode_fp8(*decode_args(side, q_t))
    assert torch.equal(out.view(torch.uint16), bf_t.view(torch.uint16))


def test_build_error_messages():
    import MPServe_cuda

    bf = torch.zeros((4, 8), dtype=torch.bfloat16)
    q = torch.zeros((4, 8), dtype=torch.uint8)
    with pytest.raises(ValueError, match="unsupported scales shape"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf, q, torch.zeros(3, dtype=torch.uint16), 7, 16)
    with pytest.raises(ValueError, match="bucket packing requires scales to be scalar, per-row"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf, q, torch.zeros(32, dtype=torch.uint16), 7, 16)
    with pytest.raises(ValueError, match="bucket packing requires bf16_params to be 2D"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf.reshape(-1), q.reshape(-1),
                                                     torch.zeros(1, dtype=torch.uint16), 7, 16)
