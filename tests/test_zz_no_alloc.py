"""mps_fp8_decode_batch_noalloc: the allocation-free batched decode, through the C-ABI.

Its output must equal the plan decode's (mps_fp8_plan_create + mps_fp8_plan_decode)
bit for bit, on two calls in a row, the second with a smaller input (the static
scratch keeps the first call's records; the second must not read them). Sizes
beyond the scratch are rejected on the host with a clear error.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import synth, to_torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _items(shapes, seed0):
    items = []
    for i, (n, m, k, scalar) in enumerate(shapes):
        bf, q, sc = synth(n, m, seed=seed0 + i)
        side = oracle.encode(bf, q, sc[:1].copy() if scalar else sc, 7, k)
        items.append((torch.from_numpy(q).to(DEV), to_torch(side, DEV), bf))
    return items


def _noalloc(items, outs):
    from mpserve_amd import _native
    from mpserve_amd.decode import sidecar_decode_args
    from mpserve_amd.mpserve_cuda import _descriptor, _stream_handle

    descs = []
    for (q_t, sc_t, _), o in zip(items, outs):
        args = sidecar_decode_args(q_t, sc_t)
        descs.append(_descriptor(*args[:13], o))
    arr = (_native.MpsFp8Tensor * len(descs))(*descs)
    rc = _native.lib().mps_fp8_decode_batch_noalloc(arr, len(descs), 7, ctypes.c_void_p(_stream_handle(torch.device(DEV))))
    _native.check(rc)


def _plan(items, outs):
    from mpserve_amd.decode import DecodePlan

    plan = DecodePlan([(q_t, sc_t, o) for (q_t, sc_t, _), o in zip(items, outs)])
    plan.decode()
    status = plan.read_status()
    plan.close()
    return status


def test_noalloc_matches_plan_on_two_calls_second_smaller():
    from mpserve_amd.mpserve_cuda import read_status

    big = _items([(256, 8192, 1024, True), (300, 4096, 1024, False), (40, 14336, 1024, False),
                  (129, 1000, 256, False), (7, 100, 1024, False), (64, 2048, 64, False)], 700)
    small = _items([(33, 4096, 1024, False), (5, 9, 3, False)], 720)
    read_status(torch.device(DEV))
    for name, items in (("first call", big), ("second call, smaller", small)):
        print(f"[noalloc] {name}: {len(items)} tensors", flush=True)
        want = [torch.zeros(q.shape, dtype=torch.bfloat16, device=DEV) for q, _, _ in items]
        got = [torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=DEV) for q, _, _ in items]
        assert _plan(items, want) == 0
        _noalloc(items, got)
        torch.cuda.synchronize()
        for (_, _, bf), w, g in zip(items, want, got):
            assert torch.equal(g.view(torch.uint16), w.view(torch.uint16)), name
            assert np.array_equal(g.view(torch.uint16).cpu().numpy(), bf), name
        assert read_status(torch.device(DEV)) == 0


def test_noalloc_rejects_inputs_beyond_its_scratch():
    from mpserve_amd import _native

    d = _native.MpsFp8Tensor()
    arr = (_native.MpsFp8Tensor * 1)(d)
    with pytest.raises(ValueError, match="static scratch"):
        _native.check(_native.lib().mps_fp8_decode_batch_noalloc(arr, 1025, 7, None))
    from mpserve_amd.decode import sidecar_decode_args
    from mpserve_amd.mpserve_cuda import _descriptor

    q_t, sc_t, _ = _items([(4, 64, 8, False)], 730)[0]
    out = torch.empty(q_t.shape, dtype=torch.bfloat16, device=DEV)
    args = sidecar_decode_args(q_t, sc_t)
    big = _descriptor(*args[:13], out)
    big.num_buckets = 1 << 20  # more work records than the scratch holds (checked before any launch)
    arr = (_native.MpsFp8Tensor * 1)(big)
    with pytest.raises(ValueError, match="static scratch"):
        _native.check(_native.lib().mps_fp8_decode_batch_noalloc(arr, 1, 7, None))


def test_noalloc_refuses_a_capturing_stream():
    """Under graph capture the descriptor copy from the caller's host array would
    replay from freed host memory: the call is refused on the host, before any
    copy or launch, and the capture itself stays usable (not replayed here)."""
    from mpserve_amd import _native
    from mpserve_amd.decode import sidecar_decode_args
    from mpserve_amd.mpserve_cuda import _descriptor, _stream_handle

    q_t, sc_t, bf = _items([(64, 1024, 1024, False)], 740)[0]
    out = torch.empty(q_t.shape, dtype=torch.bfloat16, device=DEV)
    arr = (_native.MpsFp8Tensor * 1)(_descriptor(*sidecar_decode_args(q_t, sc_t)[:13], out))
    x = torch.zeros(8, device=DEV)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    rc = None
    with torch.cuda.graph(g):
        x.add_(1)
        rc = _native.lib().mps_fp8_decode_batch_noalloc(arr, 1, 7, ctypes.c_void_p(_stream_handle(torch.device(DEV))))
        msg = _native.lib().mps_last_error().decode()
    assert rc == _native.MPS_ERR_INVALID_ARGUMENT and "capturing" in msg
    torch.cuda.synchronize()
    # outside the capture the same call runs
    _noalloc([(q_t, sc_t, bf)], [out])
    torch.cuda.synchronize()
    assert np.array_equal(out.view(torch.uint16).cpu().numpy(), bf)
