"""Host logic of the per-sidecar plan cache behind huffman_decode_fp8 (no GPU:
the device plan is replaced by a stand-in that records its lifetime)."""
import torch

import mpserve_amd.mpserve_cuda as mc


class _StandInPlan:
    made = 0

    def __init__(self, desc, stream):
        _StandInPlan.made += 1
        self.closed = False

    def close(self):
        self.closed = True


def _sidecar():
    return [torch.zeros(4, dtype=torch.int64) for _ in range(11)]


def _args(ts):
    # a fresh dtype view of the bitstream on every call, as apply() passes it
    return tuple([ts[0], ts[1].view(torch.uint64)] + ts[2:])


def test_plan_built_on_second_sighting_and_reused(monkeypatch):
    monkeypatch.setattr(mc, "_TensorPlan", _StandInPlan)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    c = mc._SidecarPlans(capacity=4)
    dev = torch.device("cuda", 0)
    ts = _sidecar()
    assert c.get(_args(ts), 4, 1, None, dev, 0) is None  # first call: whole buckets
    p = c.get(_args(ts), 4, 1, None, dev, 0)
    assert isinstance(p, _StandInPlan)
    assert c.get(_args(ts), 4, 1, None, dev, 0) is p
    assert c.get(_args(ts), 2, 2, None, dev, 0) is None  # another shape is another sidecar


def test_in_place_write_and_free_invalidate(monkeypatch):
    monkeypatch.setattr(mc, "_TensorPlan", _StandInPlan)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    c = mc._SidecarPlans(capacity=4)
    dev = torch.device("cuda", 0)
    ts = _sidecar()
    c.get(_args(ts), 4, 1, None, dev, 0)
    p = c.get(_args(ts), 4, 1, None, dev, 0)
    ts[1].view(torch.uint64)  # views share the version counter ...
    ts[1].fill_(7)            # ... so a write through the base invalidates
    assert c.get(_args(ts), 4, 1, None, dev, 0) is None and p.closed
    p2 = c.get(_args(ts), 4, 1, None, dev, 0)
    assert isinstance(p2, _StandInPlan) and not p2.closed
    # a different storage at the key's addresses (simulated: same key, new tensor objects)
    entry = next(iter(c._entries.values()))
    import weakref

    entry.refs[4] = weakref.ref(torch.zeros(1).untyped_storage())  # dead once the temporary goes
    assert c.get(_args(ts), 4, 1, None, dev, 0) is None and p2.closed


def test_no_plan_built_while_capturing_and_lru_bound(monkeypatch):
    monkeypatch.setattr(mc, "_TensorPlan", _StandInPlan)
    capturing = {"on": True}
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: capturing["on"])
    c = mc._SidecarPlans(capacity=2)
    dev = torch.device("cuda", 0)
    ts = _sidecar()
    c.get(_args(ts), 4, 1, None, dev, 0)
    assert c.get(_args(ts), 4, 1, None, dev, 0) is None  # capturing: no build
    capturing["on"] = False
    p = c.get(_args(ts), 4, 1, None, dev, 0)
    assert isinstance(p, _StandInPlan)
    capturing["on"] = True
    assert c.get(_args(ts), 4, 1, None, dev, 0) is p  # a built plan launches during capture
    others = [_sidecar() for _ in range(2)]
    for o in others:
        c.get(_args(o), 4, 1, None, dev, 0)
    # least recently used entry evicted, but a captured graph may still launch its plan: kept open
    assert len(c) == 2 and not p.closed
    capturing["on"] = False
    for o in others:
        c.get(_args(o), 4, 1, None, dev, 0)
    assert not p.closed  # still kept outside the capture
    c.clear()
    assert len(c) == 0 and p.closed


def test_no_plan_freed_during_capture(monkeypatch):
    """A plan built and launched outside any capture, whose entry is evicted or
    invalidated during a capture, is freed on the next call outside it."""
    monkeypatch.setattr(mc, "_TensorPlan", _StandInPlan)
    capturing = {"on": False}
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: capturing["on"])
    c = mc._SidecarPlans(capacity=1)
    dev = torch.device("cuda", 0)
    ts, other = _sidecar(), _sidecar()
    c.get(_args(ts), 4, 1, None, dev, 0)
    p = c.get(_args(ts), 4, 1, None, dev, 0)
    assert isinstance(p, _StandInPlan)
    capturing["on"] = True
    assert c.get(_args(other), 4, 1, None, dev, 0) is None  # evicts ts's entry during the capture
    assert not p.closed
    ts[2].fill_(3)  # and an invalidation during the capture
    assert c.get(_args(ts), 4, 1, None, dev, 0) is None
    assert not p.closed
    capturing["on"] = False
    c.get(_args(other), 4, 1, None, dev, 0)
    assert p.closed


def test_one_plan_serves_every_stream(monkeypatch):
    """The cache is not keyed by stream: a plan gives each stream its own work queue."""
    monkeypatch.setattr(mc, "_TensorPlan", _StandInPlan)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    c = mc._SidecarPlans(capacity=4)
    dev = torch.device("cuda", 0)
    ts = _sidecar()
    assert c.get(_args(ts), 4, 1, None, dev, 11) is None
    p = c.get(_args(ts), 4, 1, None, dev, 22)
    assert isinstance(p, _StandInPlan)
    assert c.get(_args(ts), 4, 1, None, dev, 33) is p and len(c) == 1


def test_env_switch_turns_cache_off(monkeypatch):
    monkeypatch.setattr(mc, "_TensorPlan", _StandInPlan)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setenv("MPSERVE_DECODE_PLANS", "0")
    c = mc._SidecarPlans(capacity=4)
    ts = _sidecar()
    for _ in range(3):
        assert c.get(_args(ts), 4, 1, None, torch.device("cuda", 0), 0) is None
    assert len(c) == 0
