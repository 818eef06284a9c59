"""NF4DeviceStage on the CPU: the pass label handed to ``iter_timer`` and the
range checks of ``forward_range`` (reference: ``stratum/stage.py:59-140``,
which labels a pass ``"re"`` under ``doing_recompute()`` and ``"fwd"``
otherwise, and times it only with CUDA present and a timer given)."""

from __future__ import annotations

import sys
import types
from contextlib import contextmanager

import pytest
import torch
import torch.nn as nn

from stratum_amd.stream import NF4DeviceStage


class _AddOne(nn.Module):
    def forward(self, inp):
        x, n = inp
        return x + 1, n + 1


class _FakeTimer:
    def __init__(self):
        self.calls = []

    @contextmanager
    def time_fwd(self, action, layer_index, stream):
        self.calls.append((action, layer_index, stream))
        yield


@pytest.fixture
def fake_cuda(monkeypatch):
    """CUDA "present" for the timing branch only (no param stream is used)."""
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: f"stream{device}")


def test_recompute_predicate_labels_passes(fake_cuda):
    state = {"re": False}
    stage = NF4DeviceStage([_AddOne() for _ in range(3)], 0, recompute=lambda: state["re"])
    stage.set_timing_recorder(None, layer_start=10)
    timer = _FakeTimer()
    out = stage.forward_range((torch.zeros(2), 0), local_start=1, iter_timer=timer)
    assert out[1] == 2 and torch.equal(out[0], torch.full((2,), 2.0))
    state["re"] = True
    stage.forward_range((torch.zeros(2), 0), iter_timer=timer)
    assert timer.calls == [("fwd", 11, "stream0"), ("fwd", 12, "stream0"),
                           ("re", 10, "stream0"), ("re", 11, "stream0"), ("re", 12, "stream0")]


def test_loaded_host_context_supplies_the_predicate(fake_cuda, monkeypatch):
    """Without a constructor predicate, an already-loaded ``stratum.context``
    (the host pipeline's) decides; without one either, every pass is "fwd"."""
    timer = _FakeTimer()
    stage = NF4DeviceStage([_AddOne()], 0)
    monkeypatch.delitem(sys.modules, "stratum.context", raising=False)
    stage.forward_range((torch.zeros(1), 0), iter_timer=timer)
    ctx = types.ModuleType("stratum.context")
    ctx.flag = True
    ctx.doing_recompute = lambda: ctx.flag
    monkeypatch.setitem(sys.modules, "stratum.context", ctx)
    stage.forward_range((torch.zeros(1), 0), iter_timer=timer)
    ctx.flag = False
    stage.forward_range((torch.zeros(1), 0), iter_timer=timer)
    assert [c[0] for c in timer.calls] == ["fwd", "re", "fwd"]


def test_no_timer_without_cuda():
    timer = _FakeTimer()
    stage = NF4DeviceStage([_AddOne(), _AddOne()], 0, recompute=lambda: True)
    out = stage((torch.zeros(1), 0))
    assert out[1] == 2
    stage.forward_range((torch.zeros(1), 0), iter_timer=timer)
    assert timer.calls == []  # the reference times only with CUDA present


@pytest.mark.parametrize("start,stop", [(-1, 2), (0, 3), (2, 2), (2, 1)])
def test_invalid_ranges(start, stop):
    stage = NF4DeviceStage([_AddOne(), _AddOne()], 0)
    with pytest.raises(ValueError, match="invalid stage layer range"):
        stage.forward_range((torch.zeros(1), 0), local_start=start, local_stop=stop)
