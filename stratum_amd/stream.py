"""Per-layer NF4 stream-in: host-to-device copy, dequantization and the layer's
compute on three streams.

The reference overlaps "upload + dequantize layer i+1" with "compute layer i"
by running ``ensure_weights`` for the next layer on a side stream and fencing
the default stream on an event (``stratum/stage.py:93-121``); the copy and the
dequantization of one layer are serial there, and the dequantized tensors are
made on the side stream but read on the default stream without a
``record_stream``, so freeing them right after use lets the caching allocator
hand their blocks to the next side-stream allocation while the reads are still
queued.

Here (``_LayerFeeder``):

* the packed payloads of the next ``lookahead`` layers are copied on the
  device's persistent copy stream (``prefetch_weights``);
* each layer is dequantized on a dequant stream once its copy has landed
  (event wait on the GPU, no host sync) -- FP16-staged and plain parameters
  and buffers are brought over by the same ``ensure_weights`` call;
* every materialised tensor is ``record_stream``-ed on the consumer stream
  (the stream that runs the layers), and the consumer waits on a per-layer
  event before the layer runs.

``NF4LayerStream`` exposes this as an iterator; ``NF4DeviceStage`` is a
drop-in for ``stratum.stage.DeviceStage`` (same constructor and
``forward_range`` signature and fence protocol).
"""

from __future__ import annotations

import sys
from contextlib import nullcontext
from typing import Any, Callable, Iterator, Optional, Sequence

import torch
import torch.nn as nn

from .upload import ensure_weights, free_weights, prefetch_weights


class _LayerFeeder:
    """Materialises layers of a list on one device ahead of a consumer stream."""

    def __init__(self, layers: Sequence[nn.Module], device_id: int, lookahead: int,
                 dequant_stream: "torch.cuda.Stream", consumers: Sequence["torch.cuda.Stream"]):
        if lookahead < 1:
            raise ValueError("lookahead must be >= 1")
        self.layers, self.device_id, self.lookahead = layers, device_id, lookahead
        self.dequant_stream, self.consumers = dequant_stream, list(consumers)
        self.copies: dict = {}   # layer index -> NF4Prefetch in flight
        self.ready: dict = {}    # layer index -> event: materialised

    def _copy(self, i: int) -> None:
        if 0 <= i < len(self.layers) and i not in self.copies and i not in self.ready:
            self.copies[i] = prefetch_weights(self.layers[i], self.device_id)

    def _materialise(self, i: int) -> None:
        if i in self.ready or not 0 <= i < len(self.layers):
            return
        self._copy(i)
        readers = self.consumers
        with torch.cuda.stream(self.dequant_stream):
            self.copies.pop(i).finalize(consumers=readers)
            ensure_weights(self.layers[i], self.device_id, consumers=readers)
            done = torch.cuda.Event()
            done.record(self.dequant_stream)
        self.ready[i] = done

    def mark_ready(self, i: int, event: Optional["torch.cuda.Event"]) -> None:
        """Layer i was materialised by the caller; *event* fences it (None: already visible)."""
        self.copies.pop(i, None)
        self.ready[i] = event

    def before(self, i: int) -> None:
        """Queue what layer i needs and fence the consumer on it; layer i + 1 is
        dequantized meanwhile and the next copies are started."""
        for j in range(i, i + 1 + self.lookahead):
            self._copy(j)
        self._materialise(i)
        self._materialise(i + 1)
        event = self.ready.pop(i)
        if event is not None:
            for c in self.consumers:
                c.wait_event(event)


class NF4LayerStream:
    """Iterate over ``layers`` with each layer's staged weights materialised on
    ``cuda:<device_id>`` just in time::

        for i, layer in NF4LayerStream(stage.layers, device_id=0):
            hidden = layer(hidden)

    At each yield the current stream is fenced on layer i's materialisation.
    When the loop body returns the layer's weights are freed (``free_after=False``
    keeps them); that is safe with kernels still queued, since every tensor was
    handed over to this stream. All streams keep the default priority.
    """

    def __init__(self, layers: Sequence[nn.Module], device_id: int = 0, *, lookahead: int = 1,
                 free_after: bool = True):
        if lookahead < 1:
            raise ValueError("lookahead must be >= 1")
        self.layers = list(layers)
        self.device_id = device_id
        self.lookahead = lookahead
        self.free_after = free_after
        self.dequant_stream = torch.cuda.Stream(device=device_id)

    def __len__(self) -> int:
        return len(self.layers)

    def __iter__(self) -> Iterator[tuple[int, nn.Module]]:
        feeder = _LayerFeeder(self.layers, self.device_id, self.lookahead, self.dequant_stream,
                              [torch.cuda.current_stream(self.device_id)])
        for i, layer in enumerate(self.layers):
            feeder.before(i)
            yield i, layer
            if self.free_after:
                free_weights(layer)


class NF4DeviceStage(nn.Module):
    """A contiguous slice of decoder layers on one device: drop-in for
    ``stratum.stage.DeviceStage`` (``stratum/stage.py:14-140``).

    Same constructor, ``set_timing_recorder`` and ``forward_range`` signature and
    semantics: without ``param_stream`` the layers run as they are (the caller
    materialised them); with it, layer weights are materialised per layer ahead
    of the compute, ``first_layer_fence`` (if given) fences a first layer the
    caller already uploaded, and the current stream waits on each layer's fence.
    The materialisation itself is the three-stream one of this module:
    ``param_stream`` is the dequant stream, payload copies run on the device's
    copy stream ``lookahead`` layers ahead, and every tensor is handed over to
    the consuming stream. ``free_after_use=True`` frees each layer's staged
    weights right after its forward is queued. ``recompute`` is the predicate
    that labels a pass as recompute for ``iter_timer`` (see ``_action``).
    """

    def __init__(self, layers: list, device_id: int, *, lookahead: int = 1, free_after_use: bool = False,
                 recompute: Optional[Callable[[], bool]] = None):
        super().__init__()
        self.device_id = device_id
        self.layers = nn.ModuleList(layers)
        self.timing_recorder = None
        self.layer_start = 0
        self.lookahead = lookahead
        self.free_after_use = free_after_use
        self.recompute = recompute

    def _action(self) -> str:
        """``"re"`` inside a recompute pass, else ``"fwd"`` -- the label the
        reference gives ``iter_timer.time_fwd`` (``stratum/stage.py:123``), whose
        scheduler keeps separate recompute estimates. The predicate is the
        constructor's ``recompute``; without one, the ``doing_recompute`` of a
        ``stratum.context`` module the host program has already loaded (this
        package never imports it); with neither, every pass is a forward."""
        pred = self.recompute
        if pred is None:
            ctx = sys.modules.get("stratum.context")
            pred = getattr(ctx, "doing_recompute", None)
        return "re" if pred is not None and pred() else "fwd"

    def set_timing_recorder(self, recorder, *, layer_start: int = 0) -> None:
        """Attach timing metadata for per-layer forward spans (``recorder.span``)."""
        self.timing_recorder = recorder
        self.layer_start = layer_start

    def _span(self, **fields: Any):
        if self.timing_recorder is None:
            return nullcontext()
        return self.timing_recorder.span("layer_forward", device_id=self.device_id, **fields)

    def forward_range(self, input_data: tuple, *, local_start: int = 0, local_stop: Optional[int] = None,
                      iter_timer=None, param_stream: Optional["torch.cuda.Stream"] = None,
                      first_layer_fence: Optional["torch.cuda.Event"] = None) -> tuple:
        """Run layers [local_start, local_stop) of this stage on *input_data*
        (each layer takes and returns the tuple)."""
        stop = len(self.layers) if local_stop is None else local_stop
        if local_start < 0 or stop > len(self.layers) or local_start >= stop:
            raise ValueError(f"invalid stage layer range {local_start}:{stop} for {len(self.layers)} layers")
        run = [self.layers[i] for i in range(local_start, stop)]
        feeder = None
        if param_stream is not None and torch.cuda.is_available():
            # the stream that runs the layers waits on each layer's fence; so does
            # the device's default stream when it is another one, as the reference
            # fences the default stream (stratum/stage.py:121)
            consumers = [torch.cuda.current_stream(self.device_id)]
            default = torch.cuda.default_stream(self.device_id)
            if default != consumers[0]:
                consumers.append(default)
            feeder = _LayerFeeder(run, self.device_id, self.lookahead, param_stream, consumers)
            if first_layer_fence is not None:
                feeder.mark_ready(0, first_layer_fence)
        for k, layer in enumerate(run):
            if feeder is not None:
                feeder.before(k)
            stage_index = local_start + k
            timed = nullcontext()
            if iter_timer is not None and torch.cuda.is_available():
                timed = iter_timer.time_fwd(self._action(), self.layer_start + stage_index,
                                            torch.cuda.current_stream(self.device_id))
            with timed, self._span(stage_device=self.device_id, layer_index=self.layer_start + stage_index,
                                   stage_layer_index=stage_index):
                input_data = layer(input_data)
            if self.free_after_use:
                free_weights(layer)
        return input_data

    def forward(self, input_data: tuple) -> tuple:
        return self.forward_range(input_data)
