"""Per-layer NF4 stream-in with the host-to-device copy, the dequantization and
the layer's compute on three streams.

The reference overlaps "upload + dequant of layer i+1" with "compute of layer i"
by running ``ensure_weights`` for the next layer on a side stream and fencing
the default stream on an event (``stratum/stage.py:99-121``); upload and
dequantization of one layer are serial on that side stream. Here the packed
payload of layer i+1 (and further, ``lookahead``) is copied on the device's
copy stream (``prefetch_weights``) while layer i is dequantized on a dequant
stream (``ensure_prefetched_weights``) and layer i-1 computes on the default
stream, so the PCIe copy, the HBM-bound dequant kernel and the compute all
overlap. The dequantized tensors are ``record_stream``-ed on the default stream
(the consumer), and ``free_weights`` after use returns them to the caching
allocator safely.
"""

from __future__ import annotations

from typing import Iterator, Sequence

import torch

from .upload import NF4_ATTR, ensure_prefetched_weights, free_weights, prefetch_weights


class NF4LayerStream:
    """Iterate over ``layers`` with each layer's staged weights materialised on
    ``cuda:<device_id>`` just in time.

        for i, layer in NF4LayerStream(stage.layers, device_id=0):
            hidden = layer(hidden)

    At each yield the current stream has been fenced on layer i's dequantization;
    when the loop body returns, the layer's dequantized weights are freed
    (``free_after=False`` keeps them). All streams keep the default priority.
    """

    def __init__(self, layers: Sequence[torch.nn.Module], device_id: int = 0, *, lookahead: int = 1,
                 free_after: bool = True):
        if lookahead < 1:
            raise ValueError("lookahead must be >= 1")
        self.layers = list(layers)
        self.device_id = device_id
        self.device = torch.device(f"cuda:{device_id}")
        self.lookahead = lookahead
        self.free_after = free_after
        self.dequant_stream = torch.cuda.Stream(device=self.device)

    def __len__(self) -> int:
        return len(self.layers)

    def _dequant(self, i: int, pending: dict) -> "torch.cuda.Event":
        with torch.cuda.stream(self.dequant_stream):
            ensure_prefetched_weights(self.layers[i], self.device_id, pending.pop(i))
            ready = torch.cuda.Event()
            ready.record(self.dequant_stream)
        return ready

    def __iter__(self) -> Iterator[tuple[int, torch.nn.Module]]:
        n = len(self.layers)
        if n == 0:
            return
        pending: dict = {}
        ready: dict = {}
        compute = torch.cuda.current_stream(self.device)
        for j in range(min(n, 1 + self.lookahead)):
            pending[j] = prefetch_weights(self.layers[j], self.device_id)
        ready[0] = self._dequant(0, pending)
        for i in range(n):
            for j in range(i + 1, min(n, i + 2 + self.lookahead)):
                if j not in pending and j not in ready:
                    pending[j] = prefetch_weights(self.layers[j], self.device_id)
            if i + 1 < n:  # dequantize the next layer while this one computes
                ready[i + 1] = self._dequant(i + 1, pending)
            compute.wait_event(ready.pop(i))
            for p in self.layers[i].parameters():  # the compute stream is the consumer
                if hasattr(p, NF4_ATTR) and p.data.is_cuda and p.data.numel():
                    p.data.record_stream(compute)
            yield i, self.layers[i]
            if self.free_after:
                free_weights(self.layers[i])
