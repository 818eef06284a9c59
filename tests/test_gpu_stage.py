"""GPU tests of the staged training lifecycle around the fused kernels:

* packed-resident weights: a 2-layer staged module swapped to NF4Linear
  (make_nf4_resident) runs forward, free, recompute and backward with no
  dequantize launch, matching the dequantize lifecycle within tolerance;
* the DeviceStage drop-in (NF4DeviceStage.forward_range with a param stream):
  each layer's weight is read on the consumer stream after a long delay while
  the layer is freed right away and the next layer is dequantized on the side
  stream into a same-size allocation -- every read is bit-exact (the tensors
  are handed over to the consumer stream, so the freed blocks are not reused
  early);
* NF4LayerStream with FP16-staged and NF4 weights in the same layer.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from gpu_checks import assert_gemm_close
from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def oracle_bits(w16):
    x = w16.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    p, a = C.quantize(x, O.DT_F16, 64, "argmin")
    return torch.from_numpy(C.dequantize(p, a, w16.numel(), 64, O.DT_F16).view(np.int16).reshape(w16.shape))


class _MLPBlock(nn.Module):
    def __init__(self, seed, hidden=512, inter=1024):
        super().__init__()
        self.up = nn.Linear(hidden, inter, bias=False, dtype=torch.float16)
        self.down = nn.Linear(inter, hidden, bias=True, dtype=torch.float16)
        with torch.no_grad():
            self.up.weight.copy_(seeded((inter, hidden), seed, 0.02, torch.float16))
            self.down.weight.copy_(seeded((hidden, inter), seed + 1, 0.02, torch.float16))
            self.down.bias.copy_(seeded((hidden,), seed + 2, 0.1, torch.float16))
        self.requires_grad_(False)

    def forward(self, x):
        return x + self.down(torch.nn.functional.gelu(self.up(x)))


def _two_layers():
    from stratum_amd.upload import prepare_nf4
    layers = nn.ModuleList([_MLPBlock(10), _MLPBlock(20)])
    prepare_nf4(layers, verbose=False)
    return layers


def _run(layers, x, dy, before=None, after=None):
    """forward (no graph), free, recompute with grad, backward -- the pipeline's
    step for a frozen stage; returns (output, input gradient)."""
    with torch.no_grad():
        h = x
        for layer in layers:
            if before:
                before(layer)
            h = layer(h)
            if after:
                after(layer)
    out = h.clone()
    xg = x.detach().requires_grad_(True)
    h = xg
    for layer in layers:
        if before:
            before(layer)
        h = layer(h)
    h.backward(dy)
    if after:
        for layer in layers:
            after(layer)
    return out, xg.grad


def test_packed_resident_layers_never_dequantize(cuda, monkeypatch):
    import stratum_amd.upload as U
    from stratum_amd import _lib
    from stratum_amd.nf4_linear import NF4Linear, make_nf4_resident
    monkeypatch.delenv("STRATUM_NF4_FUSED_MAX_ROWS", raising=False)
    x = seeded((512, 512), 1, 1.0, torch.float16).to(cuda)   # 512 rows: the fused kernels' range
    dy = seeded((512, 512), 2, 1.0, torch.float16).to(cuda)

    staged = _two_layers()
    ref_out, ref_dx = _run(staged, x, dy, before=lambda l: U.ensure_weights(l, 0),
                           after=lambda l: U.free_weights(l))

    resident = _two_layers()
    assert make_nf4_resident(resident, 0) == 4
    assert all(isinstance(m, NF4Linear) for blk in resident for m in (blk.up, blk.down))
    calls = []
    for entry in ("stm_nf4_dequantize", "stm_nf4_dequantize_many"):
        real_entry = getattr(_lib.lib(), entry)

        def counting(*a, _real=real_entry, _name=entry):
            calls.append(_name)
            return _real(*a)
        monkeypatch.setattr(_lib.lib(), entry, counting)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        out, dx = _run(resident, x, dy, before=lambda l: U.ensure_weights(l, 0),
                       after=lambda l: U.free_weights(l))
        torch.cuda.synchronize()
    assert calls == [], f"the resident layers called {sorted(set(calls))}"
    names = [e.key for e in prof.key_averages()]
    assert not any("k_dequantize" in n for n in names), names
    if any("k_" in n for n in names):  # the profiler saw device kernels: the fused GEMMs ran
        assert any("k_gemm" in n or "k_gemv" in n for n in names), names
    assert_gemm_close(out, ref_out.float(), torch.float16, "resident forward")
    assert_gemm_close(dx, ref_dx.float(), torch.float16, "resident input gradient")


class _ReadLater(nn.Module):
    """Reads its weight on the consumer stream after a long delay, then frees it
    (host side) while that read is still queued."""

    def __init__(self, seed, n=1024, k=1024):
        super().__init__()
        self.lin = nn.Linear(k, n, bias=False, dtype=torch.float16)
        with torch.no_grad():
            self.lin.weight.copy_(seeded((n, k), seed, 0.02, torch.float16))
        self.requires_grad_(False)

    def forward(self, inp):
        from stratum_amd.upload import free_weights
        x, seen = inp
        torch.cuda._sleep(50_000_000)                       # ~25 ms on the consumer stream
        seen.append(self.lin.weight.view(torch.int16).clone())
        free_weights(self)                                   # freed before the clone has run
        return x, seen


def test_device_stage_forward_range_survives_early_free(cuda):
    from stratum_amd.stream import NF4DeviceStage
    from stratum_amd.upload import prepare_nf4
    layers = [_ReadLater(100 + i) for i in range(4)]
    expect = [oracle_bits(l.lin.weight.data) for l in layers]
    for l in layers:
        prepare_nf4(l, verbose=False)
    stage = NF4DeviceStage(layers, 0)
    param_stream = torch.cuda.Stream()
    for step in range(2):
        _, seen = stage.forward_range((None, []), param_stream=param_stream)
        torch.cuda.synchronize()
        assert len(seen) == 4
        for i, (got, want) in enumerate(zip(seen, expect)):
            assert torch.equal(got.cpu(), want), f"step {step} layer {i}: weight overwritten before it was read"
    # a sub-range with a first layer the caller materialised on the param stream
    from stratum_amd.upload import ensure_weights
    with torch.cuda.stream(param_stream):
        ensure_weights(layers[1], 0)  # handed over to the default stream, the consumer here
        fence = torch.cuda.Event()
        fence.record(param_stream)
    _, seen = stage.forward_range((None, []), local_start=1, local_stop=3, param_stream=param_stream,
                                  first_layer_fence=fence)
    torch.cuda.synchronize()
    assert [torch.equal(s.cpu(), e) for s, e in zip(seen, expect[1:3])] == [True, True]
    with pytest.raises(ValueError):
        stage.forward_range((None, []), local_start=3, local_stop=3)


def test_layer_stream_mixed_nf4_and_fp16_staged(cuda):
    """A layer holding an NF4 weight and an FP16-staged weight, streamed with
    free after each yield and a long-delayed read: both bit-exact every time."""
    from stratum_amd.stream import NF4LayerStream
    from stratum_amd.upload import FP16_ATTR, prepare_fp16_staged, prepare_nf4

    class Mixed(nn.Module):
        def __init__(self, seed):
            super().__init__()
            self.a = nn.Linear(512, 512, bias=False, dtype=torch.float16)
            self.b = nn.Linear(512, 512, bias=False, dtype=torch.float16)
            with torch.no_grad():
                self.a.weight.copy_(seeded((512, 512), seed, 0.02, torch.float16))
                self.b.weight.copy_(seeded((512, 512), seed + 1, 0.02, torch.float16))
            self.requires_grad_(False)

    layers = [Mixed(200 + 2 * i) for i in range(3)]
    expect_a = [oracle_bits(l.a.weight.data) for l in layers]
    expect_b = [l.b.weight.data.clone().view(torch.int16) for l in layers]
    for l in layers:
        prepare_nf4(l.a, verbose=False, min_numel=4096)
        prepare_fp16_staged(l.b, min_numel=4096, verbose=False)
        assert hasattr(l.b.weight, FP16_ATTR)
    for rep in range(2):
        got = []
        for i, layer in NF4LayerStream(layers, device_id=0, lookahead=2):
            torch.cuda._sleep(20_000_000)
            got.append((layer.a.weight.view(torch.int16).clone(), layer.b.weight.view(torch.int16).clone()))
        torch.cuda.synchronize()
        for i, (ga, gb) in enumerate(got):
            assert torch.equal(ga.cpu(), expect_a[i]), f"rep {rep} layer {i} NF4 weight"
            assert torch.equal(gb.cpu(), expect_b[i]), f"rep {rep} layer {i} FP16-staged weight"
        assert all(l.a.weight.numel() == 0 and l.b.weight.numel() == 0 for l in layers)
