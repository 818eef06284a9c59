"""CPU tests of the build-time streaming NF4 staging from a local safetensors
checkpoint (stratum/upload.py:671-904), single file and sharded with an
index, with the GPU quantizer replaced by a recording stub."""

import json
from unittest import mock

import pytest
import torch
import torch.nn as nn
from safetensors.torch import save_file

import stratum_amd.upload as U
from stratum_amd.checkpoint import stream_load_and_quantize_module


class Tiny(nn.Module):
    def __init__(self, device="meta"):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList([nn.Module()])
        lay = self.model.layers[0]
        lay.q_proj = nn.Linear(128, 64, bias=False, device=device, dtype=torch.float16)
        lay.norm = nn.Parameter(torch.empty(64, device=device, dtype=torch.float16))
        for p in self.parameters():
            p.requires_grad_(False)


def _tensors(seed=0):
    g = torch.Generator().manual_seed(seed)
    return {"model.layers.0.q_proj.weight": (torch.randn(64, 128, generator=g) * 0.02).half(),
            "model.layers.0.norm": torch.randn(64, generator=g).half()}


def _write(root, tensors, sharded):
    if not sharded:
        save_file(tensors, str(root / "model.safetensors"))
        return
    names = sorted(tensors)
    weight_map = {}
    for i, n in enumerate(names):
        shard = f"model-0000{i + 1}-of-0000{len(names)}.safetensors"
        save_file({n: tensors[n]}, str(root / shard))
        weight_map[n] = shard
    (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


def _stub_quantizer():
    calls = []

    def fake(A, blocksize=64, compress_statistics=False, quant_type="nf4", rounding="argmin", **_):
        calls.append((tuple(A.shape), A.dtype))
        n = A.numel()
        st = U.QuantState(absmax=torch.ones(-(-n // blocksize)), shape=A.shape, code=torch.zeros(16),
                          blocksize=blocksize, quant_type=quant_type, dtype=A.dtype)
        return torch.zeros((n + 1) // 2, 1, dtype=torch.uint8), st
    return calls, fake


@pytest.mark.parametrize("sharded", [False, True])
def test_stream_load_and_quantize_then_cache_hit(tmp_path, sharded):
    t = _tensors()
    ck = tmp_path / "ckpt"
    ck.mkdir()
    _write(ck, t, sharded)
    cache = tmp_path / "cache"
    calls, fake = _stub_quantizer()
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        m = Tiny()
        stats = stream_load_and_quantize_module(m, str(ck), min_numel=4096, cache_dir=cache)
        assert stats is not None and stats.tensors == 1 and stats.cache_writes == 1 and stats.cache_misses == 1
        q = m.model.layers[0].q_proj.weight
        assert hasattr(q, U.NF4_ATTR) and q.numel() == 0 and calls == [((64, 128), torch.float16)]
        assert torch.equal(m.model.layers[0].norm, t["model.layers.0.norm"])  # small: loaded, kept
        m2 = Tiny()  # second build: the payload comes from the cache, the quantizer is not called
        stats2 = stream_load_and_quantize_module(m2, str(ck), min_numel=4096, cache_dir=cache)
        assert stats2.cache_hits == 1 and stats2.tensors == 1 and len(calls) == 1
        # everything staged already: counted, nothing read
        assert stream_load_and_quantize_module(m2, str(ck), min_numel=4096, cache_dir=cache).tensors == 1


def test_single_file_path_and_key_function(tmp_path):
    t = {"q.weight": _tensors()["model.layers.0.q_proj.weight"], "n": _tensors()["model.layers.0.norm"]}
    save_file(t, str(tmp_path / "w.safetensors"))
    calls, fake = _stub_quantizer()
    keys = {"model.layers.0.q_proj.weight": ["q.weight"], "model.layers.0.norm": ["n"]}
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        m = Tiny()
        stats = stream_load_and_quantize_module(m, str(tmp_path / "w.safetensors"), key_fn=lambda n: keys[n])
    assert stats.tensors == 1 and calls == [((64, 128), torch.float16)]
    assert torch.equal(m.model.layers[0].norm, t["n"])


def test_missing_key_or_checkpoint_returns_none(tmp_path):
    t = _tensors()
    del t["model.layers.0.q_proj.weight"]
    _write(tmp_path, t, False)
    calls, fake = _stub_quantizer()
    with mock.patch.object(U, "quantize_4bit", fake):
        assert stream_load_and_quantize_module(Tiny(), str(tmp_path)) is None
        assert stream_load_and_quantize_module(Tiny(), str(tmp_path / "absent")) is None
    assert calls == []


def test_shape_mismatch_is_an_error(tmp_path):
    t = _tensors()
    t["model.layers.0.q_proj.weight"] = t["model.layers.0.q_proj.weight"][:32].contiguous()
    _write(tmp_path, t, False)
    calls, fake = _stub_quantizer()
    with mock.patch.object(U, "quantize_4bit", fake), pytest.raises(ValueError, match="shape"):
        stream_load_and_quantize_module(Tiny(), str(tmp_path))
