"""CPU tests of the checkpoint loaders (stratum/upload.py:425-904,1325-1440) on
small safetensors checkpoints written to a temporary directory (single file and
sharded with an index), with the GPU quantizer replaced by a recording stub
as in the lifecycle tests. The reference's own test of the key mapping is
tests/test_mlp_opt.py:156-166 (wrapper names canonicalised)."""

import json
from unittest import mock

import pytest
import torch
import torch.nn as nn
from safetensors.torch import save_file

import stratum_amd.upload as U
from stratum_amd.checkpoint import (_build_ckpt_key_fn, _try_load_fused_experts, load_module_fp16_from_checkpoint,
                                    populate_from_hf_checkpoint, stream_load_and_quantize_module)


class Wrapped(nn.Module):
    """A transparent wrapper (like TokenChunkedModule) adding '.module.' to names."""

    def __init__(self, module):
        super().__init__()
        self.module = module


class LayerWithIdx(nn.Module):
    """Stratum's decoder-layer wrapper: '.layer.' plus a global index."""

    def __init__(self, idx, layer):
        super().__init__()
        self.idx = idx
        self.layer = layer


def test_wrapper_names_are_canonicalized_for_checkpoint_lookup():
    ff = nn.Module()
    ff.w1 = nn.Linear(3, 3, bias=False)
    model = nn.Module()
    model.model = nn.Module()
    model.model.layers = nn.ModuleList([nn.Module()])
    model.model.layers[0].feed_forward = Wrapped(ff)
    keys = _build_ckpt_key_fn(model)("model.layers.0.feed_forward.module.w1.weight")
    assert "model.layers.0.feed_forward.w1.weight" in keys
    assert "model.layers.0.feed_forward.module.w1.weight" not in keys


def test_key_variants_for_layer_wrappers_peft_and_tied_head():
    inner = nn.Module()
    inner.self_attn = nn.Module()
    inner.self_attn.q_proj = nn.Linear(2, 2, bias=False)
    stage = nn.Module()
    stage.layers = nn.ModuleList([LayerWithIdx(7, inner)])
    fn = _build_ckpt_key_fn(stage)
    keys = fn("layers.0.layer.self_attn.q_proj.base_layer.weight")
    assert keys[0] == "layers.0.layer.self_attn.q_proj.base_layer.weight"
    assert "model.layers.7.self_attn.q_proj.weight" in keys          # global index
    assert "layers.0.self_attn.q_proj.weight" in keys                # '.layer.' and PEFT stripped
    assert "model.lm_head.weight" in fn("lm_head.weight") and "model.embed_tokens.weight" in fn("lm_head.weight")
    assert "a.b.weight" in fn("a.inner.b.weight")
    assert len(keys) == len(set(keys))


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


def _write(tmp_path, tensors, sharded):
    if not sharded:
        save_file(tensors, str(tmp_path / "model.safetensors"))
        return
    names = sorted(tensors)
    wm = {}
    for i, n in enumerate(names):
        shard = f"model-0000{i + 1}-of-0000{len(names)}.safetensors"
        save_file({n: tensors[n]}, str(tmp_path / shard))
        wm[n] = shard
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))


@pytest.mark.parametrize("sharded", [False, True])
def test_load_module_fp16_from_checkpoint(tmp_path, sharded):
    t = _tensors()
    _write(tmp_path, t, sharded)
    m = Tiny()
    assert load_module_fp16_from_checkpoint(m, str(tmp_path))
    assert torch.equal(m.model.layers[0].q_proj.weight, t["model.layers.0.q_proj.weight"])
    assert torch.equal(m.model.layers[0].norm, t["model.layers.0.norm"])
    assert load_module_fp16_from_checkpoint(m, str(tmp_path))  # nothing left on meta


@pytest.mark.parametrize("sharded", [False, True])
def test_load_fails_on_missing_key_or_checkpoint(tmp_path, sharded):
    t = _tensors()
    del t["model.layers.0.norm"]
    _write(tmp_path, t, sharded)
    assert not load_module_fp16_from_checkpoint(Tiny(), str(tmp_path))
    assert not load_module_fp16_from_checkpoint(Tiny(), str(tmp_path / "absent"))


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
        assert stream_load_and_quantize_module(m2, str(ck), min_numel=4096, cache_dir=cache).tensors == 1


def test_stream_load_missing_key_returns_none(tmp_path):
    t = _tensors()
    del t["model.layers.0.q_proj.weight"]
    _write(tmp_path, t, False)
    calls, fake = _stub_quantizer()
    with mock.patch.object(U, "quantize_4bit", fake):
        assert stream_load_and_quantize_module(Tiny(), str(tmp_path)) is None


def test_fused_experts_are_stacked_from_per_expert_keys():
    E, I, H = 3, 4, 6
    per = {}
    for e in range(E):
        per[f"model.layers.0.feed_forward.experts.{e}.w1.weight"] = torch.full((I, H), 10.0 * e + 1)
        per[f"model.layers.0.feed_forward.experts.{e}.w3.weight"] = torch.full((I, H), 10.0 * e + 3)
        per[f"model.layers.0.feed_forward.experts.{e}.w2.weight"] = torch.full((H, I), 10.0 * e + 2)

    class H_:
        def get_tensor(self, k):
            return per[k]

    keys_of = _build_ckpt_key_fn(nn.Module())
    gu = nn.Parameter(torch.empty(E, 2 * I, H, device="meta"), requires_grad=False)
    dn = nn.Parameter(torch.empty(E, H, I, device="meta"), requires_grad=False)
    got = _try_load_fused_experts(H_(), set(per), "model.layers.0.feed_forward.experts.gate_up_proj", gu, keys_of)
    assert got.shape == (E, 2 * I, H) and got[2, 0, 0] == 21 and got[2, I, 0] == 23
    got = _try_load_fused_experts(H_(), set(per), "model.layers.0.feed_forward.experts.down_proj", dn, keys_of)
    assert got.shape == (E, H, I) and got[1, 0, 0] == 12
    assert _try_load_fused_experts(H_(), set(), "model.layers.0.feed_forward.experts.down_proj", dn, keys_of) is None
    assert _try_load_fused_experts(H_(), set(per), "model.layers.0.mlp.down_proj", dn, keys_of) is None


def test_populate_from_checkpoint_and_cache(tmp_path):
    t = _tensors()
    ck = tmp_path / "ckpt"
    ck.mkdir()
    t_ckpt = {"model.layers.0.norm": t["model.layers.0.norm"]}  # populate reads small params by their own name
    _write(ck, t_ckpt, False)
    cache = tmp_path / "cache"
    calls, fake = _stub_quantizer()
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        src = Tiny(device="cpu")
        src.model.layers[0].q_proj.weight.data.copy_(t["model.layers.0.q_proj.weight"])
        U.prepare_nf4(src, cache_dir=cache, verbose=False)
        m = Tiny()
        # parameter names inside Tiny are model.layers.0.*; the checkpoint holds the norm under that name
        ok = populate_from_hf_checkpoint(m, str(ck), cache, verbose=False)
        assert ok
        assert hasattr(m.model.layers[0].q_proj.weight, U.NF4_ATTR)
        assert torch.equal(m.model.layers[0].norm, t["model.layers.0.norm"])
        assert not populate_from_hf_checkpoint(Tiny(), str(ck), tmp_path / "empty-cache", verbose=False)
