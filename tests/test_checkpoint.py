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


# ---- checkpoint key mapping (stratum/upload.py:425-531): stage wrappers with a
# layer index, PEFT base_layer, .inner./.layer. segments, tied lm_head, fused
# expert banks, hub ids from the local cache


class _Wrapped(nn.Module):
    """A stage wrapper as the reference builds them: global layer index ``idx``
    around the decoder layer ``layer``."""

    def __init__(self, idx, inner):
        super().__init__()
        self.idx = idx
        self.layer = inner


class _Lora(nn.Module):
    """PEFT's wrapper: the frozen Linear under ``base_layer``."""

    def __init__(self, base):
        super().__init__()
        self.base_layer = base


class _Decoder(nn.Module):
    def __init__(self, experts=0):
        super().__init__()
        self.self_attn = nn.Module()
        self.self_attn.q_proj = _Lora(nn.Linear(128, 64, bias=False, device="meta", dtype=torch.float16))
        self.mlp = nn.Module()
        self.mlp.inner = nn.Module()
        self.mlp.inner.up_proj = nn.Linear(128, 64, bias=False, device="meta", dtype=torch.float16)
        if experts:
            self.feed_forward = nn.Module()
            self.feed_forward.experts = nn.Module()
            self.feed_forward.experts.gate_up_proj = nn.Parameter(
                torch.empty(experts, 2 * 32, 64, device="meta", dtype=torch.float16))
            self.feed_forward.experts.down_proj = nn.Parameter(
                torch.empty(experts, 64, 32, device="meta", dtype=torch.float16))


class _Stage(nn.Module):
    def __init__(self, first, n, experts=0):
        super().__init__()
        self.layers = nn.ModuleList([_Wrapped(first + i, _Decoder(experts)) for i in range(n)])
        for p in self.parameters():
            p.requires_grad_(False)


def _rand(shape, seed):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * 0.02).half()


def test_key_function_order_and_variants():
    keys = __import__("stratum_amd.checkpoint", fromlist=["x"]).checkpoint_key_fn(_Stage(7, 1))
    ks = keys("layers.0.layer.mlp.inner.up_proj.weight")
    assert ks[0] == "layers.0.layer.mlp.inner.up_proj.weight"           # the name itself first
    assert "model.layers.7.mlp.up_proj.weight" in ks                      # global index, .inner. dropped
    assert "model.layers.7.mlp.inner.up_proj.weight" in ks
    assert len(ks) == len(set(ks))
    q = keys("layers.0.layer.self_attn.q_proj.base_layer.weight")
    assert "model.layers.7.self_attn.q_proj.weight" in q and q.index("model.layers.7.self_attn.q_proj.weight") > 0
    assert keys("layers.0.module.layer.mlp.inner.up_proj.weight")[0] == "layers.0.layer.mlp.inner.up_proj.weight"
    # the plain spellings come before the model.-prefixed ones of the same name
    plain = keys("norm.weight")
    assert plain.index("norm.weight") < plain.index("model.norm.weight")
    tied = keys("lm_head.weight")
    assert tied[0] == "lm_head.weight" and "model.embed_tokens.weight" in tied and "embed_tokens.weight" in tied


@pytest.mark.parametrize("sharded", [False, True])
def test_stage_local_wrapped_layers_load_their_global_keys(tmp_path, sharded):
    ck = tmp_path / "ck"
    ck.mkdir()
    t = {}
    for g in (4, 5):
        t[f"model.layers.{g}.self_attn.q_proj.weight"] = _rand((64, 128), g)
        t[f"model.layers.{g}.mlp.up_proj.weight"] = _rand((64, 128), 10 + g)
    _write(ck, t, sharded)
    calls, fake = _stub_quantizer()
    stage = _Stage(4, 2)
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        stats = stream_load_and_quantize_module(stage, str(ck), min_numel=4096)
    assert stats is not None and stats.tensors == 4 and len(calls) == 4
    # small enough to stay dense: the values are the global layer's
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        stage2 = _Stage(4, 2)
        stats2 = stream_load_and_quantize_module(stage2, str(ck), min_numel=1 << 20)
    assert stats2 is not None and stats2.tensors == 0
    assert torch.equal(stage2.layers[1].layer.self_attn.q_proj.base_layer.weight, t["model.layers.5.self_attn.q_proj.weight"])
    assert torch.equal(stage2.layers[0].layer.mlp.inner.up_proj.weight, t["model.layers.4.mlp.up_proj.weight"])


def test_tied_lm_head_reads_the_embedding(tmp_path):
    class Postfix(nn.Module):
        def __init__(self):
            super().__init__()
            self.lm_head = nn.Linear(128, 256, bias=False, device="meta", dtype=torch.float16)
            self.lm_head.weight.requires_grad_(False)

    emb = _rand((256, 128), 3)
    save_file({"model.embed_tokens.weight": emb}, str(tmp_path / "model.safetensors"))
    calls, fake = _stub_quantizer()
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        m = Postfix()
        assert stream_load_and_quantize_module(m, str(tmp_path), min_numel=1 << 20).tensors == 0
    assert torch.equal(m.lm_head.weight, emb)


def test_fused_expert_banks_stack_per_expert_tensors(tmp_path):
    E = 3
    t = {f"model.layers.2.self_attn.q_proj.weight": _rand((64, 128), 1),
         f"model.layers.2.mlp.up_proj.weight": _rand((64, 128), 2)}
    for e in range(E):
        t[f"model.layers.2.feed_forward.experts.{e}.w1.weight"] = _rand((32, 64), 100 + e)
        t[f"model.layers.2.feed_forward.experts.{e}.w3.weight"] = _rand((32, 64), 200 + e)
        t[f"model.layers.2.feed_forward.experts.{e}.w2.weight"] = _rand((64, 32), 300 + e)
    _write(tmp_path, t, True)
    calls, fake = _stub_quantizer()
    stage = _Stage(2, 1, experts=E)
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        stats = stream_load_and_quantize_module(stage, str(tmp_path), min_numel=1 << 20)
    assert stats is not None
    ex = stage.layers[0].layer.feed_forward.experts
    want_gu = torch.stack([torch.cat([t[f"model.layers.2.feed_forward.experts.{e}.w1.weight"],
                                      t[f"model.layers.2.feed_forward.experts.{e}.w3.weight"]]) for e in range(E)])
    want_d = torch.stack([t[f"model.layers.2.feed_forward.experts.{e}.w2.weight"] for e in range(E)])
    assert torch.equal(ex.gate_up_proj, want_gu) and torch.equal(ex.down_proj, want_d)
    # a missing expert: no bank, no key -> None
    del t["model.layers.2.feed_forward.experts.1.w2.weight"]
    (tmp_path / "b").mkdir()
    _write(tmp_path / "b", t, False)
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        assert stream_load_and_quantize_module(_Stage(2, 1, experts=E), str(tmp_path / "b"), min_numel=1 << 20) is None


def test_hub_id_resolves_through_the_local_cache_only(tmp_path, monkeypatch):
    import huggingface_hub.constants as C
    snap = tmp_path / "hub" / "models--org--tiny" / "snapshots" / "abc123"
    snap.mkdir(parents=True)
    (tmp_path / "hub" / "models--org--tiny" / "refs").mkdir()
    (tmp_path / "hub" / "models--org--tiny" / "refs" / "main").write_text("abc123")
    _write(snap, _tensors(), False)
    monkeypatch.setattr(C, "HF_HUB_CACHE", str(tmp_path / "hub"))
    monkeypatch.setenv("HF_HUB_OFFLINE", "1")
    calls, fake = _stub_quantizer()
    with mock.patch.object(U, "quantize_4bit", fake), mock.patch.object(U, "_pin_cpu", lambda x: x):
        m = Tiny()
        stats = stream_load_and_quantize_module(m, "org/tiny", min_numel=4096)
        assert stats is not None and stats.tensors == 1
        assert stream_load_and_quantize_module(Tiny(), "org/absent", min_numel=4096) is None
