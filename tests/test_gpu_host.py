"""GPU tests of the host layer: the NF4 staging lifecycle (prepare_nf4 ->
ensure_weights -> free_weights, prefetch, cache) and NF4Linear / NF4LoRALinear
autograd, checked against the oracle (bit-exact weights) and fp32 references."""

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_weight(w, dtype, device):
    """Oracle dequantization of an fp16 weight to *dtype*, as a float32 tensor."""
    p, a = C.quantize(bits16(w), O.DT_F16, 64, "argmin")
    tag = O.DT_F16 if dtype == torch.float16 else O.DT_BF16
    bits = C.dequantize(p, a, w.numel(), 64, tag).view(np.int16).reshape(w.shape)
    return torch.from_numpy(bits).view(dtype).float().to(device)


def oracle_dequant_bits(w, bs=64):
    x = bits16(w)
    p, a = C.quantize(x, O.DT_F16 if w.dtype == torch.float16 else O.DT_BF16, bs, "argmin")
    return C.dequantize(p, a, w.numel(), bs, O.DT_F16 if w.dtype == torch.float16 else O.DT_BF16)


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(256, 512, bias=False, dtype=torch.float16)
        self.experts = nn.Parameter(seeded((4, 128, 64), 3, 0.02, torch.float16), requires_grad=False)
        self.norm = nn.LayerNorm(256, dtype=torch.float16).requires_grad_(False)
        self.register_buffer("running", torch.zeros(8))
        with torch.no_grad():
            self.q_proj.weight.copy_(seeded((512, 256), 1, 0.02, torch.float16))
        self.q_proj.weight.requires_grad_(False)


def test_prepare_ensure_free_lifecycle_is_bit_exact(cuda):
    from stratum_amd.upload import NF4_ATTR, ensure_weights, free_weights, prepare_nf4
    m = _Block()
    w_q = m.q_proj.weight.detach().clone()
    w_e = m.experts.detach().clone()
    stats = prepare_nf4(m, min_numel=4096, verbose=False)
    assert stats.tensors == 2
    assert m.q_proj.weight.numel() == 0 and m.experts.numel() == 0
    pay = getattr(m.experts, NF4_ATTR)
    assert pay.shape == (4, 128, 64) and pay.quantized.is_pinned() and pay.quantized.shape == (4 * 128 * 64 // 2, 1)
    n = ensure_weights(m, 0)
    assert n >= 2
    assert m.q_proj.weight.device.type == "cuda" and m.q_proj.weight.dtype == torch.float16
    np.testing.assert_array_equal(bits16(m.q_proj.weight).ravel(), oracle_dequant_bits(w_q))
    np.testing.assert_array_equal(bits16(m.experts).ravel(), oracle_dequant_bits(w_e.reshape(-1, 64)))
    assert m.experts.shape == (4, 128, 64)
    assert m.running.device.type == "cuda" and m.norm.weight.device.type == "cuda"
    assert ensure_weights(m, 0) == 0  # everything already materialised
    assert free_weights(m) == 2
    assert m.q_proj.weight.numel() == 0
    assert ensure_weights(m, 0) == 2  # second step re-materialises from the payload
    np.testing.assert_array_equal(bits16(m.q_proj.weight).ravel(), oracle_dequant_bits(w_q))


def test_side_stream_upload_with_fence(cuda):
    """DeviceStage pattern: ensure_weights on a param stream, event, default stream waits."""
    from stratum_amd.upload import ensure_weights, free_weights, prepare_nf4
    layers = [nn.Linear(512, 512, bias=False, dtype=torch.float16) for _ in range(3)]
    ref = []
    for i, l in enumerate(layers):
        with torch.no_grad():
            l.weight.copy_(seeded((512, 512), 10 + i, 0.02, torch.float16))
        l.weight.requires_grad_(False)
        ref.append(oracle_dequant_bits(l.weight.detach().clone()))
        prepare_nf4(l, verbose=False)
    x = seeded((64, 512), 99, 1.0, torch.float16).to(cuda)
    param_stream = torch.cuda.Stream()
    default = torch.cuda.default_stream()
    outs = []
    for step in range(2):
        fences = []
        for l in layers:
            with torch.cuda.stream(param_stream):
                ensure_weights(l, 0)
            ev = torch.cuda.Event()
            ev.record(param_stream)
            fences.append(ev)
        h = x
        for l, ev in zip(layers, fences):
            default.wait_event(ev)
            h = l(h)
        outs.append(h.float().cpu())
        for i, l in enumerate(layers):
            np.testing.assert_array_equal(bits16(l.weight).ravel(), ref[i])
            free_weights(l)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_prefetch_then_finalize(cuda):
    from stratum_amd.upload import ensure_prefetched_weights, free_weights, prefetch_weights, prepare_nf4
    m = _Block()
    w_q = m.q_proj.weight.detach().clone()
    prepare_nf4(m, verbose=False)
    pf = prefetch_weights(m, 0)
    assert len(pf.entries) == 2 and pf.event is not None
    assert m.q_proj.weight.numel() == 0  # parameter data untouched until finalize
    n = ensure_prefetched_weights(m, 0, pf)
    assert n >= 2
    np.testing.assert_array_equal(bits16(m.q_proj.weight).ravel(), oracle_dequant_bits(w_q))
    with pytest.raises(ValueError):
        ensure_prefetched_weights(m, 1, pf)
    free_weights(m)
    assert prefetch_weights(nn.Linear(4, 4), 0).entries == []


def test_cache_roundtrip_and_from_cache(cuda, tmp_path):
    from stratum_amd.upload import NF4_ATTR, ensure_weights, prepare_nf4, prepare_nf4_from_cache
    m1 = _Block()
    w_q = m1.q_proj.weight.detach().clone()
    s1 = prepare_nf4(m1, cache_dir=tmp_path, verbose=False)
    assert s1.cache_misses == 2 and s1.cache_writes == 2
    m2 = _Block()
    s2 = prepare_nf4(m2, cache_dir=tmp_path, verbose=False)
    assert s2.cache_hits == 2 and s2.cache_writes == 0
    p1, p2 = getattr(m1.q_proj.weight, NF4_ATTR), getattr(m2.q_proj.weight, NF4_ATTR)
    assert torch.equal(p1.quantized, p2.quantized) and torch.equal(p1.absmax, p2.absmax)
    m3 = _Block()
    # weights never materialised on the host: meta parameters, as in a meta-device build
    m3.q_proj.weight = nn.Parameter(torch.empty(512, 256, dtype=torch.float16, device="meta"), requires_grad=False)
    m3.experts = nn.Parameter(torch.empty(4, 128, 64, dtype=torch.float16, device="meta"), requires_grad=False)
    s3 = prepare_nf4_from_cache(m3, tmp_path, verbose=False)
    assert s3 is not None and s3.tensors == 2 and s3.cache_hits == 2
    assert m3.q_proj.weight.device.type == "cpu" and m3.q_proj.weight.numel() == 0
    ensure_weights(m3, 0)
    np.testing.assert_array_equal(bits16(m3.q_proj.weight).ravel(), oracle_dequant_bits(w_q))


# NF4Linear picks the fused kernels up to STRATUM_NF4_FUSED_MAX_ROWS rows and
# dequantize + library GEMM above; both paths are checked at the same sizes.
PATHS = {"fused": "-1", "library": "0"}


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_nf4_linear_forward_backward(cuda, dtype, path, monkeypatch):
    from stratum_amd.functional import quantize_4bit
    from stratum_amd.nf4_linear import NF4Linear
    monkeypatch.setenv("STRATUM_NF4_FUSED_MAX_ROWS", PATHS[path])
    N, K, M = 384, 256, 200
    w = seeded((N, K), 5, 0.02, torch.float16)
    q, st = quantize_4bit(w.to(cuda))
    st.dtype = dtype
    bias = seeded((N,), 6, 0.1, dtype).to(cuda)
    lin = NF4Linear(q, st, bias=bias)
    assert lin.in_features == K and lin.out_features == N
    wq = oracle_weight(w, dtype, cuda)
    x = seeded((4, M // 4, K), 7, 1.0, dtype).to(cuda).requires_grad_(True)
    y = lin(x)
    xr = x.detach().float().requires_grad_(True)
    yr = xr @ wq.t().contiguous() + bias.float()
    tol = 1e-2 if dtype == torch.bfloat16 else 5e-3
    assert ((y.float() - yr).norm() / yr.norm()).item() <= tol
    g = seeded(tuple(y.shape), 8, 1.0, dtype).to(cuda)
    y.backward(g)
    yr.backward(g.float())
    assert ((x.grad.float() - xr.grad).norm() / xr.grad.norm()).item() <= tol


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("r,dtype", [(16, torch.bfloat16), (32, torch.float16), (8, torch.bfloat16),
                                     (48, torch.bfloat16)])
def test_nf4_lora_linear_gradients(cuda, path, monkeypatch, r, dtype):
    """Rank 16 and 32 take the fused kernels' LoRA epilogues and the LoRA side
    kernels; rank 8 takes the unfused module path; rank 48 the torch side products."""
    from stratum_amd.functional import quantize_4bit
    from stratum_amd.nf4_linear import NF4LoRALinear
    monkeypatch.setenv("STRATUM_NF4_FUSED_MAX_ROWS", PATHS[path])
    N, K, M = 512, 256, 160
    w = seeded((N, K), 15, 0.02, torch.float16)
    q, st = quantize_4bit(w.to(cuda))
    st.dtype = dtype
    lin = NF4LoRALinear(q, st, r=r, lora_alpha=32.0, dtype=dtype)
    with torch.no_grad():
        lin.lora_A.copy_(seeded((r, K), 16, 0.05, dtype))
        lin.lora_B.copy_(seeded((N, r), 17, 0.05, dtype))
    wq = oracle_weight(w, dtype, cuda)
    x = seeded((M, K), 18, 1.0, dtype).to(cuda).requires_grad_(True)
    y = lin(x)
    g = seeded((M, N), 19, 1.0, dtype).to(cuda)
    y.backward(g)
    A = lin.lora_A.detach().float().requires_grad_(True)
    B = lin.lora_B.detach().float().requires_grad_(True)
    xr = x.detach().float().requires_grad_(True)
    yr = xr @ wq.t().contiguous() + (xr @ A.t().contiguous()) @ B.t().contiguous() * lin.scaling
    yr.backward(g.float())

    def rel(a_, b_):
        return ((a_.float() - b_).norm() / b_.norm()).item()

    tol = 1e-2 if dtype == torch.bfloat16 else 5e-3
    assert rel(y, yr) <= tol
    assert rel(x.grad, xr.grad) <= tol
    assert rel(lin.lora_A.grad, A.grad) <= 2 * tol
    assert rel(lin.lora_B.grad, B.grad) <= 2 * tol


def test_layer_stream_materialises_each_layer_then_frees_it(cuda):
    from stratum_amd.stream import NF4LayerStream
    from stratum_amd.upload import prepare_nf4
    layers, refs = [], []
    for i in range(4):
        l = nn.Linear(256, 384, bias=False, dtype=torch.float16)
        with torch.no_grad():
            l.weight.copy_(seeded((384, 256), 40 + i, 0.02, torch.float16))
        l.weight.requires_grad_(False)
        refs.append(oracle_dequant_bits(l.weight.detach().clone()))
        prepare_nf4(l, verbose=False)
        layers.append(l)
    x = seeded((32, 256), 50, 1.0, torch.float16).to(cuda)
    seen = []
    for i, layer in NF4LayerStream(layers, 0, lookahead=2):
        np.testing.assert_array_equal(bits16(layer.weight).ravel(), refs[i])
        y = layer(x)
        seen.append(i)
    torch.cuda.synchronize()
    assert seen == [0, 1, 2, 3]
    assert all(l.weight.numel() == 0 for l in layers)
    assert torch.isfinite(y.float()).all()
    # a second pass re-materialises from the pinned payloads
    for i, layer in NF4LayerStream(layers, 0, free_after=False):
        np.testing.assert_array_equal(bits16(layer.weight).ravel(), refs[i])
    assert all(l.weight.numel() == 384 * 256 for l in layers)


def test_nf4_linear_default_policy_by_rows(cuda, monkeypatch):
    """Default threshold: 768 rows fused, 769 rows through the library GEMM (with
    a LoRA adapter 1024 and 1025); every call agrees with the fp32 reference."""
    import importlib
    from stratum_amd.functional import quantize_4bit
    NL = importlib.import_module("stratum_amd.nf4_linear")  # the package exports a function of that name
    monkeypatch.delenv("STRATUM_NF4_FUSED_MAX_ROWS", raising=False)
    assert NL.fused_max_rows() == 768
    N, K = 256, 128
    w = seeded((N, K), 21, 0.02, torch.float16)
    q, st = quantize_4bit(w.to(cuda))
    st.dtype = torch.bfloat16
    wq = oracle_weight(w, torch.bfloat16, cuda)
    calls = []
    real = NL._NF4LinearFn.apply
    # argument 9 of _NF4LinearFn.apply is the fused flag
    monkeypatch.setattr(NL._NF4LinearFn, "apply", lambda *a: calls.append(a[9]) or real(*a))
    for M in (768, 769):
        x = seeded((M, K), 22, 1.0, torch.bfloat16).to(cuda)
        y = NL.NF4Linear(q, st)(x)
        ref = x.float() @ wq.t().contiguous()
        assert ((y.float() - ref).norm() / ref.norm()).item() <= 1e-2
    assert calls == [True, False]

    # with a LoRA adapter the threshold is 1024 rows
    assert NL.fused_max_rows(lora=True) == 1024
    calls.clear()
    lin = NL.NF4LoRALinear(q, st, r=16, lora_alpha=16.0).to(cuda)
    with torch.no_grad():
        lin.lora_B.copy_(seeded((N, 16), 23, 0.01, torch.float32).to(cuda))
    a, b = lin.lora_A.detach().float(), lin.lora_B.detach().float()
    for M in (1024, 1025):
        x = seeded((M, K), 24, 1.0, torch.bfloat16).to(cuda)
        y = lin(x)
        xf = x.float()
        ref = xf @ wq.t().contiguous() + (xf @ a.t().contiguous()) @ b.t().contiguous() * lin.scaling
        assert ((y.float() - ref).norm() / ref.norm()).item() <= 1e-2
    assert calls == [True, False]


def test_stream_load_and_quantize_from_checkpoint_bit_exact(cuda, tmp_path):
    """Cold build straight from a safetensors checkpoint: every eligible weight is
    quantized by the GPU kernel; payload codes/absmax and the later ensure_weights
    dequantization are bit-exact against the oracle; the cache written on the way
    serves a second build."""
    from safetensors.torch import save_file
    from stratum_amd.upload import NF4_ATTR, ensure_weights, stream_load_and_quantize_module
    w = seeded((512, 256), 31, 0.02, torch.float16)
    norm = seeded((512,), 32, 1.0, torch.float16)
    save_file({"model.layers.0.proj.weight": w, "model.layers.0.norm": norm}, str(tmp_path / "model.safetensors"))

    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.model = nn.Module()
            self.model.layers = nn.ModuleList([nn.Module()])
            lay = self.model.layers[0]
            lay.proj = nn.Linear(256, 512, bias=False, device="meta", dtype=torch.float16)
            lay.norm = nn.Parameter(torch.empty(512, device="meta", dtype=torch.float16))
            for p in self.parameters():
                p.requires_grad_(False)

    m = M()
    stats = stream_load_and_quantize_module(m, str(tmp_path), cache_dir=tmp_path / "cache")
    assert stats is not None and stats.tensors == 1 and stats.cache_writes == 1
    pl = getattr(m.model.layers[0].proj.weight, NF4_ATTR)
    ref_p, ref_a = C.quantize(bits16(w), O.DT_F16, 64, "argmin")
    np.testing.assert_array_equal(pl.quantized.numpy().ravel(), ref_p)
    np.testing.assert_array_equal(pl.absmax.numpy().view(np.uint32), ref_a.view(np.uint32))
    assert pl.quantized.is_pinned()
    assert ensure_weights(m, 0) >= 1
    np.testing.assert_array_equal(bits16(m.model.layers[0].proj.weight).ravel(), oracle_dequant_bits(w))
    assert torch.equal(m.model.layers[0].norm.cpu(), norm)
    m2 = M()
    stats2 = stream_load_and_quantize_module(m2, str(tmp_path), cache_dir=tmp_path / "cache")
    assert stats2.cache_hits == 1
