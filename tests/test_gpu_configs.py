"""GPU parity at the full sizes of the workloads the path is measured on.

* Qwen3-0.6B layer, M = 4096 tokens: all seven frozen projections, forward and
  input gradient.
* MoE expert bank (Qwen3-30B-A3B-like): 128 experts of gate_up [1536, 2048]
  and down [2048, 768], 8192 tokens routed top-8 from softmax(N(0, 1) logits),
  grouped forward and input gradient of both banks, every expert checked.
* 8B decoder layer stream-in: two full layers (q/o [4096, 4096], k/v
  [1024, 4096], gate/up [14336, 4096], down [4096, 14336]) staged to pinned
  host memory and streamed through NF4LayerStream with lookahead 1; every
  weight bit-exact against the oracle at its yield.

* Decode-sized rows (1, 16, 32) on the full W [14336, 4096]: the small-M
  forward and input gradient with their rank-16 LoRA terms.

GEMMs are held to the whole-matrix and the per-32x32-fragment bar
(tests/gpu_checks.py) against an fp32 matmul of the oracle-dequantized weight;
packed codes, absmax and dequantized weights are bit-exact.
"""

import numpy as np
import pytest
import torch

from gpu_checks import assert_gemm_close
from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu

TAG = {torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16}


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def f16_bits(w):
    return w.contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_weight(w16, dtype, bs=64):
    """Oracle codes, absmax and the dequantized weight in ``dtype`` (CPU tensor)."""
    rp, ra = C.quantize(f16_bits(w16.reshape(-1, w16.shape[-1])), O.DT_F16, bs, "argmin")
    deq = C.dequantize(rp, ra, w16.numel(), bs, TAG[dtype]).view(np.int16).reshape(tuple(w16.shape))
    return rp, ra, torch.from_numpy(deq).view(dtype)


# ------------------------------------------------------------ Qwen3-0.6B layer
QWEN06 = {  # name: (N, K) of W [out_features, in_features]
    "q_proj": (2048, 1024), "k_proj": (1024, 1024), "v_proj": (1024, 1024), "o_proj": (1024, 2048),
    "gate_proj": (3072, 1024), "up_proj": (3072, 1024), "down_proj": (1024, 3072),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", list(QWEN06))
def test_qwen06_projection_forward_and_input_gradient(cuda, name, dtype):
    from stratum_amd.functional import nf4_gemm_bwd_dx, nf4_gemm_fwd
    N, K = QWEN06[name]
    M = 4096
    seed = sum(map(ord, name))
    w = seeded((N, K), seed, 0.02, torch.float16)
    rp, ra, wq = oracle_weight(w, dtype)
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    wf = wq.to(cuda).float()
    x = seeded((M, K), seed + 1, 1.0, dtype).to(cuda)
    y = nf4_gemm_fwd(x, q, a, (N, K), 64)
    assert y.shape == (M, N) and y.dtype == dtype
    assert_gemm_close(y, x.float() @ wf.t().contiguous(), dtype, f"{name} forward")
    dy = seeded((M, N), seed + 2, 1.0, dtype).to(cuda)
    dx = nf4_gemm_bwd_dx(dy, q, a, (N, K), 64)
    assert dx.shape == (M, K) and dx.dtype == dtype
    assert_gemm_close(dx, dy.float() @ wf, dtype, f"{name} input gradient")


@pytest.mark.parametrize("group", [("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj")])
def test_qwen06_stacked_projections_match_each_projection(cuda, group):
    """q|k|v and gate|up stacked into one NF4 weight (stack_nf4): one fused
    forward at M = 4096 whose column slices are each projection's output, within
    the tolerance of the fp32 reference (and per 32 x 32 fragment)."""
    from stratum_amd.functional import QuantState, nf4_gemm_fwd, stack_nf4
    dtype = torch.bfloat16
    M = 4096
    K = QWEN06[group[0]][1]
    items, refs = [], []
    for name in group:
        N = QWEN06[name][0]
        seed = sum(map(ord, name))
        rp, ra, wq = oracle_weight(seeded((N, K), seed, 0.02, torch.float16), dtype)
        items.append((torch.from_numpy(rp).reshape(-1, 1).to(cuda),
                      QuantState(absmax=torch.from_numpy(ra).to(cuda), shape=(N, K), blocksize=64, dtype=dtype)))
        refs.append(wq.to(cuda).float())
    p, st = stack_nf4(items)
    x = seeded((M, K), 99, 1.0, dtype).to(cuda)
    y = nf4_gemm_fwd(x, p, st.absmax, tuple(st.shape), 64)
    col = 0
    for name, wf in zip(group, refs):
        n = wf.shape[0]
        assert_gemm_close(y[:, col:col + n].contiguous(), x.float() @ wf.t().contiguous(), dtype, f"stacked {name}")
        col += n
    assert col == y.shape[1]


# ------------------------------------------------------------ MoE expert bank
def route_top8(tokens, experts, seed):
    """softmax(N(0, 1) logits) -> top-8 experts per token (transformers Qwen3-MoE
    routing); returns the (token, slot) pairs grouped by expert and the int32
    row offsets of each expert's group."""
    logits = seeded((tokens, experts), seed, 1.0, torch.float32)
    probs = torch.softmax(logits, dim=-1)
    top = probs.topk(8, dim=-1).indices                     # [tokens, 8]
    flat = top.reshape(-1)
    order = torch.argsort(flat, stable=True)
    token_of_row = order // 8
    counts = torch.bincount(flat, minlength=experts)
    offsets = torch.zeros(experts + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(counts, 0).to(torch.int32)
    return token_of_row, offsets


def test_moe_bank_full_size_grouped_forward_and_input_gradient(cuda):
    from stratum_amd.functional import nf4_grouped_gemm, quantize_4bit, swiglu_fwd
    dtype = torch.bfloat16
    E, H, I, T = 128, 2048, 768, 8192
    token_of_row, off = route_top8(T, E, 4)
    rows = int(off[-1])
    assert rows == 8 * T
    counts = (off[1:] - off[:-1]).tolist()
    print(f"moe: {E} experts, rows per expert {min(counts)}..{max(counts)}", flush=True)

    w_gu = seeded((E, 2 * I, H), 40, 0.02, torch.float16)
    w_dn = seeded((E, H, I), 41, 0.02, torch.float16)
    gu_p, gu_a, gu_q = oracle_weight(w_gu, dtype)
    dn_p, dn_a, dn_q = oracle_weight(w_dn, dtype)
    # the GPU quantizer produces the same bytes at this size (the stacked bank
    # flattened to [E * N, K], as prepare_nf4 stores 3-D expert weights)
    p_dev, s_dev = quantize_4bit(w_gu.reshape(-1, H).to(cuda))
    assert torch.equal(p_dev.view(-1).cpu(), torch.from_numpy(gu_p)), "gate_up codes differ from the oracle"
    assert torch.equal(s_dev.absmax.cpu().view(torch.int32), torch.from_numpy(gu_a).view(torch.int32))
    del p_dev, s_dev
    gu_p, gu_a = torch.from_numpy(gu_p).to(cuda), torch.from_numpy(gu_a).to(cuda)
    dn_p, dn_a = torch.from_numpy(dn_p).to(cuda), torch.from_numpy(dn_a).to(cuda)
    gu_q, dn_q = gu_q.to(cuda), dn_q.to(cuda)
    offd = off.to(cuda)

    x = seeded((T, H), 42, 1.0, dtype).to(cuda)[token_of_row.to(cuda)].contiguous()   # rows grouped by expert
    g = nf4_grouped_gemm(x, gu_p, gu_a, offd, (2 * I, H), 64)
    h = swiglu_fwd(g)
    y = nf4_grouped_gemm(h, dn_p, dn_a, offd, (H, I), 64)
    d_g = seeded((rows, 2 * I), 43, 1.0, dtype).to(cuda)
    d_h = seeded((rows, H), 44, 1.0, dtype).to(cuda)
    dx = nf4_grouped_gemm(d_g, gu_p, gu_a, offd, (2 * I, H), 64, backward=True)
    dh = nf4_grouped_gemm(d_h, dn_p, dn_a, offd, (H, I), 64, backward=True)
    assert g.shape == (rows, 2 * I) and y.shape == (rows, H) and dx.shape == (rows, H) and dh.shape == (rows, I)
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi == lo:
            continue
        wgu, wdn = gu_q[e].float(), dn_q[e].float()
        assert_gemm_close(g[lo:hi], x[lo:hi].float() @ wgu.t().contiguous(), dtype, f"expert {e} gate_up")
        assert_gemm_close(y[lo:hi], h[lo:hi].float() @ wdn.t().contiguous(), dtype, f"expert {e} down")
        assert_gemm_close(dx[lo:hi], d_g[lo:hi].float() @ wgu, dtype, f"expert {e} gate_up input gradient")
        assert_gemm_close(dh[lo:hi], d_h[lo:hi].float() @ wdn, dtype, f"expert {e} down input gradient")


# ------------------------------------------------------------ 8B layer stream-in
LAYER_8B = {  # name: (out_features, in_features)
    "q_proj": (4096, 4096), "k_proj": (1024, 4096), "v_proj": (1024, 4096), "o_proj": (4096, 4096),
    "gate_proj": (14336, 4096), "up_proj": (14336, 4096), "down_proj": (4096, 14336),
}


class _Layer8B(torch.nn.Module):
    def __init__(self, seed):
        super().__init__()
        for i, (name, (n, k)) in enumerate(LAYER_8B.items()):
            lin = torch.nn.Linear(k, n, bias=False, dtype=torch.float16)
            lin.weight.requires_grad_(False)
            lin.weight.data.copy_(seeded((n, k), seed + i, 0.02, torch.float16))
            setattr(self, name, lin)


def test_8b_layers_stream_in_bit_exact_at_every_yield(cuda):
    from stratum_amd.stream import NF4LayerStream
    from stratum_amd.upload import NF4_ATTR, prepare_nf4
    layers = [_Layer8B(1000 * (i + 1)) for i in range(2)]
    expect = []
    for layer in layers:
        per = {}
        for name in LAYER_8B:
            w = getattr(layer, name).weight.data
            rp, ra, wq = oracle_weight(w, torch.float16)
            per[name] = (rp, ra, wq)
        expect.append(per)
    for layer in layers:
        prepare_nf4(layer, verbose=False)
    for layer, per in zip(layers, expect):  # payloads: pinned host memory, oracle bytes
        for name, (rp, ra, _) in per.items():
            pl = getattr(getattr(layer, name).weight, NF4_ATTR)
            assert pl.quantized.is_pinned() and pl.absmax.is_pinned()
            assert np.array_equal(pl.quantized.numpy().ravel(), rp), name
            assert np.array_equal(pl.absmax.numpy().view(np.uint32), ra.view(np.uint32)), name
    x = seeded((64, 4096), 7, 1.0, torch.float16).to(cuda)
    seen = []
    for i, layer in NF4LayerStream(layers, device_id=0, lookahead=1):
        for name, (_, _, wq) in expect[i].items():
            wt = getattr(layer, name).weight
            assert wt.data.is_cuda and wt.data.dtype == torch.float16 and tuple(wt.data.shape) == LAYER_8B[name]
            assert torch.equal(wt.data.view(torch.int16), wq.to(cuda).view(torch.int16)), f"layer {i} {name}"
        # compute on the consumer stream while the next layer streams in
        y = torch.nn.functional.linear(x, layer.q_proj.weight)
        torch.cuda.synchronize()
        ref = x.float() @ expect[i]["q_proj"][2].to(cuda).float().t()
        assert_gemm_close(y, ref, torch.float16, f"layer {i} q_proj use")
        seen.append(i)
        print(f"layer {i}: 7 weights bit-exact", flush=True)
    assert seen == [0, 1]
    for layer in layers:  # freed after each yield, payload kept
        for name in LAYER_8B:
            wt = getattr(layer, name).weight
            assert wt.data.numel() == 0 and hasattr(wt, NF4_ATTR)


# ----------------------------------------- LoRA step, W [14336, 4096], M = 8192
LORA_STEP = (8192, 14336, 4096, 16)  # M, N, K, rank (r = 16, alpha = 16: scaling 1)


@pytest.fixture(scope="module")
def lora_step(cuda):
    """The LoRA-step workload: W [14336, 4096] N(0, 0.02) fp16 -> NF4, X bf16
    [8192, 4096] N(0, 1), dY bf16 N(0, 1); oracle codes and bf16 weight."""
    M, N, K, R = LORA_STEP
    rp, ra, wq = oracle_weight(seeded((N, K), 55, 0.02, torch.float16), torch.bfloat16)
    return dict(q=torch.from_numpy(rp).to(cuda), a=torch.from_numpy(ra).to(cuda), w=wq.to(cuda).float(),
                x=seeded((M, K), 1, 1.0, torch.bfloat16).to(cuda), dy=seeded((M, N), 2, 1.0, torch.bfloat16).to(cuda))


@pytest.mark.parametrize("lora_std", [0.01, 0.1])
def test_lora_step_fused_kernels_with_lora_terms(cuda, lora_step, lora_std):
    """Forward with the rank-16 epilogue (T . B^T) and input gradient with the
    U . A term, at the full LoRA-step size, whole matrix and every 32 x 32
    fragment against fp32 on the oracle weight. A, B ~ N(0, 0.01) is the
    workload's init; at 0.1 the LoRA term is as large as the base product, so
    a wrong or dropped epilogue fails the bar everywhere."""
    from stratum_amd.functional import lora_down, lora_dy, nf4_gemm_bwd_dx, nf4_gemm_fwd
    M, N, K, R = LORA_STEP
    s = lora_step
    A = seeded((R, K), 10, lora_std, torch.bfloat16).to(cuda)
    B = seeded((N, R), 11, lora_std, torch.bfloat16).to(cuda)
    t = lora_down(s["x"], A, 1.0)
    y = nf4_gemm_fwd(s["x"], s["q"], s["a"], (N, K), 64, lora_t=t, lora_b=B)
    ref = s["x"].float() @ s["w"].t().contiguous() + t.float() @ B.float().t().contiguous()
    assert_gemm_close(y, ref, torch.bfloat16, "forward with LoRA epilogue")
    del y, ref
    u, _ = lora_dy(s["dy"], B, None, 1.0)
    dx = nf4_gemm_bwd_dx(s["dy"], s["q"], s["a"], (N, K), 64, lora_u=u, lora_at=A.t().contiguous())
    ref = s["dy"].float() @ s["w"] + u.float() @ A.float()
    assert_gemm_close(dx, ref, torch.bfloat16, "input gradient with U . A")


def test_lora_step_forced_fused_module_step(cuda, lora_step, monkeypatch):
    """The step bench.py times: NF4LoRALinear forward and backward with the fused
    kernels forced at 8192 rows -- y, dX, dA and dB against fp32 autograd on the
    oracle weight (whole matrix and per fragment)."""
    from stratum_amd.functional import QuantState
    from stratum_amd.nf4_linear import NF4LoRALinear
    monkeypatch.setenv("STRATUM_NF4_FUSED_MAX_ROWS", "-1")
    M, N, K, R = LORA_STEP
    s = lora_step
    st = QuantState(absmax=s["a"], shape=(N, K), blocksize=64, dtype=torch.bfloat16)
    lin = NF4LoRALinear(s["q"], st, r=R, lora_alpha=16.0)
    with torch.no_grad():
        lin.lora_A.copy_(seeded((R, K), 10, 0.1, torch.bfloat16))
        lin.lora_B.copy_(seeded((N, R), 11, 0.1, torch.bfloat16))
    x = s["x"].clone().requires_grad_(True)
    y = lin(x)
    y.backward(s["dy"])
    torch.cuda.synchronize()
    xr = s["x"].float().requires_grad_(True)
    Ar = lin.lora_A.detach().float().requires_grad_(True)
    Br = lin.lora_B.detach().float().requires_grad_(True)
    yr = xr @ s["w"].t().contiguous() + (xr @ Ar.t().contiguous()) @ Br.t().contiguous()
    yr.backward(s["dy"].float())
    assert_gemm_close(y.detach(), yr.detach(), torch.bfloat16, "module forward")
    del y, yr
    assert_gemm_close(x.grad, xr.grad, torch.bfloat16, "module dX")
    assert_gemm_close(lin.lora_A.grad, Ar.grad, torch.bfloat16, "dA")
    assert_gemm_close(lin.lora_B.grad, Br.grad, torch.bfloat16, "dB")


@pytest.mark.parametrize("M", [1, 16, 32, 64])
def test_decode_size_forward_and_input_gradient_at_full_weight_size(cuda, lora_step, M):
    """Decode-sized rows on the full W [14336, 4096]: the weight-streaming
    small-M forward (split-free up to 16 rows, ranges + reduce at 32 and 64) and
    input gradient (ranges of weight rows + reduce), each with its rank-16
    LoRA term at an init that makes the term as large as the base product;
    whole matrix and every fragment against fp32 on the oracle weight."""
    from stratum_amd.functional import nf4_gemm_bwd_dx, nf4_gemm_fwd
    _, N, K, R = LORA_STEP
    s = lora_step
    x, dy = s["x"][:M].contiguous(), s["dy"][:M].contiguous()
    A = seeded((R, K), 20, 0.1, torch.bfloat16).to(cuda)
    B = seeded((N, R), 21, 0.1, torch.bfloat16).to(cuda)
    t = (x.float() @ A.float().t().contiguous()).to(torch.bfloat16)
    u = (dy.float() @ B.float()).to(torch.bfloat16)
    y = nf4_gemm_fwd(x, s["q"], s["a"], (N, K), 64, lora_t=t, lora_b=B)
    ref = x.float() @ s["w"].t().contiguous() + t.float() @ B.float().t().contiguous()
    assert_gemm_close(y, ref, torch.bfloat16, f"M = {M} forward with LoRA")
    dx = nf4_gemm_bwd_dx(dy, s["q"], s["a"], (N, K), 64, lora_u=u, lora_at=A.t().contiguous())
    ref = dy.float() @ s["w"] + u.float() @ A.float()
    assert_gemm_close(dx, ref, torch.bfloat16, f"M = {M} input gradient with U . A")
