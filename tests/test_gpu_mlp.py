"""GPU tests of the frozen SwiGLU MLP path: the SwiGLU kernels against fp32
torch, and MemoryFlatFrozenMLP with NF4 projections against an fp32 reference
computed on the oracle-dequantized weights (floating point: rel-err tolerance
1e-2 for bf16, 5e-3 for fp16, written below)."""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-3}


def rel(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def ulps16(a, ref, dtype):
    """Max distance in units of the 16-bit format's spacing at the reference value."""
    eps = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
    scale = ref.abs().clamp_min(torch.finfo(dtype).tiny)
    return ((a.float() - ref) / (scale * eps)).abs().max().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,inter", [(257, 1024), (3, 8), (50, 36), (0, 16)])
def test_swiglu_fwd_matches_fp32(cuda, dtype, rows, inter):
    from stratum_amd.functional import swiglu_fwd
    g = torch.Generator().manual_seed(rows * 31 + inter)
    gu = (torch.randn(rows, 2 * inter, generator=g) * 3).to(dtype).to(cuda)
    h = swiglu_fwd(gu)
    assert h.shape == (rows, inter) and h.dtype == dtype
    gf, uf = gu[:, :inter].float(), gu[:, inter:].float()
    ref = F.silu(gf) * uf
    if rows:
        # one rounding of an fp32 result: within one 16-bit step of the fp32 value
        assert ulps16(h, ref, dtype) <= 1.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,inter", [(129, 2048), (7, 24)])
def test_swiglu_bwd_matches_autograd(cuda, dtype, rows, inter):
    from stratum_amd.functional import swiglu_bwd
    g = torch.Generator().manual_seed(rows + inter)
    gu = (torch.randn(rows, 2 * inter, generator=g) * 3).to(dtype).to(cuda)
    dh = torch.randn(rows, inter, generator=g).to(dtype).to(cuda)
    dgu = swiglu_bwd(dh, gu)
    x = gu.float().requires_grad_(True)
    (F.silu(x[:, :inter]) * x[:, inter:]).backward(dh.float())
    ref = x.grad
    # products of up to four fp32 factors rounded once: a few fp32 ulps, then one 16-bit rounding
    assert ulps16(dgu, ref, dtype) <= 1.01


def test_swiglu_unaligned_input_uses_scalar_path(cuda):
    from stratum_amd.functional import swiglu_fwd
    base = torch.randn(1, 2 * 64 * 5 + 1, device=cuda).to(torch.bfloat16)
    gu = base[0, 1:].reshape(5, 128)  # 2-byte offset: not 16-byte aligned, contiguous
    h = swiglu_fwd(gu)
    ref = F.silu(gu[:, :64].float()) * gu[:, 64:].float()
    assert ulps16(h, ref, torch.bfloat16) <= 1.0


class DenseMlp(nn.Module):
    def __init__(self, h, i, dtype, device, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        mk = lambda o, n: nn.Linear(n, o, bias=False)
        self.gate_proj, self.up_proj, self.down_proj = mk(i, h), mk(i, h), mk(h, i)
        for lin in (self.gate_proj, self.up_proj, self.down_proj):
            lin.weight.data = (torch.randn(lin.weight.shape, generator=g) * 0.02).half().to(dtype).to(device)
            lin.weight.requires_grad_(False)
        self.act_fn = nn.SiLU()

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


def _oracle_weights(dense, dtype, device):
    """fp32 copies of the oracle's dequantization of each projection weight."""
    out = {}
    tag = O.DT_F16 if dtype == torch.float16 else O.DT_BF16
    for name in ("gate_proj", "up_proj", "down_proj"):
        w = getattr(dense, name).weight.detach().cpu().contiguous()
        bits = w.view(torch.int16).numpy().view(np.uint16)
        p, a = C.quantize(bits, tag, 64, "argmin")
        deq = C.dequantize(p, a, w.numel(), 64, tag).view(np.int16).reshape(w.shape)
        out[name] = torch.from_numpy(deq).view(dtype).float().to(device)
    return out


@pytest.mark.parametrize("chunk", [96, 300])  # 192 rows per chunk: fused kernels; 600: library GEMM
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_nf4_memory_flat_mlp_matches_fp32_reference(cuda, dtype, chunk, monkeypatch):
    from stratum_amd.mlp import MemoryFlatFrozenMLP, _STACK_ATTR, quantize_mlp_
    monkeypatch.delenv("STRATUM_NF4_FUSED_MAX_ROWS", raising=False)
    H, I = 1024, 3072
    dense = DenseMlp(H, I, dtype, cuda, seed=5)
    W = _oracle_weights(dense, dtype, cuda)
    mlp = quantize_mlp_(dense)
    wrapped = MemoryFlatFrozenMLP(mlp, token_chunk_size=chunk)
    g = torch.Generator().manual_seed(9)
    x0 = torch.randn(2, 300, H, generator=g).to(dtype).to(cuda)
    x = x0.clone().requires_grad_(True)
    y = wrapped(x)
    assert getattr(mlp, _STACK_ATTR, None) is not None, "NF4 fast path not taken"
    wy = torch.randn(y.shape, generator=g).to(dtype).to(cuda)
    (y.float() * wy.float()).sum().backward()

    xr = x0.float().requires_grad_(True)
    yr = F.linear(F.silu(F.linear(xr, W["gate_proj"])) * F.linear(xr, W["up_proj"]), W["down_proj"])
    (yr * wy.float()).sum().backward()
    assert rel(y, yr) < TOL[dtype]
    assert rel(x.grad, xr.grad) < TOL[dtype]


def test_nf4_mlp_result_does_not_depend_on_chunking(cuda):
    from stratum_amd.mlp import MemoryFlatFrozenMLP, quantize_mlp_
    H, I = 512, 1536
    mlp = quantize_mlp_(DenseMlp(H, I, torch.bfloat16, cuda, seed=2))
    x0 = torch.randn(3, 200, H, device=cuda).to(torch.bfloat16)
    dy = torch.randn(3, 200, H, device=cuda).to(torch.bfloat16)
    outs, grads = [], []
    for chunk in (1000, 64, 7):
        x = x0.clone().requires_grad_(True)
        y = MemoryFlatFrozenMLP(mlp, token_chunk_size=chunk)(x)
        y.backward(dy)
        outs.append(y.detach())
        grads.append(x.grad)
    # rows are independent; chunk size only changes how the GEMMs split their
    # reductions (fp32 summation order), so results agree to 16-bit rounding
    for o, gr in zip(outs[1:], grads[1:]):
        assert rel(o, outs[0]) < 4e-3
        assert rel(gr, grads[0]) < 4e-3


def test_nf4_mlp_no_grad_short_sequence_uses_fast_path(cuda):
    from stratum_amd.mlp import MemoryFlatFrozenMLP, quantize_mlp_
    H, I = 256, 512
    mlp = quantize_mlp_(DenseMlp(H, I, torch.bfloat16, cuda, seed=4))
    x = torch.randn(1, 40, H, device=cuda).to(torch.bfloat16)
    with torch.no_grad():
        y_fast = MemoryFlatFrozenMLP(mlp, token_chunk_size=64)(x)
        y_mod = mlp(x)  # the module's own forward: three NF4Linear calls and torch's silu/mul
    assert rel(y_fast, y_mod) < 1e-2


def test_dense_mlp_on_gpu_matches_unwrapped(cuda):
    from stratum_amd.mlp import MemoryFlatFrozenMLP
    dense = DenseMlp(128, 256, torch.float32, cuda, seed=8)
    x = torch.randn(2, 33, 128, device=cuda, requires_grad=True)
    xr = x.detach().clone().requires_grad_(True)
    y = MemoryFlatFrozenMLP(dense, token_chunk_size=5)(x)
    yr = dense(xr)
    y.square().sum().backward()
    yr.square().sum().backward()
    assert torch.allclose(y, yr, atol=1e-5, rtol=1e-5)
    assert torch.allclose(x.grad, xr.grad, atol=1e-5, rtol=1e-5)


def test_nf4_mlp_unsupported_shape_falls_back_to_module_math(cuda):
    from stratum_amd.mlp import MemoryFlatFrozenMLP, _STACK_ATTR, quantize_mlp_
    H, I = 192, 200  # 2 I = 400 is not a multiple of 64: the fused input gradient does not apply
    dense = DenseMlp(H, I, torch.bfloat16, cuda, seed=6)
    W = _oracle_weights(dense, torch.bfloat16, cuda)
    mlp = quantize_mlp_(dense)
    x0 = torch.randn(1, 50, H, device=cuda).to(torch.bfloat16)
    x = x0.clone().requires_grad_(True)
    y = MemoryFlatFrozenMLP(mlp, token_chunk_size=16)(x)
    assert getattr(mlp, _STACK_ATTR, None) is None
    y.float().sum().backward()
    xr = x0.float().requires_grad_(True)
    yr = F.linear(F.silu(F.linear(xr, W["gate_proj"])) * F.linear(xr, W["up_proj"]), W["down_proj"])
    yr.sum().backward()
    assert rel(y, yr) < 1e-2 and rel(x.grad, xr.grad) < 1e-2


def test_quantize_mlp_stacks_gate_and_up_without_a_copy(cuda):
    """quantize_mlp_ quantizes gate and up as one [2 I, H] weight: each half is
    bit-exact to the oracle's quantization of that projection alone, the two
    NF4Linear hold views of the one buffer, and the fused MLP path uses it
    without concatenating a copy; an in-place change to a payload rebuilds the
    stacked view's key."""
    from stratum_amd.mlp import NF4StackedMLP, _nf4_stack, _mlp_projection_names, quantize_mlp_
    H, I = 512, 1536
    dense = DenseMlp(H, I, torch.bfloat16, cuda, seed=11)
    src = {n: getattr(dense, n).weight.detach().cpu().clone() for n in ("gate_proj", "up_proj", "down_proj")}
    mlp = quantize_mlp_(dense)
    for n, w in src.items():
        bits = w.contiguous().view(torch.int16).numpy().view(np.uint16)
        rp, ra = C.quantize(bits, O.DT_BF16, 64, "argmin")
        lin = getattr(mlp, n)
        np.testing.assert_array_equal(lin.quantized.cpu().numpy().ravel(), rp)
        np.testing.assert_array_equal(lin.quant_state.absmax.cpu().numpy().view(np.uint32), ra.view(np.uint32))
    gq, uq = mlp.gate_proj.quantized, mlp.up_proj.quantized
    assert gq.untyped_storage().data_ptr() == uq.untyped_storage().data_ptr()
    x = torch.randn(1, 8, H, device=cuda).to(torch.bfloat16)
    stack = _nf4_stack(mlp, _mlp_projection_names(mlp), x)
    assert isinstance(stack, NF4StackedMLP) and stack.shares_storage
    assert stack.gu_packed.data_ptr() == gq.data_ptr() and stack.gu_packed.numel() == gq.numel() + uq.numel()
    mlp.down_proj.quant_state.absmax.mul_(1.0)  # in place: version bump
    assert _nf4_stack(mlp, _mlp_projection_names(mlp), x) is not stack
