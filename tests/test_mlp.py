"""CPU tests of the memory-flat frozen MLP wrapper (dense projections), in the
shape of the reference's own tests (tests/test_mlp_opt.py:24-105): forward and
input gradient equal the unwrapped MLP for both projection naming schemes, and
the validation errors of stratum/model/mlp_opt.py:118-151."""

import pytest
import torch
import torch.nn as nn

from stratum_amd.mlp import (MemoryFlatFrozenMLP, MemoryFlatFrozenMLPFunction, _assert_frozen_mlp,
                             _mlp_projection_names)


class StandardDenseMlp(nn.Module):
    def __init__(self, h=4, i=6):
        super().__init__()
        self.gate_proj = nn.Linear(h, i, bias=False)
        self.up_proj = nn.Linear(h, i, bias=False)
        self.down_proj = nn.Linear(i, h, bias=False)
        self.act_fn = nn.SiLU()

    def forward(self, hidden_states):
        return self.down_proj(self.act_fn(self.gate_proj(hidden_states)) * self.up_proj(hidden_states))


class FfnDenseMlp(nn.Module):
    def __init__(self):
        super().__init__()
        self.ffn_gate_proj = nn.Linear(4, 6, bias=False)
        self.ffn_up_proj = nn.Linear(4, 6, bias=False)
        self.ffn_down_proj = nn.Linear(6, 4, bias=False)
        self.act_fn = nn.SiLU()

    def forward(self, hidden_states):
        return self.ffn_down_proj(self.act_fn(self.ffn_gate_proj(hidden_states)) * self.ffn_up_proj(hidden_states))


def _freeze(module):
    for p in module.parameters():
        p.requires_grad_(False)
    return module


def _assert_matches_unwrapped(module, shape=(2, 7, 4), chunk=3):
    torch.manual_seed(1234)
    module = _freeze(module)
    wrapped = MemoryFlatFrozenMLP(module, token_chunk_size=chunk)
    expected_input = torch.randn(*shape, requires_grad=True)
    actual_input = expected_input.detach().clone().requires_grad_(True)
    expected = module(expected_input)
    actual = wrapped(actual_input)
    assert torch.allclose(actual, expected, atol=1e-6, rtol=1e-6)
    expected.square().sum().backward()
    actual.square().sum().backward()
    assert torch.allclose(actual_input.grad, expected_input.grad, atol=1e-6, rtol=1e-6)


def test_standard_projection_names_match_unwrapped_mlp():
    _assert_matches_unwrapped(StandardDenseMlp())


def test_lfm_ffn_projection_names_match_unwrapped_mlp():
    _assert_matches_unwrapped(FfnDenseMlp())


@pytest.mark.parametrize("chunk", [1, 2, 7, 50])
def test_chunk_sizes_including_one_chunk_and_ragged_last(chunk):
    _assert_matches_unwrapped(StandardDenseMlp(8, 12), shape=(3, 7, 8), chunk=chunk)


def test_short_sequence_without_grad_calls_module_directly():
    calls = []
    m = _freeze(StandardDenseMlp())
    m.register_forward_hook(lambda *a: calls.append(1))
    y = MemoryFlatFrozenMLP(m, token_chunk_size=8)(torch.randn(1, 5, 4))
    assert y.shape == (1, 5, 4) and calls == [1]


def test_projection_names():
    assert _mlp_projection_names(StandardDenseMlp()).gate == "gate_proj"
    assert _mlp_projection_names(FfnDenseMlp()).down == "ffn_down_proj"


def test_moe_module_rejected():
    m = nn.Module()
    m.gate_exps = nn.Parameter(torch.empty(1), requires_grad=False)
    with pytest.raises(TypeError, match="MoE"):
        _mlp_projection_names(m)


def test_missing_projection_rejected():
    m = _freeze(StandardDenseMlp())
    del m.up_proj
    with pytest.raises(TypeError, match="missing"):
        _assert_frozen_mlp(m)


def test_missing_act_fn_rejected():
    m = _freeze(StandardDenseMlp())
    del m.act_fn
    with pytest.raises(TypeError, match="act_fn"):
        _assert_frozen_mlp(m)


def test_trainable_parameters_rejected():
    m = StandardDenseMlp()
    with pytest.raises(ValueError, match="trainable parameters found"):
        MemoryFlatFrozenMLP(m, token_chunk_size=4)


def test_bias_rejected():
    m = StandardDenseMlp()
    m.down_proj = nn.Linear(6, 4, bias=True)
    with pytest.raises(TypeError, match="bias=False"):
        _assert_frozen_mlp(_freeze(m))


def test_non_linear_projection_rejected():
    m = StandardDenseMlp()
    m.gate_proj = nn.Identity()
    with pytest.raises(TypeError, match="nn.Linear"):
        _assert_frozen_mlp(_freeze(m))


def test_bad_chunk_and_rank():
    m = _freeze(StandardDenseMlp())
    with pytest.raises(ValueError, match="positive"):
        MemoryFlatFrozenMLP(m, token_chunk_size=0)
    with pytest.raises(ValueError, match="batch, seq, hidden"):
        MemoryFlatFrozenMLPFunction.apply(torch.randn(5, 4, requires_grad=True), m, 2)


def test_extra_arguments_rejected():
    w = MemoryFlatFrozenMLP(_freeze(StandardDenseMlp()), token_chunk_size=2)
    with pytest.raises(ValueError, match="hidden_states positional"):
        w(torch.randn(1, 3, 4), torch.randn(1))


def test_named_parameters_pass_through():
    m = _freeze(StandardDenseMlp())
    w = MemoryFlatFrozenMLP(m, token_chunk_size=2)
    assert [n for n, _ in w.named_parameters()] == [n for n, _ in m.named_parameters()]


def test_silu_detection_accepts_transformers_activation():
    from transformers.activations import ACT2FN
    from stratum_amd.mlp import _is_silu
    assert _is_silu(nn.SiLU()) and _is_silu(ACT2FN["silu"])
    assert not _is_silu(nn.GELU()) and not _is_silu(torch.tanh)


def test_stacked_nf4_weights_are_rebuilt_when_a_source_changes():
    """The stacked [gate; up] copy is served only for the very payload tensors it
    was built from, unmodified: an in-place update or a replacement (even one
    that reuses the freed tensor's id or address) does not match."""
    from stratum_amd.functional import QuantState
    from stratum_amd.mlp import NF4StackedMLP
    from stratum_amd.nf4_linear import NF4Linear

    H, I, bs = 64, 128, 64

    def lin(rows, cols, seed):
        g = torch.Generator().manual_seed(seed)
        q = torch.randint(0, 256, (rows * cols // 2, 1), dtype=torch.uint8, generator=g)
        st = QuantState(absmax=torch.rand(rows * cols // bs, generator=g), shape=(rows, cols), blocksize=bs,
                        quant_type="nf4", dtype=torch.bfloat16)
        return NF4Linear(q, st)

    gate, up, down = lin(I, H, 1), lin(I, H, 2), lin(H, I, 3)
    stack = NF4StackedMLP(gate, up, down)
    assert not stack.shares_storage  # separate payloads: one concatenated copy
    assert torch.equal(stack.gu_packed, torch.cat([gate.quantized.reshape(-1), up.quantized.reshape(-1)]))
    assert stack.matches(gate, up, down)
    up.quant_state.absmax.mul_(1.0)  # in-place: version bump
    assert not stack.matches(gate, up, down)
    stack = NF4StackedMLP(gate, up, down)
    assert stack.matches(gate, up, down)
    gate.quantized = gate.quantized.clone()  # a new tensor with the same contents
    assert not stack.matches(gate, up, down)
