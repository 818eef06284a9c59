"""Frozen SwiGLU MLP with a token-chunked forward and a chunk-by-chunk
backward recompute, with an NF4 fast path for MI355X.

Same module and autograd function as the reference's memory-flat frozen MLP
(``stratum/model/mlp_opt.py:103-245``): ``MemoryFlatFrozenMLP(module,
token_chunk_size)`` wraps a frozen dense MLP ``down(act_fn(gate(x)) * up(x))``
with either Qwen (``gate_proj``/``up_proj``/``down_proj``) or LFM2.5
(``ffn_*_proj``) projection names, runs the forward over token chunks without
keeping the 3x-hidden intermediate, and recomputes one chunk at a time in the
backward to produce the input gradient (the parameters are frozen).

When the three projections are :class:`~stratum_amd.nf4_linear.NF4Linear`
(packed NF4 weights resident on the GPU) the chunk math runs on the HIP
library instead of autograd:

* gate and up are stacked once into one packed payload ``[2 I, H]`` (NF4 rows
  are independent: the stack is the byte concatenation of the two payloads and
  of their absmax), so each is ONE fused dequant-GEMM with N = 2 I;
* ``silu(gate) * up`` and its gradient are single HIP passes (``swiglu_fwd``,
  ``swiglu_bwd``) in fp32 with one rounding;
* the backward of a chunk is ``gu = X Wguᵀ`` (recompute), ``dh = dY Wd``,
  ``dgu = swiglu_bwd(dh, gu)``, ``dX = dgu Wgu``: five GEMM units of
  ``2·rows·H·I`` flops against the reference's six (it also recomputes the
  down projection's output, which the input gradient does not need);
* chunks larger than ``fused_max_rows()`` rows dequantize the stacked weights
  once per call and run those GEMMs on the library (see ``nf4_linear``).

Chunks are taken over the flattened tokens, ``token_chunk_size`` tokens of
every batch row at a time, so the peak intermediate is the reference's
(``token_chunk_size · batch · 2 I``); the MLP is positionwise, so each token's
result does not depend on the chunking.
"""

from __future__ import annotations

from typing import Any, NamedTuple, Optional

import torch
import torch.nn as nn

from .functional import (dequantize_4bit, fused_supported, nf4_gemm_bwd_dx, nf4_gemm_fwd, quantize_4bit, swiglu_bwd,
                         swiglu_fwd)
from .nf4_linear import NF4Linear, fused_max_rows

__all__ = [
    "MemoryFlatFrozenMLP",
    "MemoryFlatFrozenMLPFunction",
    "NF4StackedMLP",
    "quantize_mlp_",
]


class _MlpProjectionNames(NamedTuple):
    gate: str
    up: str
    down: str


def _mlp_projection_names(module: nn.Module) -> _MlpProjectionNames:
    """Projection attribute names of a dense MLP (``stratum/model/mlp_opt.py:109-115``)."""
    if hasattr(module, "gate_exps"):
        raise TypeError("memory-flat frozen MLP does not support MoE expert modules")
    if hasattr(module, "ffn_gate_proj"):
        return _MlpProjectionNames("ffn_gate_proj", "ffn_up_proj", "ffn_down_proj")
    return _MlpProjectionNames("gate_proj", "up_proj", "down_proj")


def _assert_frozen_mlp(module: nn.Module) -> _MlpProjectionNames:
    """Validate a frozen dense MLP (``stratum/model/mlp_opt.py:118-151``).

    Projections may be ``nn.Linear`` (dense weights) or ``NF4Linear`` (packed
    NF4 weights); the errors are the reference's.
    """
    proj_names = _mlp_projection_names(module)
    missing = [name for name in proj_names if not hasattr(module, name)]
    if missing:
        raise TypeError(f"memory-flat frozen MLP requires gate/up/down projections, missing: {missing}")
    if not hasattr(module, "act_fn"):
        raise TypeError("memory-flat frozen MLP requires act_fn (SiLU)")
    trainable = [name for name, param in module.named_parameters() if param.requires_grad]
    if trainable:
        raise ValueError("--memory-flat-frozen-mlp only supports frozen MLP parameters; "
                         f"trainable parameters found: {trainable[:8]}")
    for name in proj_names:
        proj = getattr(module, name)
        if not isinstance(proj, (nn.Linear, NF4Linear)):
            raise TypeError(f"memory-flat frozen MLP expected {name} to be nn.Linear, got {type(proj)!r}")
        if proj.bias is not None:
            raise TypeError(f"memory-flat frozen MLP currently expects bias=False for {name}")
    return proj_names


class NF4StackedMLP:
    """Device-resident packed weights of an NF4 SwiGLU MLP: ``[gate; up]``
    stacked into one ``[2 I, H]`` payload, and ``down`` ``[H, I]``."""

    def __init__(self, gate: NF4Linear, up: NF4Linear, down: NF4Linear):
        gs, us, ds = gate.quant_state, up.quant_state, down.quant_state
        inter, hidden = (int(s) for s in gs.shape)
        if tuple(us.shape) != (inter, hidden) or tuple(ds.shape) != (hidden, inter):
            raise ValueError("gate/up must be [I, H] and down [H, I]")
        if not (gs.blocksize == us.blocksize == ds.blocksize):
            raise ValueError("gate, up and down must share one blocksize")
        self.hidden, self.inter, self.blocksize = hidden, inter, gs.blocksize
        self.gu_packed = torch.cat([gate.quantized.reshape(-1), up.quantized.reshape(-1)])
        self.gu_absmax = torch.cat([gs.absmax.reshape(-1), us.absmax.reshape(-1)]).float()
        self.d_packed = down.quantized.reshape(-1)
        self.d_absmax = ds.absmax.reshape(-1).float()
        self.key = (gate.quantized.data_ptr(), up.quantized.data_ptr(), down.quantized.data_ptr())

    @staticmethod
    def supported(hidden: int, inter: int, blocksize: int) -> bool:
        return (fused_supported(2 * inter, hidden, blocksize, backward=True)
                and fused_supported(hidden, inter, blocksize, backward=True))

    def _fused(self, rows_per_chunk: int) -> bool:
        limit = fused_max_rows()
        return limit < 0 or rows_per_chunk <= limit

    def _dense(self, dtype: torch.dtype):
        """Dequantized [2 I, H] and [H, I] temporaries for the library-GEMM path."""
        H, I, bs = self.hidden, self.inter, self.blocksize
        w_gu = dequantize_4bit(self.gu_packed, absmax=self.gu_absmax, blocksize=bs, dtype=dtype, shape=(2 * I, H))
        w_d = dequantize_4bit(self.d_packed, absmax=self.d_absmax, blocksize=bs, dtype=dtype, shape=(H, I))
        return w_gu, w_d

    def forward_rows(self, x: torch.Tensor, out: torch.Tensor, rows_per_chunk: int) -> None:
        """``out[r] = down(silu(gate(x[r])) * up(x[r]))`` for the rows of ``x`` [rows, H].

        Chunks of at most ``fused_max_rows()`` rows run the fused kernels; larger
        chunks dequantize the stacked weights once for the whole call and run
        the library GEMM (the faster choice there, see ``nf4_linear``).
        """
        H, I, bs = self.hidden, self.inter, self.blocksize
        if not self._fused(rows_per_chunk):
            w_gu, w_d = self._dense(x.dtype)
            for s in range(0, x.shape[0], rows_per_chunk):
                e = min(s + rows_per_chunk, x.shape[0])
                h = swiglu_fwd(x[s:e] @ w_gu.t())
                torch.matmul(h, w_d.t(), out=out[s:e])
            return
        for s in range(0, x.shape[0], rows_per_chunk):
            e = min(s + rows_per_chunk, x.shape[0])
            gu = nf4_gemm_fwd(x[s:e], self.gu_packed, self.gu_absmax, (2 * I, H), bs)
            h = swiglu_fwd(gu)
            nf4_gemm_fwd(h, self.d_packed, self.d_absmax, (H, I), bs, out=out[s:e])

    def input_grad_rows(self, x: torch.Tensor, dy: torch.Tensor, dx: torch.Tensor, rows_per_chunk: int) -> None:
        """``dx[r]`` = gradient of the MLP output row r (given ``dy[r]``) with respect to ``x[r]``."""
        H, I, bs = self.hidden, self.inter, self.blocksize
        if not self._fused(rows_per_chunk):
            w_gu, w_d = self._dense(x.dtype)
            for s in range(0, x.shape[0], rows_per_chunk):
                e = min(s + rows_per_chunk, x.shape[0])
                gu = x[s:e] @ w_gu.t()
                dgu = swiglu_bwd(dy[s:e] @ w_d, gu)
                torch.matmul(dgu, w_gu, out=dx[s:e])
            return
        for s in range(0, x.shape[0], rows_per_chunk):
            e = min(s + rows_per_chunk, x.shape[0])
            gu = nf4_gemm_fwd(x[s:e], self.gu_packed, self.gu_absmax, (2 * I, H), bs)
            dh = nf4_gemm_bwd_dx(dy[s:e], self.d_packed, self.d_absmax, (H, I), bs)
            dgu = swiglu_bwd(dh, gu)
            nf4_gemm_bwd_dx(dgu, self.gu_packed, self.gu_absmax, (2 * I, H), bs, out=dx[s:e])


_STACK_ATTR = "_stratum_nf4_stack"
_SILU_PROBE = torch.tensor([-6.0, -1.25, -0.5, 0.0, 0.75, 2.0, 9.0])


def _is_silu(act) -> bool:
    """``act`` computes SiLU (``nn.SiLU``, transformers' ``SiLUActivation``, ...): checked once
    on a few CPU values, cached on the object."""
    if isinstance(act, nn.SiLU):
        return True
    cached = getattr(act, "_stratum_is_silu", None)
    if cached is None:
        try:
            with torch.no_grad():
                cached = bool(torch.allclose(act(_SILU_PROBE.clone()), nn.functional.silu(_SILU_PROBE),
                                             rtol=1e-6, atol=1e-7))
        except Exception:
            cached = False
        try:
            object.__setattr__(act, "_stratum_is_silu", cached)
        except (AttributeError, TypeError):
            pass
    return cached


def _nf4_stack(module: nn.Module, names: _MlpProjectionNames, x: torch.Tensor) -> Optional[NF4StackedMLP]:
    """The NF4 fast path for ``module`` and input ``x``, or None when it does not apply."""
    gate, up, down = (getattr(module, n) for n in names)
    if not (isinstance(gate, NF4Linear) and isinstance(up, NF4Linear) and isinstance(down, NF4Linear)):
        return None
    if not _is_silu(module.act_fn):
        return None
    if not (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)):
        return None
    if any(p.quantized.device != x.device for p in (gate, up, down)):
        return None
    inter, hidden = (int(s) for s in gate.quant_state.shape)
    if x.shape[-1] != hidden or not NF4StackedMLP.supported(hidden, inter, gate.quant_state.blocksize):
        return None
    stack = getattr(module, _STACK_ATTR, None)
    key = (gate.quantized.data_ptr(), up.quantized.data_ptr(), down.quantized.data_ptr())
    if stack is None or stack.key != key:
        stack = NF4StackedMLP(gate, up, down)
        object.__setattr__(module, _STACK_ATTR, stack)  # not a submodule / parameter
    return stack


def _rows_per_chunk(hidden_states: torch.Tensor, token_chunk_size: int) -> int:
    batch = 1
    for d in hidden_states.shape[:-2]:
        batch *= int(d)
    return max(1, token_chunk_size * batch)


class MemoryFlatFrozenMLPFunction(torch.autograd.Function):
    """Custom autograd: forward runs the MLP in chunks, backward recomputes one
    chunk at a time (``stratum/model/mlp_opt.py:154-215``)."""

    @staticmethod
    def forward(ctx: Any, hidden_states: torch.Tensor, module: nn.Module, token_chunk_size: int) -> torch.Tensor:
        proj_names = _assert_frozen_mlp(module)
        if token_chunk_size <= 0:
            raise ValueError("token_chunk_size must be positive")
        if hidden_states.dim() < 3:
            raise ValueError("memory-flat frozen MLP expects [batch, seq, hidden] input")

        ctx.module = module
        ctx.proj_names = proj_names
        ctx.token_chunk_size = token_chunk_size
        ctx.save_for_backward(hidden_states)

        stack = _nf4_stack(module, proj_names, hidden_states)
        ctx.stack = stack
        if stack is not None:
            x = hidden_states.reshape(-1, stack.hidden).contiguous()
            out = torch.empty_like(x)
            stack.forward_rows(x, out, _rows_per_chunk(hidden_states, token_chunk_size))
            return out.reshape(hidden_states.shape)

        seq_len = hidden_states.shape[1]
        gate_proj, up_proj, down_proj = (getattr(module, n) for n in proj_names)
        output = hidden_states.new_empty(*hidden_states.shape[:-1], down_proj.out_features)
        with torch.no_grad():
            for start in range(0, seq_len, token_chunk_size):
                end = min(start + token_chunk_size, seq_len)
                chunk = hidden_states[:, start:end, :]
                output[:, start:end, :] = down_proj(module.act_fn(gate_proj(chunk)) * up_proj(chunk))
        return output

    @staticmethod
    def backward(ctx: Any, grad_output: torch.Tensor) -> tuple[Optional[torch.Tensor], None, None]:
        (hidden_states,) = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None
        module, proj_names, token_chunk_size = ctx.module, ctx.proj_names, ctx.token_chunk_size
        stack = ctx.stack
        if stack is not None:
            x = hidden_states.reshape(-1, stack.hidden).contiguous()
            dy = grad_output.reshape(-1, stack.hidden).contiguous()
            dx = torch.empty_like(x)
            stack.input_grad_rows(x, dy, dx, _rows_per_chunk(hidden_states, token_chunk_size))
            return dx.reshape(hidden_states.shape), None, None

        seq_len = hidden_states.shape[1]
        grad_hidden_states = torch.empty_like(hidden_states)
        gate_proj, up_proj, down_proj = (getattr(module, n) for n in proj_names)
        with torch.enable_grad():
            for start in range(0, seq_len, token_chunk_size):
                end = min(start + token_chunk_size, seq_len)
                chunk = hidden_states[:, start:end, :].detach().requires_grad_(True)
                chunk_output = down_proj(module.act_fn(gate_proj(chunk)) * up_proj(chunk))
                (grad_chunk,) = torch.autograd.grad(chunk_output, chunk, grad_outputs=grad_output[:, start:end, :],
                                                    retain_graph=False, create_graph=False)
                grad_hidden_states[:, start:end, :] = grad_chunk
        return grad_hidden_states, None, None


class MemoryFlatFrozenMLP(nn.Module):
    """Frozen MLP with token-sliced backward recompute (``stratum/model/mlp_opt.py:218-245``)."""

    def __init__(self, module: nn.Module, token_chunk_size: int) -> None:
        super().__init__()
        if token_chunk_size <= 0:
            raise ValueError("token_chunk_size must be positive")
        _assert_frozen_mlp(module)
        self.module = module
        self.token_chunk_size = token_chunk_size

    def forward(self, hidden_states: torch.Tensor, *args: Any, **kwargs: Any) -> torch.Tensor:
        if args or kwargs:
            raise ValueError("MemoryFlatFrozenMLP only supports a hidden_states positional argument")
        if hidden_states.shape[1] <= self.token_chunk_size and not hidden_states.requires_grad:
            stack = _nf4_stack(self.module, _mlp_projection_names(self.module), hidden_states)
            if stack is None:
                return self.module(hidden_states)
            with torch.no_grad():
                x = hidden_states.reshape(-1, stack.hidden).contiguous()
                out = torch.empty_like(x)
                stack.forward_rows(x, out, x.shape[0])
            return out.reshape(hidden_states.shape)
        return MemoryFlatFrozenMLPFunction.apply(hidden_states, self.module, self.token_chunk_size)

    def named_parameters(self, prefix: str = "", recurse: bool = True, remove_duplicate: bool = True):
        yield from self.module.named_parameters(prefix=prefix, recurse=recurse, remove_duplicate=remove_duplicate)

    def named_buffers(self, prefix: str = "", recurse: bool = True, remove_duplicate: bool = True):
        yield from self.module.named_buffers(prefix=prefix, recurse=recurse, remove_duplicate=remove_duplicate)


@torch.no_grad()
def quantize_mlp_(module: nn.Module, device: Optional[torch.device] = None, blocksize: int = 64) -> nn.Module:
    """Replace the dense gate/up/down ``nn.Linear`` of ``module`` with NF4Linear
    (quantized on the GPU, packed weights resident on ``device``). In place."""
    names = _mlp_projection_names(module)
    for name in names:
        lin = getattr(module, name)
        if isinstance(lin, NF4Linear):
            continue
        if not isinstance(lin, nn.Linear) or lin.bias is not None:
            raise TypeError(f"{name} must be a bias-free nn.Linear")
        w = lin.weight.detach()
        dev = torch.device(device) if device is not None else (w.device if w.is_cuda else torch.device("cuda"))
        packed, state = quantize_4bit(w.to(dev), blocksize=blocksize)
        setattr(module, name, NF4Linear(packed, state))
    return module
