"""Frozen SwiGLU MLP with a token-chunked forward and a chunk-by-chunk
recompute in the backward, with an NF4 fast path for MI355X.

Interface of the reference's memory-flat frozen MLP
(``stratum/model/mlp_opt.py:103-245``): ``MemoryFlatFrozenMLP(module,
token_chunk_size)`` wraps a frozen MLP ``down(act_fn(gate(x)) * up(x))`` with
either Qwen (``gate_proj``/``up_proj``/``down_proj``) or LFM2.5 (``ffn_*_proj``)
projection names, never holds the whole ``[tokens, intermediate]`` activation,
and recomputes one chunk at a time in the backward to produce the input
gradient (the parameters are frozen).

Here the MLP is treated as a function of token rows: the input is flattened to
``[rows, hidden]`` and processed ``token_chunk_size * batch`` rows at a time
(each token's result does not depend on the chunking). Two row engines do the
work:

* ``NF4StackedMLP`` when the projections are :class:`NF4Linear` (packed
  weights resident on the GPU) with a SiLU gate: gate and up are one stacked
  ``[2 I, H]`` payload (``quantize_mlp_`` quantizes them into one buffer and
  the two NF4Linear hold views of it, so nothing is duplicated), each
  projection pair is ONE fused dequant-GEMM, ``silu(g) * u`` and its gradient
  are single HIP passes, and the input gradient of a chunk is
  ``dX = swiglu_bwd(dY Wd, X Wguᵀ) Wgu`` -- five GEMM units per chunk, against
  six for a recompute through autograd (which also recomputes the down
  projection's output);
* ``_ModuleRows`` otherwise: the module's own projections, with the input
  gradient of a chunk taken by a backward pass over that chunk's recompute.
"""

from __future__ import annotations

import weakref

from typing import Any, NamedTuple, Optional

import torch
import torch.nn as nn

from .functional import (QuantState, dequantize_4bit, fused_supported, nf4_gemm_bwd_dx, nf4_gemm_fwd, quantize_4bit,
                         swiglu_bwd, swiglu_fwd)
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
    prefix = "ffn_" if hasattr(module, "ffn_gate_proj") else ""
    return _MlpProjectionNames(f"{prefix}gate_proj", f"{prefix}up_proj", f"{prefix}down_proj")


def _assert_frozen_mlp(module: nn.Module) -> _MlpProjectionNames:
    """Check that *module* is a frozen, bias-free gate/up/down MLP with an
    ``act_fn``; projections may be ``nn.Linear`` or ``NF4Linear``. Exception types
    and messages follow ``stratum/model/mlp_opt.py:118-151``."""
    names = _mlp_projection_names(module)
    missing = [n for n in names if not hasattr(module, n)]
    if missing:
        raise TypeError(f"memory-flat frozen MLP requires gate/up/down projections, missing: {missing}")
    if not hasattr(module, "act_fn"):
        raise TypeError("memory-flat frozen MLP requires act_fn (SiLU)")
    trainable = [n for n, p in module.named_parameters() if p.requires_grad]
    if trainable:
        raise ValueError("--memory-flat-frozen-mlp only supports frozen MLP parameters; "
                         f"trainable parameters found: {trainable[:8]}")
    for n in names:
        proj = getattr(module, n)
        if not isinstance(proj, (nn.Linear, NF4Linear)):
            raise TypeError(f"memory-flat frozen MLP expected {n} to be nn.Linear, got {type(proj)!r}")
        if proj.bias is not None:
            raise TypeError(f"memory-flat frozen MLP currently expects bias=False for {n}")
    return names


def _adjacent_view(a: torch.Tensor, b: torch.Tensor) -> Optional[torch.Tensor]:
    """A flat view covering *a* then *b* when *b* starts right where *a* ends in
    the same storage (both contiguous); None otherwise."""
    if not (a.is_contiguous() and b.is_contiguous() and a.dtype == b.dtype and a.device == b.device):
        return None
    if a.untyped_storage().data_ptr() != b.untyped_storage().data_ptr():
        return None
    if b.storage_offset() != a.storage_offset() + a.numel():
        return None
    return a.new_empty(0).set_(a.untyped_storage(), a.storage_offset(), (a.numel() + b.numel(),))


class NF4StackedMLP:
    """Device-resident packed weights of an NF4 SwiGLU MLP as the kernels take
    them: ``[gate; up]`` as one ``[2 I, H]`` payload and ``down`` ``[H, I]``.

    When gate and up are adjacent views of one buffer (``quantize_mlp_``) the
    stacked payload is a view of it; otherwise it is one concatenated copy,
    rebuilt when any source tensor changes (identity or in-place version).
    """

    def __init__(self, gate: NF4Linear, up: NF4Linear, down: NF4Linear):
        gs, us, ds = gate.quant_state, up.quant_state, down.quant_state
        inter, hidden = (int(s) for s in gs.shape)
        if tuple(us.shape) != (inter, hidden) or tuple(ds.shape) != (hidden, inter):
            raise ValueError("gate/up must be [I, H] and down [H, I]")
        if not (gs.blocksize == us.blocksize == ds.blocksize):
            raise ValueError("gate, up and down must share one blocksize")
        self.hidden, self.inter, self.blocksize = hidden, inter, gs.blocksize
        gq, uq = gate.quantized.reshape(-1), up.quantized.reshape(-1)
        ga, ua = gs.absmax.reshape(-1), us.absmax.reshape(-1)
        self.gu_packed = _adjacent_view(gq, uq)
        self.gu_absmax = _adjacent_view(ga, ua) if ga.dtype == torch.float32 else None
        self.shares_storage = self.gu_packed is not None and self.gu_absmax is not None
        if not self.shares_storage:
            self.gu_packed = torch.cat([gq, uq])
            self.gu_absmax = torch.cat([ga, ua]).float()
        self.d_packed = down.quantized.reshape(-1)
        self.d_absmax = ds.absmax.reshape(-1).float()
        # weak references, so a source freed and another tensor allocated at the
        # same address (or with the same id) can never match
        self.key = tuple((weakref.ref(t), t._version) for t in self._sources(gate, up, down))

    @staticmethod
    def _sources(gate: NF4Linear, up: NF4Linear, down: NF4Linear) -> tuple:
        return (gate.quantized, up.quantized, down.quantized, gate.quant_state.absmax, up.quant_state.absmax,
                down.quant_state.absmax)

    def matches(self, gate: NF4Linear, up: NF4Linear, down: NF4Linear) -> bool:
        """Built from these very tensors, none modified in place since."""
        return all(ref() is t and version == t._version
                   for (ref, version), t in zip(self.key, self._sources(gate, up, down)))

    @staticmethod
    def supported(hidden: int, inter: int, blocksize: int) -> bool:
        return (fused_supported(2 * inter, hidden, blocksize, backward=True)
                and fused_supported(hidden, inter, blocksize, backward=True))

    def _library_weights(self, dtype: torch.dtype):
        """Dequantized [2 I, H] and [H, I] temporaries for chunks above the fused
        kernels' row range (dequantized once per call, library GEMMs)."""
        H, I, bs = self.hidden, self.inter, self.blocksize
        return (dequantize_4bit(self.gu_packed, absmax=self.gu_absmax, blocksize=bs, dtype=dtype, shape=(2 * I, H)),
                dequantize_4bit(self.d_packed, absmax=self.d_absmax, blocksize=bs, dtype=dtype, shape=(H, I)))

    def forward_rows(self, x: torch.Tensor, out: torch.Tensor, rows_per_chunk: int) -> None:
        """``out = down(silu(gate(x)) * up(x))`` for x [rows, H], chunk by chunk."""
        H, I, bs = self.hidden, self.inter, self.blocksize
        limit = fused_max_rows()
        if limit < 0 or rows_per_chunk <= limit:
            for s in range(0, x.shape[0], rows_per_chunk):
                c = slice(s, s + rows_per_chunk)
                h = swiglu_fwd(nf4_gemm_fwd(x[c], self.gu_packed, self.gu_absmax, (2 * I, H), bs))
                nf4_gemm_fwd(h, self.d_packed, self.d_absmax, (H, I), bs, out=out[c])
            return
        w_gu, w_d = self._library_weights(x.dtype)
        for s in range(0, x.shape[0], rows_per_chunk):
            c = slice(s, s + rows_per_chunk)
            torch.mm(swiglu_fwd(torch.mm(x[c], w_gu.t())), w_d.t(), out=out[c])

    def input_grad_rows(self, x: torch.Tensor, dy: torch.Tensor, dx: torch.Tensor, rows_per_chunk: int) -> None:
        """``dx`` = gradient of the MLP output rows (``dy``) with respect to ``x``."""
        H, I, bs = self.hidden, self.inter, self.blocksize
        limit = fused_max_rows()
        if limit < 0 or rows_per_chunk <= limit:
            for s in range(0, x.shape[0], rows_per_chunk):
                c = slice(s, s + rows_per_chunk)
                gu = nf4_gemm_fwd(x[c], self.gu_packed, self.gu_absmax, (2 * I, H), bs)
                dgu = swiglu_bwd(nf4_gemm_bwd_dx(dy[c], self.d_packed, self.d_absmax, (H, I), bs), gu)
                nf4_gemm_bwd_dx(dgu, self.gu_packed, self.gu_absmax, (2 * I, H), bs, out=dx[c])
            return
        w_gu, w_d = self._library_weights(x.dtype)
        for s in range(0, x.shape[0], rows_per_chunk):
            c = slice(s, s + rows_per_chunk)
            dgu = swiglu_bwd(torch.mm(dy[c], w_d), torch.mm(x[c], w_gu.t()))
            torch.mm(dgu, w_gu, out=dx[c])


class _ModuleRows:
    """Row engine over the module's own projections (any act_fn)."""

    def __init__(self, module: nn.Module, names: _MlpProjectionNames):
        self.gate, self.up, self.down = (getattr(module, n) for n in names)
        self.act = module.act_fn

    def _mlp(self, x: torch.Tensor) -> torch.Tensor:
        return self.down(self.act(self.gate(x)) * self.up(x))

    def forward_rows(self, x: torch.Tensor, out: torch.Tensor, rows_per_chunk: int) -> None:
        with torch.no_grad():
            for s in range(0, x.shape[0], rows_per_chunk):
                out[s:s + rows_per_chunk] = self._mlp(x[s:s + rows_per_chunk])

    def input_grad_rows(self, x: torch.Tensor, dy: torch.Tensor, dx: torch.Tensor, rows_per_chunk: int) -> None:
        for s in range(0, x.shape[0], rows_per_chunk):
            c = slice(s, s + rows_per_chunk)
            with torch.enable_grad():
                leaf = x[c].detach().requires_grad_(True)
                self._mlp(leaf).backward(dy[c])
            dx[c] = leaf.grad


_STACK_ATTR = "_stratum_nf4_stack"
_SILU_PROBE = torch.tensor([-6.0, -1.25, -0.5, 0.0, 0.75, 2.0, 9.0])


def _is_silu(act) -> bool:
    """``act`` computes SiLU (``nn.SiLU``, transformers' ``SiLUActivation``, ...):
    checked once on a few CPU values and remembered on the object."""
    if isinstance(act, nn.SiLU):
        return True
    known = getattr(act, "_stratum_is_silu", None)
    if known is None:
        try:
            with torch.no_grad():
                known = bool(torch.allclose(act(_SILU_PROBE.clone()), nn.functional.silu(_SILU_PROBE),
                                            rtol=1e-6, atol=1e-7))
        except Exception:
            known = False
        try:
            object.__setattr__(act, "_stratum_is_silu", known)
        except (AttributeError, TypeError):
            pass
    return known


def _nf4_stack(module: nn.Module, names: _MlpProjectionNames, x: torch.Tensor) -> Optional[NF4StackedMLP]:
    """The NF4 row engine for *module* and input *x*, or None when it does not apply."""
    gate, up, down = (getattr(module, n) for n in names)
    if not all(isinstance(p, NF4Linear) for p in (gate, up, down)) or not _is_silu(module.act_fn):
        return None
    if not (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)):
        return None
    if any(p.quantized.device != x.device for p in (gate, up, down)):
        return None
    inter, hidden = (int(s) for s in gate.quant_state.shape)
    if x.shape[-1] != hidden or not NF4StackedMLP.supported(hidden, inter, gate.quant_state.blocksize):
        return None
    stack = getattr(module, _STACK_ATTR, None)
    if stack is None or not stack.matches(gate, up, down):
        stack = NF4StackedMLP(gate, up, down)
        object.__setattr__(module, _STACK_ATTR, stack)  # not a submodule, not state
    return stack


def _rows_engine(module: nn.Module, names: _MlpProjectionNames, x: torch.Tensor):
    return _nf4_stack(module, names, x) or _ModuleRows(module, names)


def _rows_per_chunk(hidden_states: torch.Tensor, token_chunk_size: int) -> int:
    """token_chunk_size tokens of every leading (batch) row."""
    lead = 1
    for d in hidden_states.shape[:-2]:
        lead *= int(d)
    return max(1, token_chunk_size * lead)


class MemoryFlatFrozenMLPFunction(torch.autograd.Function):
    """Chunked forward; the backward recomputes and differentiates one chunk at a
    time (``stratum/model/mlp_opt.py:154-215``)."""

    @staticmethod
    def forward(ctx: Any, hidden_states: torch.Tensor, module: nn.Module, token_chunk_size: int) -> torch.Tensor:
        names = _assert_frozen_mlp(module)
        if token_chunk_size <= 0:
            raise ValueError("token_chunk_size must be positive")
        if hidden_states.dim() < 3:
            raise ValueError("memory-flat frozen MLP expects [batch, seq, hidden] input")
        engine = _rows_engine(module, names, hidden_states)
        rows = _rows_per_chunk(hidden_states, token_chunk_size)
        x = hidden_states.reshape(-1, hidden_states.shape[-1]).contiguous()
        out_features = getattr(module, names.down).out_features
        out = x.new_empty(x.shape[0], out_features)
        engine.forward_rows(x, out, rows)
        ctx.engine, ctx.rows = engine, rows
        ctx.save_for_backward(hidden_states)
        return out.reshape(*hidden_states.shape[:-1], out_features)

    @staticmethod
    def backward(ctx: Any, grad_output: torch.Tensor):
        if not ctx.needs_input_grad[0]:
            return None, None, None
        (hidden_states,) = ctx.saved_tensors
        x = hidden_states.reshape(-1, hidden_states.shape[-1]).contiguous()
        dy = grad_output.reshape(x.shape[0], -1).contiguous()
        dx = torch.empty_like(x)
        ctx.engine.input_grad_rows(x, dy, dx, ctx.rows)
        return dx.reshape(hidden_states.shape), None, None


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
            # nothing to save for a backward and one chunk: the NF4 engine in one
            # pass, or the module itself
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
    """Replace the dense gate/up/down ``nn.Linear`` of *module* with NF4Linear
    (quantized on the GPU, packed weights resident on *device*), in place.

    Gate and up are quantized together as one ``[2 I, H]`` weight (NF4 rows are
    independent and a block never straddles a row when H is a multiple of the
    blocksize, so the bytes equal two separate quantizations); the two
    NF4Linear hold views of that one payload, which the fused MLP path uses
    without copying."""
    names = _mlp_projection_names(module)
    gate, up = getattr(module, names.gate), getattr(module, names.up)
    for name in names:
        lin = getattr(module, name)
        if not isinstance(lin, (nn.Linear, NF4Linear)) or (isinstance(lin, nn.Linear) and lin.bias is not None):
            raise TypeError(f"{name} must be a bias-free nn.Linear")

    def target(w: torch.Tensor) -> torch.device:
        return torch.device(device) if device is not None else (w.device if w.is_cuda else torch.device("cuda"))

    if (type(gate) is nn.Linear and type(up) is nn.Linear and gate.weight.shape == up.weight.shape
            and gate.weight.shape[1] % blocksize == 0):
        inter, hidden = gate.weight.shape
        dev = target(gate.weight)
        stacked = torch.cat([gate.weight.detach().to(dev), up.weight.detach().to(dev)])
        packed, state = quantize_4bit(stacked, blocksize=blocksize)
        half_q, half_a = inter * hidden // 2, inter * hidden // blocksize
        for name, sl_q, sl_a in ((names.gate, slice(0, half_q), slice(0, half_a)),
                                 (names.up, slice(half_q, 2 * half_q), slice(half_a, 2 * half_a))):
            st = QuantState(absmax=state.absmax[sl_a], shape=(inter, hidden), code=state.code,
                            blocksize=blocksize, quant_type=state.quant_type, dtype=state.dtype)
            setattr(module, name, NF4Linear(packed[sl_q], st))
    for name in names:
        lin = getattr(module, name)
        if isinstance(lin, NF4Linear):
            continue
        packed, state = quantize_4bit(lin.weight.detach().to(target(lin.weight)), blocksize=blocksize)
        setattr(module, name, NF4Linear(packed, state))
    return module
