"""NF4Linear: frozen Linear whose weight stays NF4-packed on the GPU.

Mirrors ``stratum/nf4_linear.py:17-47`` (same constructor, ``in_features`` /
``out_features`` from ``quant_state.shape``). The reference dequantizes the
whole weight to a temporary fp16 tensor and calls ``F.linear``
(``stratum/nf4_linear.py:46-47``). Here each call picks the faster of two GPU
paths for its row count M (tokens), measured on MI355X:

* M <= ``fused_max_rows()`` (default 768; 1024 with a LoRA adapter): one
  fused dequant-GEMM forward and one fused dequant-GEMM for ``dX = dY . W``;
  the dequantized weight never exists in HBM, and the packed weight (0.56 B/element) is all the weight
  traffic -- forward plus input gradient, the fused kernels are faster there
  (at M = 768 on the 8B-class weights: 0.22 against 0.25 ms);
* larger M: ``dequantize_4bit`` into a temporary, then the library GEMM
  (hipBLASLt), whose forward is 1.2-1.3x faster than the fused kernel at
  M = 2048..8192, because the dequantization is paid once for all rows instead
  of once per 256-row tile. When the call records a graph for the input
  gradient (a recompute pass, or a plain training forward), the temporary is
  kept for the backward, as the reference keeps ``param.data`` from its
  recompute to its backward: the pipeline's forward, recompute and backward
  then dequantize twice per step, as the reference does
  (``stratum/pipeline.py:906``). ``NF4Linear.keep_weight_for_backward = False``
  trades that for memory (the backward dequantizes again).

``NF4LoRALinear`` adds the PEFT-style LoRA update (``scripts/train.py:568-573``:
r=16, alpha=16), folded into the fused kernels' epilogues on the first path.
Shapes the fused kernels do not take (K not a multiple of 64, ...) and dtypes
other than bf16/fp16 always take the second path. ``STRATUM_NF4_FUSED_MAX_ROWS``
overrides the threshold (``-1``: always fused where the shape allows, ``0``:
never).
"""

from __future__ import annotations

import math
from contextlib import contextmanager
from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

import os

from .functional import (QuantState, dequantize_4bit, fused_supported, lora_da, lora_down, lora_dy, lora_supported,
                         nf4_gemm_bwd_dx, nf4_gemm_fwd)

_DEFAULT_FUSED_MAX_ROWS = 768
# With a LoRA adapter the fused kernels fold the rank-R terms into their
# epilogues, while the library path pays extra passes over Y and dX for them, so
# the crossover sits higher: forward + backward on the 8B-class weights at
# M = 1024, 0.30-0.32 ms fused against 0.33 ms; even at 1536-2048 rows;
# library ahead from 4096 rows (8192: 1.81 against 1.70 ms).
_DEFAULT_FUSED_MAX_ROWS_LORA = 1024


def fused_max_rows(lora: bool = False) -> int:
    """Largest row count (tokens) sent to the fused kernels; -1 = no limit.
    ``STRATUM_NF4_FUSED_MAX_ROWS`` overrides both defaults."""
    v = os.environ.get("STRATUM_NF4_FUSED_MAX_ROWS")
    if v not in (None, ""):
        return int(v)
    return _DEFAULT_FUSED_MAX_ROWS_LORA if lora else _DEFAULT_FUSED_MAX_ROWS


def _mm_scaled(a: torch.Tensor, b: torch.Tensor, scaling: float) -> torch.Tensor:
    """scaling * (a @ b) with the factor applied in the GEMM's epilogue (no
    separate elementwise pass; none at all for scaling == 1)."""
    if scaling == 1.0:
        return a @ b
    return torch.addmm(a.new_empty(()), a, b, beta=0, alpha=scaling)  # beta = 0: the input is never read


class _NF4LinearFn(torch.autograd.Function):
    """y = x . W^T (+ bias) (+ scaling * (x . A^T) . B^T) with W frozen in NF4."""

    @staticmethod
    def forward(ctx, x, packed, absmax, shape, blocksize, bias, lora_a, lora_b, scaling, fused, w_dense=None,
                keep_w=True):
        t = None
        if lora_a is not None:
            if lora_supported(lora_a.shape[0], x.shape[-1], x.numel() // max(x.shape[-1], 1)):
                t = lora_down(x, lora_a, scaling)
            else:
                t = _mm_scaled(x.reshape(-1, x.shape[-1]), lora_a.t().to(x.dtype), scaling)
        if fused:
            y = nf4_gemm_fwd(x, packed, absmax, shape, blocksize, bias=bias, lora_t=t,
                             lora_b=lora_b.to(x.dtype) if lora_b is not None else None)
        else:
            if w_dense is not None and w_dense.dtype == x.dtype:
                w = w_dense
            else:
                w = dequantize_4bit(packed, absmax=absmax, blocksize=blocksize, dtype=x.dtype, shape=shape)
            b = bias.to(x.dtype) if bias is not None else None
            if t is not None:
                # rank-R term (and bias) first, then the base GEMM accumulates into it
                # (beta = 1): no separate full-size add
                lb_t = lora_b.to(x.dtype).t()
                y2 = torch.addmm(b, t, lb_t) if b is not None else t @ lb_t
                y = y2.addmm_(x.reshape(-1, x.shape[-1]), w.t()).reshape(*x.shape[:-1], w.shape[0])
            else:
                y = F.linear(x, w, b)
            # needs_input_grad is all False when no graph is recorded (no_grad forward)
            ctx.w = w if keep_w and ctx.needs_input_grad[0] else None
            del w
        ctx.shape, ctx.blocksize, ctx.scaling, ctx.fused = shape, blocksize, scaling, fused
        ctx.has_bias_grad = bias is not None and bias.requires_grad
        ctx.save_for_backward(x if lora_a is not None else None, packed, absmax, lora_a, lora_b, t)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, packed, absmax, lora_a, lora_b, t = ctx.saved_tensors
        N, K = ctx.shape
        dy2 = dy.reshape(-1, N).contiguous()
        u = d_b = None
        if lora_a is not None:
            if lora_supported(lora_a.shape[0], N, dy2.shape[0]):
                # one pass over dY for U and (when B trains) dB
                u, d_b = lora_dy(dy2, lora_b, t if ctx.needs_input_grad[7] else None, ctx.scaling)
            else:
                u = _mm_scaled(dy2, lora_b.to(dy2.dtype), ctx.scaling)      # [M, R]
                if ctx.needs_input_grad[7]:
                    d_b = dy2.t() @ t                                       # [N, R]
        dx = None
        if ctx.needs_input_grad[0]:
            if ctx.fused:
                dx = nf4_gemm_bwd_dx(dy2, packed, absmax, ctx.shape, ctx.blocksize, lora_u=u,
                                     lora_at=lora_a.t().contiguous().to(dy2.dtype) if lora_a is not None else None)
            else:
                w = ctx.w if ctx.w is not None and ctx.w.dtype == dy2.dtype else \
                    dequantize_4bit(packed, absmax=absmax, blocksize=ctx.blocksize, dtype=dy2.dtype, shape=ctx.shape)
                ctx.w = None
                if u is not None:
                    dx = (u @ lora_a.to(dy2.dtype)).addmm_(dy2, w)     # rank-R term, then the base GEMM into it
                else:
                    dx = dy2 @ w
                del w
            dx = dx.reshape(*dy.shape[:-1], K)
        d_bias = dy2.sum(0).to(dy.dtype) if ctx.has_bias_grad else None
        d_a = None
        if lora_a is not None:
            x2 = x.reshape(-1, K)
            if ctx.needs_input_grad[6]:
                d_a = lora_da(u, x2) if lora_supported(lora_a.shape[0], K, x2.shape[0]) else u.t() @ x2  # [R, K]
                d_a = d_a.to(lora_a.dtype)
            if d_b is not None:
                d_b = d_b.to(lora_b.dtype)
        ctx.w = None
        return dx, None, None, None, None, d_bias, d_a, d_b, None, None, None, None


def nf4_linear(x: torch.Tensor, quantized: torch.Tensor, quant_state: QuantState, bias: Optional[torch.Tensor] = None,
               lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
               scaling: float = 1.0, *, w_dense: Optional[torch.Tensor] = None,
               keep_weight_for_backward: bool = True) -> torch.Tensor:
    """``x . W^T (+ bias) (+ scaling * (x . A^T) . B^T)`` with W in NF4.

    ``w_dense``: an already dequantized W (same dtype as x) that the library
    path uses instead of dequantizing (``NF4Linear.dense_weight``); the fused
    path ignores it. ``keep_weight_for_backward``: see the module docstring."""
    shape = tuple(int(s) for s in quant_state.shape)
    N, K = shape
    bs = quant_state.blocksize
    rank = lora_a.shape[0] if lora_a is not None else 0
    if x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and rank % 16 == 0:
        rows = x.numel() // max(K, 1)
        limit = fused_max_rows(lora=rank > 0)
        fused = fused_supported(N, K, bs, backward=True) and (limit < 0 or rows <= limit)
        return _NF4LinearFn.apply(x, quantized, quant_state.absmax, shape, bs, bias, lora_a, lora_b, scaling, fused,
                                  w_dense, keep_weight_for_backward)
    # unfused GPU path: dequantize into a temporary, then the library GEMM
    w = w_dense if w_dense is not None and w_dense.dtype == x.dtype else dequantize_4bit(quantized, quant_state,
                                                                                         dtype=x.dtype)
    y = F.linear(x, w, bias.to(x.dtype) if bias is not None else None)
    if lora_a is not None:
        y = y + F.linear(F.linear(x, lora_a.to(x.dtype)), lora_b.to(x.dtype)) * scaling
    return y


class NF4Linear(nn.Module):
    """Frozen Linear layer with an NF4-compressed weight kept on the GPU.

    Same constructor as the reference (``stratum/nf4_linear.py:27-41``): the
    packed codes, their ``QuantState`` and an optional bias (stored frozen).

    ``weight`` (read-only) dequantizes the packed weight into a new dense
    tensor on every read, for code that reads ``module.weight`` directly (the
    reference's chunked loss reads ``lm_head.weight``,
    ``stratum/model/chunked_loss.py:184``); it costs a dequantization and 2
    bytes per weight while the tensor lives. ``dense_weight()`` holds one such
    tensor for a stretch of calls that all use it.
    """

    keep_weight_for_backward = True

    def __init__(self, quantized: torch.Tensor, quant_state: QuantState, bias: Optional[torch.Tensor] = None):
        super().__init__()
        self.quantized = quantized
        self.quant_state = quant_state
        if bias is not None:
            self.bias = nn.Parameter(bias.contiguous(), requires_grad=False)
        else:
            self.bias = None
        self.in_features = quant_state.shape[1]
        self.out_features = quant_state.shape[0]
        self._w_dense = None

    @property
    def weight(self) -> torch.Tensor:
        """The dequantized weight ``[out_features, in_features]`` in the
        payload's source dtype: a new tensor per read (see the class docstring)."""
        if self._w_dense is not None:
            return self._w_dense
        return dequantize_4bit(self.quantized, self.quant_state)

    @contextmanager
    def dense_weight(self, dtype: Optional[torch.dtype] = None):
        """Dequantize once and let every call inside the block that takes the
        library path (and ``weight``) use that tensor; freed on exit."""
        w = dequantize_4bit(self.quantized, self.quant_state, dtype=dtype or self.quant_state.dtype)
        prev, self._w_dense = self._w_dense, w
        try:
            yield w
        finally:
            self._w_dense = prev

    def _linear(self, x: torch.Tensor, lora_a=None, lora_b=None, scaling: float = 1.0) -> torch.Tensor:
        return nf4_linear(x, self.quantized, self.quant_state, self.bias, lora_a, lora_b, scaling,
                          w_dense=self._w_dense, keep_weight_for_backward=self.keep_weight_for_backward)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._linear(x)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, nf4 blocksize={self.quant_state.blocksize}"


class NF4LoRALinear(NF4Linear):
    """NF4Linear plus a trainable LoRA update ``scaling * B(A(x))`` (PEFT's
    ``lora.Linear`` with r, alpha; A ~ kaiming-uniform, B = 0 at init)."""

    def __init__(self, quantized: torch.Tensor, quant_state: QuantState, bias: Optional[torch.Tensor] = None, *,
                 r: int = 16, lora_alpha: float = 16.0, dtype: torch.dtype = torch.bfloat16):
        super().__init__(quantized, quant_state, bias)
        dev = quantized.device
        self.r = r
        self.scaling = lora_alpha / r
        self.lora_A = nn.Parameter(torch.empty(r, self.in_features, dtype=dtype, device=dev))
        self.lora_B = nn.Parameter(torch.zeros(self.out_features, r, dtype=dtype, device=dev))
        nn.init.kaiming_uniform_(self.lora_A, a=math.sqrt(5))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._linear(x, self.lora_A, self.lora_B, self.scaling)


@torch.no_grad()
def make_nf4_resident(module: nn.Module, device_id: int, *, lora_r: int = 0, lora_alpha: float = 16.0,
                      lora_dtype: torch.dtype = torch.bfloat16, exclude: Sequence[str] = ("lm_head",)) -> int:
    """Keep the staged NF4 weights of *module* packed on ``cuda:<device_id>``.

    Every ``nn.Linear`` inside *module* whose weight carries an NF4 payload
    (``prepare_nf4``) is replaced by an :class:`NF4Linear` -- or, with
    ``lora_r > 0``, an :class:`NF4LoRALinear` with fresh PEFT-style adapters --
    that holds the payload's packed codes and absmax on the device: 0.5625
    bytes per weight uploaded once, instead of the dequantized 2 bytes per
    weight materialised by ``ensure_weights`` before every forward and again
    before the recompute (``stratum/nf4_linear.py:1-8`` names this as the
    intended use; ``stratum/pipeline.py:906`` frees after the forward). The
    replacement keeps the payload (``.payload``) and the original bias; the
    staging calls (``ensure_weights`` / ``free_weights``) then find nothing to
    do for these layers. Layers whose attribute name is in ``exclude`` keep
    the staged lifecycle: by default ``lm_head``, whose ``.weight`` the
    reference's chunked loss reads directly (``stratum/model/chunked_loss.py:184``;
    ``chunked_linear_cross_entropy`` of this package takes a swapped head).
    Returns the number of layers replaced.
    """
    from .upload import NF4_ATTR  # local: upload imports this module's package

    device = torch.device("cuda", device_id)
    skip = set(exclude)
    replaced = 0
    for parent in list(module.modules()):
        for name, child in list(parent.named_children()):
            if name in skip or type(child) is not nn.Linear or not hasattr(child.weight, NF4_ATTR):
                continue
            payload = getattr(child.weight, NF4_ATTR)
            if len(payload.shape) != 2:
                continue
            state = QuantState(absmax=payload.absmax.to(device, non_blocking=True), shape=payload.shape,
                               code=payload.code.to(device, non_blocking=True), blocksize=payload.blocksize,
                               quant_type=payload.quant_type, dtype=payload.dtype)
            packed = payload.quantized.to(device, non_blocking=True)
            bias = child.bias.detach().to(device) if child.bias is not None else None
            if lora_r > 0:
                new = NF4LoRALinear(packed, state, bias, r=lora_r, lora_alpha=lora_alpha, dtype=lora_dtype)
            else:
                new = NF4Linear(packed, state, bias)
            new.payload = payload
            setattr(parent, name, new)
            replaced += 1
    return replaced
