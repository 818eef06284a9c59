"""Chunked linear cross-entropy over an NF4 (or dense) language-model head.

Same call as the reference's ``chunked_linear_cross_entropy``
(``stratum/model/chunked_loss.py:151-192``): token rows are split into chunks,
each chunk's logits and summed cross-entropy are computed and differentiated
at once inside the forward, only the input gradients are kept, and the outer
backward scales them by the incoming gradient -- so no ``[tokens, vocab]``
logits graph stays alive. The loss is normalised by the number of tokens whose
label is not ``ignore_index``.

The reference reads ``lm_head.weight`` and runs ``F.linear`` on it, so its
head must be dense on the device (materialised by ``ensure_weights``). Here
the head may also be an :class:`~stratum_amd.nf4_linear.NF4Linear` (or
``NF4LoRALinear``) holding the packed weight:

* chunks of at most ``fused_max_rows()`` rows run the fused dequant-GEMM
  kernels for the logits and for the hidden-state gradient -- the vocab x
  hidden weight is never dequantized;
* larger chunks share one dequantized temporary for the whole call (one
  dequantization per loss, as the reference's staged head has one per step),
  freed on return.

A LoRA adapter on an NF4 head gets its gradients (scaled like the rest); the
NF4 base weight is frozen and has none. A dense ``nn.Linear`` head behaves as
in the reference, weight and bias gradients included.
"""

from __future__ import annotations

from contextlib import contextmanager, nullcontext
from typing import Any, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .nf4_linear import NF4Linear, fused_max_rows
from .functional import fused_supported

__all__ = ["chunked_linear_cross_entropy", "ChunkedLinearCrossEntropyFunction"]


@contextmanager
def _default_stream_of(t: torch.Tensor):
    """Run the block on the device's default stream, as the reference computes
    the chunks there; when the caller's stream is another one, the default
    stream first waits for it (the hidden states were made there) and the
    caller's stream waits for the block's work afterwards."""
    if not (isinstance(t, torch.Tensor) and t.is_cuda):
        yield
        return
    caller = torch.cuda.current_stream(t.device)
    dflt = torch.cuda.default_stream(t.device)
    if caller != dflt:
        dflt.wait_stream(caller)
    with torch.cuda.stream(dflt):
        yield
    if caller != dflt:
        caller.wait_stream(dflt)


def _trainables(head: nn.Module) -> list:
    """The head's parameters that take a gradient, in a fixed order."""
    return [p for _, p in sorted(head.named_parameters(), key=lambda kv: kv[0]) if p.requires_grad]


def _chunk_loss_and_grads(head: nn.Module, h: torch.Tensor, labels: torch.Tensor, ignore_index: int,
                          want_h: bool, params: list) -> tuple:
    """Summed cross-entropy of one chunk and its gradients w.r.t. the chunk's
    hidden rows (if wanted) and *params*."""
    h = h.detach().requires_grad_(want_h)
    logits = head(h)
    loss = F.cross_entropy(logits.float(), labels, ignore_index=ignore_index, reduction="sum")
    inputs = ([h] if want_h else []) + params
    grads = torch.autograd.grad(loss, inputs) if inputs and loss.requires_grad else [None] * len(inputs)
    return loss.detach(), grads


class ChunkedLinearCrossEntropyFunction(torch.autograd.Function):
    """Summed chunked cross-entropy of ``head(hidden)``; saves the gradients of
    the hidden states and of the head's trainable parameters, not the logits.

    Arguments after ``ctx``: hidden ``[..., H]``, labels, the head module,
    ignore_index, token_chunk_size, whether gradients are wanted, then the
    head's trainable parameters (so autograd routes their gradients)."""

    @staticmethod
    def forward(ctx: Any, hidden: torch.Tensor, labels: torch.Tensor, head: nn.Module, ignore_index: int,
                token_chunk_size: int, want_grad: bool, *params: torch.Tensor) -> torch.Tensor:
        if token_chunk_size <= 0:
            raise ValueError(f"token_chunk_size must be > 0, got {token_chunk_size}")
        flat = hidden.reshape(-1, hidden.shape[-1])
        flat_labels = labels.reshape(-1).to(flat.device)
        want_h = want_grad and ctx.needs_input_grad[0]
        want_p = [want_grad and ctx.needs_input_grad[6 + i] for i in range(len(params))]
        grad_params = [p for p, w in zip(params, want_p) if w]
        g_h = torch.zeros_like(flat) if want_h else None
        g_p = [torch.zeros_like(p) for p in grad_params]
        total = flat.new_zeros((), dtype=torch.float32)

        hold = nullcontext()
        if isinstance(head, NF4Linear) and flat.is_cuda:
            rows = min(token_chunk_size, flat.shape[0])
            N, K = (int(s) for s in head.quant_state.shape)
            limit = fused_max_rows(lora=getattr(head, "r", 0) > 0)
            fused = fused_supported(N, K, head.quant_state.blocksize, backward=True) and (limit < 0 or rows <= limit)
            if not fused:  # one dequantized temporary for every chunk of this call
                hold = head.dense_weight(dtype=flat.dtype)
        grad_mode = torch.enable_grad() if want_grad else torch.no_grad()
        with _default_stream_of(flat), hold, grad_mode:
            for start in range(0, flat.shape[0], token_chunk_size):
                stop = min(start + token_chunk_size, flat.shape[0])
                loss, grads = _chunk_loss_and_grads(head, flat[start:stop], flat_labels[start:stop], ignore_index,
                                                    want_h, grad_params)
                total = total + loss
                if want_h:
                    g_h[start:stop] = grads[0]
                    grads = grads[1:]
                for acc, g in zip(g_p, grads):
                    if g is not None:
                        acc += g
        ctx.hidden_shape = tuple(hidden.shape)
        ctx.want_p = want_p
        ctx.save_for_backward(*(([g_h] if want_h else []) + g_p))
        ctx.want_h = want_h
        return total

    @staticmethod
    def backward(ctx: Any, grad_loss: torch.Tensor):
        saved = list(ctx.saved_tensors)
        d_hidden = saved.pop(0).mul(grad_loss).reshape(ctx.hidden_shape) if ctx.want_h else None
        d_params = []
        for w in ctx.want_p:
            d_params.append(saved.pop(0).mul(grad_loss) if w else None)
        return (d_hidden, None, None, None, None, None, *d_params)


def chunked_linear_cross_entropy(hidden_states: torch.Tensor, lm_head: nn.Module, labels: torch.Tensor, *,
                                 num_items: Optional[torch.Tensor] = None, ignore_index: int = -100,
                                 token_chunk_size: int = 4096, use_torch_compile: bool = False) -> torch.Tensor:
    """Token-normalised cross-entropy of ``lm_head(hidden_states)`` against
    *labels* (same shape as ``hidden_states.shape[:-1]``), computed in chunks
    of ``token_chunk_size`` rows (reference: ``stratum/model/chunked_loss.py:151-192``).

    ``lm_head``: an ``nn.Linear`` or an ``NF4Linear`` / ``NF4LoRALinear``.
    ``num_items``: the count of non-ignored labels (computed when omitted).
    ``use_torch_compile`` is accepted for the reference's signature; the chunks
    here run eagerly (the NF4 kernels are already fused)."""
    del use_torch_compile
    flat_labels = labels.reshape(-1)
    if num_items is None:
        num_items = (flat_labels != ignore_index).sum()
    num_items = num_items.to(hidden_states.device)
    if int(num_items.detach().cpu().item()) == 0:
        return hidden_states.sum() * 0.0
    params = _trainables(lm_head)
    loss_sum = ChunkedLinearCrossEntropyFunction.apply(hidden_states, labels, lm_head, ignore_index,
                                                       token_chunk_size, torch.is_grad_enabled(), *params)
    return loss_sum / num_items
