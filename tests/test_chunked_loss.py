"""Chunked linear cross-entropy on the CPU with a dense head: loss and every
gradient equal regular (unchunked) linear + cross-entropy -- the reference's
own checks (``tests/test_chunked_loss.py`` of the reference), restated."""

import pytest
import torch
import torch.nn as nn

from stratum_amd.chunked_loss import chunked_linear_cross_entropy


def _regular(hidden, weight, bias, labels, ignore_index=-100):
    logits = nn.functional.linear(hidden, weight, bias)
    n = (labels != ignore_index).sum()
    return nn.functional.cross_entropy(logits.reshape(-1, weight.shape[0]), labels.reshape(-1),
                                       ignore_index=ignore_index, reduction="sum") / n


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("chunk", [1, 3, 4096])
def test_matches_regular_linear_cross_entropy(bias, chunk):
    torch.manual_seed(7)
    B, T, H, V = 2, 5, 4, 9
    h0 = torch.randn(B, T, H)
    head = nn.Linear(H, V, bias=bias)
    labels = torch.randint(0, V, (B, T))
    labels[0, 1] = -100
    ref_h = h0.clone().requires_grad_(True)
    ref_w = head.weight.detach().clone().requires_grad_(True)
    ref_b = head.bias.detach().clone().requires_grad_(True) if bias else None
    ref = _regular(ref_h, ref_w, ref_b, labels)
    ref.backward()
    h = h0.clone().requires_grad_(True)
    loss = chunked_linear_cross_entropy(h, head, labels, token_chunk_size=chunk)
    loss.backward()
    torch.testing.assert_close(loss, ref, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(h.grad, ref_h.grad, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(head.weight.grad, ref_w.grad, atol=1e-6, rtol=1e-6)
    if bias:
        torch.testing.assert_close(head.bias.grad, ref_b.grad, atol=1e-6, rtol=1e-6)


def test_scaled_outer_gradient_and_frozen_head():
    """The outer backward's gradient scales the saved ones; a frozen head gets none."""
    torch.manual_seed(3)
    h0 = torch.randn(7, 6)
    head = nn.Linear(6, 11, bias=False).requires_grad_(False)
    labels = torch.randint(0, 11, (7,))
    ref_h = h0.clone().requires_grad_(True)
    (3.0 * _regular(ref_h, head.weight, None, labels)).backward()
    h = h0.clone().requires_grad_(True)
    (3.0 * chunked_linear_cross_entropy(h, head, labels, token_chunk_size=2)).backward()
    torch.testing.assert_close(h.grad, ref_h.grad, atol=1e-6, rtol=1e-6)
    assert head.weight.grad is None


def test_all_ignored_labels_returns_zero_loss():
    h = torch.randn(2, 3, 4, requires_grad=True)
    head = nn.Linear(4, 5)
    loss = chunked_linear_cross_entropy(h, head, torch.full((2, 3), -100))
    loss.backward()
    assert loss.item() == 0.0 and torch.equal(h.grad, torch.zeros_like(h)) and head.weight.grad is None


def test_no_grad_and_bad_chunk():
    head = nn.Linear(4, 5)
    labels = torch.randint(0, 5, (6,))
    with torch.no_grad():
        loss = chunked_linear_cross_entropy(torch.randn(6, 4), head, labels, token_chunk_size=4)
    assert loss.requires_grad is False and torch.isfinite(loss)
    with pytest.raises(ValueError, match="token_chunk_size"):
        chunked_linear_cross_entropy(torch.randn(6, 4), head, labels, token_chunk_size=0)
