"""GPU tests of the NF4 head and of resident layers at training row counts.

* Resident layers above the fused row threshold (2048 rows): the pipeline's
  forward (no graph), recompute and backward dequantize each weight at most
  twice per step, as the reference's staged lifecycle does
  (``stratum/pipeline.py:906``), and match the staged lifecycle.
* A staged postfix holding ``lm_head``: ``make_nf4_resident`` leaves the head
  staged, so the reference's loss (``F.linear(h, lm_head.weight)``,
  ``stratum/model/chunked_loss.py:31-44,184``) still finds a dense weight;
  ``NF4Linear.weight`` dequantizes bit-exactly when a swapped head is read.
* ``chunked_linear_cross_entropy`` over an NF4 head (fused chunks, and one
  dequantized temporary for larger chunks) against fp32 cross-entropy on the
  oracle weight: loss, hidden-state gradient and LoRA gradients.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from gpu_checks import assert_gemm_close
from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def oracle_weight(w16, dtype):
    """(packed, absmax, dequantized W in dtype) of the oracle for an fp16 weight."""
    bits = w16.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    rp, ra = C.quantize(bits, O.DT_F16, 64, "argmin")
    tag = {torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16}[dtype]
    deq = C.dequantize(rp, ra, w16.numel(), 64, tag).view(np.int16).reshape(tuple(w16.shape))
    return rp, ra, torch.from_numpy(deq).view(dtype)


def count_dequantize(monkeypatch):
    """Record every dequantize call into the library (single and batched)."""
    from stratum_amd import _lib
    calls = []
    for entry in ("stm_nf4_dequantize", "stm_nf4_dequantize_many"):
        real_entry = getattr(_lib.lib(), entry)

        def counting(*a, _real=real_entry, _name=entry):
            calls.append(_name)
            return _real(*a)
        monkeypatch.setattr(_lib.lib(), entry, counting)
    return calls


class _Block(nn.Module):
    def __init__(self, seed, hidden=512, inter=1024):
        super().__init__()
        self.up = nn.Linear(hidden, inter, bias=False, dtype=torch.float16)
        self.down = nn.Linear(inter, hidden, bias=False, dtype=torch.float16)
        with torch.no_grad():
            self.up.weight.copy_(seeded((inter, hidden), seed, 0.02, torch.float16))
            self.down.weight.copy_(seeded((hidden, inter), seed + 1, 0.02, torch.float16))
        self.requires_grad_(False)

    def forward(self, x):
        return x + self.down(torch.nn.functional.gelu(self.up(x)))


def _step(layers, x, dy, before, after):
    """The pipeline's step for a frozen stage: forward without a graph, free,
    recompute with a graph, backward, free."""
    with torch.no_grad():
        h = x
        for layer in layers:
            before(layer)
            h = layer(h)
            after(layer)
    out = h.clone()
    xg = x.detach().requires_grad_(True)
    h = xg
    for layer in layers:
        before(layer)
        h = layer(h)
    h.backward(dy)
    for layer in layers:
        after(layer)
    return out, xg.grad


def test_resident_layers_dequantize_at_most_twice_per_step_at_2048_rows(cuda, monkeypatch):
    import stratum_amd.upload as U
    from stratum_amd.nf4_linear import fused_max_rows, make_nf4_resident
    monkeypatch.delenv("STRATUM_NF4_FUSED_MAX_ROWS", raising=False)
    rows = 2048
    assert rows > fused_max_rows()  # the library path with a dequantized temporary
    x = seeded((rows, 512), 1, 1.0, torch.float16).to(cuda)
    dy = seeded((rows, 512), 2, 1.0, torch.float16).to(cuda)
    staged = nn.ModuleList([_Block(10), _Block(20)])
    U.prepare_nf4(staged, verbose=False)
    ref_out, ref_dx = _step(staged, x, dy, lambda l: U.ensure_weights(l, 0), U.free_weights)

    resident = nn.ModuleList([_Block(10), _Block(20)])
    U.prepare_nf4(resident, verbose=False)
    assert make_nf4_resident(resident, 0) == 4
    calls = count_dequantize(monkeypatch)
    out, dx = _step(resident, x, dy, lambda l: U.ensure_weights(l, 0), U.free_weights)
    torch.cuda.synchronize()
    # 4 weights: forward + recompute, the backward reuses the recompute's temporary
    assert len(calls) == 8, calls
    assert_gemm_close(out, ref_out.float(), torch.float16, "resident forward")
    assert_gemm_close(dx, ref_dx.float(), torch.float16, "resident input gradient")


class _Postfix(nn.Module):
    def __init__(self, hidden=512, vocab=4096):
        super().__init__()
        self.norm = nn.LayerNorm(hidden, dtype=torch.float16)
        self.lm_head = nn.Linear(hidden, vocab, bias=False, dtype=torch.float16)
        self.proj = nn.Linear(hidden, hidden, bias=False, dtype=torch.float16)
        with torch.no_grad():
            self.lm_head.weight.copy_(seeded((vocab, hidden), 7, 0.02, torch.float16))
            self.proj.weight.copy_(seeded((hidden, hidden), 8, 0.02, torch.float16))
        self.requires_grad_(False)


def test_staged_postfix_keeps_lm_head_for_the_reference_loss(cuda):
    """make_nf4_resident swaps proj but not lm_head; the reference's chunked
    loss reads lm_head.weight after ensure_weights: bit-exact to the oracle."""
    import stratum_amd.upload as U
    from stratum_amd.nf4_linear import NF4Linear, make_nf4_resident
    post = _Postfix()
    _, _, w_ref = oracle_weight(post.lm_head.weight.data, torch.float16)
    U.prepare_nf4(post, verbose=False)
    assert make_nf4_resident(post, 0) == 1
    assert isinstance(post.proj, NF4Linear) and type(post.lm_head) is nn.Linear
    U.ensure_weights(post, 0)
    h = seeded((300, 512), 3, 1.0, torch.float16).to(cuda)
    logits = nn.functional.linear(h, post.lm_head.weight)        # the reference's loss, chunked_loss.py:38
    assert torch.equal(post.lm_head.weight.cpu(), w_ref)
    assert_gemm_close(logits, h.float() @ w_ref.to(cuda).float().t().contiguous(), torch.float16, "lm_head")
    U.free_weights(post)
    assert post.lm_head.weight.numel() == 0


def test_nf4_linear_weight_property_is_the_oracle_dequantization(cuda):
    from stratum_amd.functional import QuantState
    from stratum_amd.nf4_linear import NF4Linear
    w16 = seeded((1024, 512), 5, 0.02, torch.float16)
    rp, ra, w_ref = oracle_weight(w16, torch.float16)
    st = QuantState(absmax=torch.from_numpy(ra).to(cuda), shape=(1024, 512), blocksize=64, dtype=torch.float16)
    lin = NF4Linear(torch.from_numpy(rp).to(cuda), st)
    assert torch.equal(lin.weight.cpu(), w_ref)
    with lin.dense_weight() as w:
        assert lin.weight is w and torch.equal(w.cpu(), w_ref)
    assert lin.weight is not w


def _nf4_head(cuda, vocab, hidden, lora):
    from stratum_amd.functional import QuantState
    from stratum_amd.nf4_linear import NF4Linear, NF4LoRALinear
    w16 = seeded((vocab, hidden), 21, 0.02, torch.float16)
    rp, ra, w_ref = oracle_weight(w16, torch.bfloat16)
    st = QuantState(absmax=torch.from_numpy(ra).to(cuda), shape=(vocab, hidden), blocksize=64, dtype=torch.bfloat16)
    q = torch.from_numpy(rp).to(cuda)
    if lora:
        head = NF4LoRALinear(q, st, r=16, lora_alpha=32.0)
        with torch.no_grad():
            head.lora_A.copy_(seeded((16, hidden), 22, 0.05, torch.bfloat16))
            head.lora_B.copy_(seeded((vocab, 16), 23, 0.05, torch.bfloat16))
    else:
        head = NF4Linear(q, st)
    return head, w_ref.to(cuda).float()


@pytest.mark.parametrize("lora", [False, True])
@pytest.mark.parametrize("chunk,dequants", [(512, 0), (1536, 1)])
def test_chunked_loss_over_an_nf4_head(cuda, monkeypatch, lora, chunk, dequants):
    """Loss and gradients of the chunked loss over an NF4 head against fp32
    cross-entropy on the oracle weight. Chunks of 512 rows run the fused
    kernels (no dequantization); 1536-row chunks share one dequantized
    temporary (one dequantization per call)."""
    from stratum_amd.chunked_loss import chunked_linear_cross_entropy
    monkeypatch.delenv("STRATUM_NF4_FUSED_MAX_ROWS", raising=False)
    T, H, V = 3000, 1024, 8192
    head, w = _nf4_head(cuda, V, H, lora)
    h0 = seeded((T, H), 24, 1.0, torch.bfloat16).to(cuda)
    labels = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(25)).to(cuda)
    labels[::7] = -100
    calls = count_dequantize(monkeypatch)
    h = h0.clone().requires_grad_(True)
    loss = chunked_linear_cross_entropy(h, head, labels, token_chunk_size=chunk)
    loss.backward()
    torch.cuda.synchronize()
    assert len(calls) == dequants, calls

    hr = h0.float().requires_grad_(True)
    logits = hr @ w.t().contiguous()
    if lora:
        Ar = head.lora_A.detach().float().requires_grad_(True)
        Br = head.lora_B.detach().float().requires_grad_(True)
        logits = logits + head.scaling * (hr @ Ar.t().contiguous()) @ Br.t().contiguous()
    ref = nn.functional.cross_entropy(logits, labels, ignore_index=-100, reduction="sum") / (labels != -100).sum()
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-2 * abs(ref.item()), (loss.item(), ref.item())
    assert_gemm_close(h.grad, hr.grad, torch.bfloat16, "hidden-state gradient")
    if lora:
        assert_gemm_close(head.lora_A.grad, Ar.grad, torch.bfloat16, "dA")
        assert_gemm_close(head.lora_B.grad, Br.grad, torch.bfloat16, "dB")
