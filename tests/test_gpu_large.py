"""Sizes past 32-bit offsets.

The register-weight GEMM kernels address with 32-bit offsets from uniform
bases, and the planner hands larger problems to the LDS-weight kernels, whose
addresses are 64-bit; the (de)quantize kernels index with 64-bit element and
block numbers. These tests put outputs past 2^32 bytes (GEMMs) and tensors
past 2^32 elements ((de)quantize) on the GPU and check slices at the start,
around 2^31 and past 2^32 against the oracle / an fp32 reference.
"""

import numpy as np
import pytest
import torch

from gpu_checks import assert_gemm_close
from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _release_memory():
    """Each test holds several GB; give them back to the device afterwards."""
    yield
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def _weight(shape, seed):
    """Packed codes and absmax of a seeded fp16 N(0, 0.02) weight (oracle) and its
    oracle dequantization in bf16, as fp32."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(*shape, generator=g) * 0.02).half()
    rp, ra = C.quantize(w.view(torch.int16).numpy().view(np.uint16), O.DT_F16, 64, "argmin")
    n = int(np.prod(shape))
    deq = C.dequantize(rp, ra, n, 64, O.DT_BF16).view(np.int16).reshape(shape)
    return torch.from_numpy(rp), torch.from_numpy(ra), torch.from_numpy(deq).view(torch.bfloat16).float()


# rows whose output bytes start at 0, straddle 2^31 and lie past 2^32 (32768 columns
# of bf16 = 64 KiB per row: row 32768 starts at 2^31 bytes, row 65536 at 2^32)
ROWS = 65536 + 256
SLICES = [slice(0, 256), slice(32768 - 128, 32768 + 128), slice(65536, ROWS)]


def test_forward_output_past_4_gib(cuda):
    from stratum_amd.functional import nf4_gemm_fwd
    N, K = 32768, 64
    rp, ra, wq = _weight((N, K), 51)
    g = torch.Generator(device=cuda).manual_seed(52)
    x = torch.randn(ROWS, K, generator=g, device=cuda).bfloat16()
    y = nf4_gemm_fwd(x, rp.to(cuda), ra.to(cuda), (N, K), 64)
    assert y.shape == (ROWS, N) and y.numel() * 2 > 2 ** 32
    wt = wq.to(cuda).t().contiguous()
    for s in SLICES:
        assert_gemm_close(y[s], x[s].float() @ wt, torch.bfloat16, f"forward rows {s.start}:{s.stop}")


def test_input_gradient_output_past_4_gib(cuda):
    from stratum_amd.functional import nf4_gemm_bwd_dx
    N, K = 64, 32768
    rp, ra, wq = _weight((N, K), 53)
    g = torch.Generator(device=cuda).manual_seed(54)
    dy = torch.randn(ROWS, N, generator=g, device=cuda).bfloat16()
    dx = nf4_gemm_bwd_dx(dy, rp.to(cuda), ra.to(cuda), (N, K), 64)
    assert dx.shape == (ROWS, K) and dx.numel() * 2 > 2 ** 32
    w = wq.to(cuda)
    for s in SLICES:
        assert_gemm_close(dx[s], dy[s].float() @ w, torch.bfloat16, f"input gradient rows {s.start}:{s.stop}")


def test_quantize_and_dequantize_past_2_to_the_32_elements(cuda):
    """A [65537, 65536] fp16 weight (2^32 + 2^16 elements): packed codes, absmax
    and the bf16 dequantization bit-exact against the oracle on blocks at the
    start, around element 2^31 and past element 2^32."""
    from stratum_amd.functional import dequantize_4bit, quantize_4bit
    rows, cols = 65537, 65536
    g = torch.Generator(device=cuda).manual_seed(55)
    w = (torch.randn(rows, cols, generator=g, device=cuda, dtype=torch.float16) * 0.02)
    packed, st = quantize_4bit(w)
    n = rows * cols
    assert n > 2 ** 32 and packed.numel() == n // 2 and st.absmax.numel() == n // 64
    flat = w.view(-1)
    blocks = [(0, 1024), (2 ** 25 - 512, 2 ** 25 + 512), (n // 64 - 1024, n // 64)]  # element 2^31 = block 2^25
    refs = []
    for b0, b1 in blocks:
        src = flat[b0 * 64:b1 * 64].cpu().view(torch.int16).numpy().view(np.uint16)
        rp, ra = C.quantize(src, O.DT_F16, 64, "argmin")
        assert np.array_equal(packed.view(-1)[b0 * 32:b1 * 32].cpu().numpy(), rp), f"codes of blocks {b0}:{b1}"
        assert np.array_equal(st.absmax[b0:b1].cpu().numpy().view(np.uint32), ra.view(np.uint32)), \
            f"absmax of blocks {b0}:{b1}"
        refs.append(C.dequantize(rp, ra, (b1 - b0) * 64, 64, O.DT_BF16))
    del w, flat
    torch.cuda.empty_cache()
    out = dequantize_4bit(packed, st, dtype=torch.bfloat16).view(-1)
    for (b0, b1), ref in zip(blocks, refs):
        got = out[b0 * 64:b1 * 64].cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, ref), f"dequantized blocks {b0}:{b1}"
