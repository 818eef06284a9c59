"""The allocation-free forward entry point (stm_nf4_gemm_fwd_noalloc) against
the workspace entry point (stm_nf4_gemm_fwd) through the C ABI: two calls in a
row, the second smaller, each equal to the workspace result (same kernels, same
split plan) and within the bf16/fp16 bar of an fp32 matmul on the oracle
weight; and a problem too large for the static scratch is refused."""

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


def ptr(t):
    return t.data_ptr() if t is not None else None


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_forward_matches_the_workspace_forward_on_two_calls(cuda, dtype):
    from stratum_amd import _lib
    from stratum_amd.functional import _gemm_dtype
    L = _lib.lib()
    N, K, R = 4096, 2048, 16
    w = seeded((N, K), 31, 0.02, torch.float16)
    rp, ra = C.quantize(w.view(torch.int16).numpy().view(np.uint16), O.DT_F16, 64, "argmin")
    wq = torch.from_numpy(C.dequantize(rp, ra, N * K, 64, TAG[dtype]).view(np.int16).reshape(N, K)).view(dtype)
    wq = wq.to(cuda).float()
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    stream = _lib.stream_handle(cuda)
    for call, M in enumerate((32, 7)):  # the second call is smaller
        need = L.stm_nf4_gemm_workspace_bytes(M, N, K, 0)
        assert 0 < need <= 16 << 20, need  # a split problem: it uses the static scratch
        x = seeded((M, K), 40 + call, 1.0, dtype).to(cuda)
        bias = seeded((N,), 50 + call, 0.1, dtype).to(cuda)
        t = seeded((M, R), 60 + call, 0.5, dtype).to(cuda)
        lb = seeded((N, R), 70 + call, 0.01, dtype).to(cuda)
        ws = torch.empty(need // 4, dtype=torch.float32, device=cuda)
        y_ws = torch.empty(M, N, dtype=dtype, device=cuda)
        y = torch.full((M, N), 7.0, dtype=dtype, device=cuda)
        rc = L.stm_nf4_gemm_fwd(ptr(x), ptr(q), ptr(a), ptr(bias), ptr(t), ptr(lb), R, ptr(y_ws), M, N, K, 64,
                                _gemm_dtype(x), ptr(ws), need, stream)
        assert rc == 0, L.stm_last_error()
        rc = L.stm_nf4_gemm_fwd_noalloc(ptr(x), ptr(q), ptr(a), ptr(bias), ptr(t), ptr(lb), R, ptr(y), M, N, K, 64,
                                        _gemm_dtype(x), stream)
        assert rc == 0, L.stm_last_error()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ws), f"call {call}: the static-scratch result differs from the workspace result"
        ref = x.float() @ wq.t().contiguous() + bias.float() + t.float() @ lb.float().t().contiguous()
        assert_gemm_close(y, ref, dtype, f"noalloc call {call}")
    # an unsplit problem (no scratch needed) also runs
    M = 4096
    assert L.stm_nf4_gemm_workspace_bytes(M, N, K, 0) == 0
    x = seeded((M, K), 80, 1.0, dtype).to(cuda)
    y = torch.empty(M, N, dtype=dtype, device=cuda)
    rc = L.stm_nf4_gemm_fwd_noalloc(ptr(x), ptr(q), ptr(a), None, None, None, 0, ptr(y), M, N, K, 64,
                                    _gemm_dtype(x), stream)
    assert rc == 0, L.stm_last_error()
    assert_gemm_close(y, x.float() @ wq.t().contiguous(), dtype, "noalloc unsplit")


def test_noalloc_forward_refuses_problems_beyond_the_scratch(cuda):
    from stratum_amd import _lib
    L = _lib.lib()
    M, N, K = 512, 4096, 14336
    assert L.stm_nf4_gemm_workspace_bytes(M, N, K, 0) > 16 << 20
    buf = torch.empty(64, dtype=torch.uint8, device=cuda)
    rc = L.stm_nf4_gemm_fwd_noalloc(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), None, None, None, 0,
                                    buf.data_ptr(), M, N, K, 64, _lib.STM_BF16, _lib.stream_handle(cuda))
    assert rc == _lib.STM_ERR_UNSUPPORTED and b"static scratch" in L.stm_last_error()
