"""The per-fragment GEMM check (tests/gpu_checks.py) on the CPU: it fails a
result with one wrong fragment that the whole-matrix norm lets through."""

import pytest
import torch

from gpu_checks import assert_gemm_close, fragment_errors


def _ref(M, N, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, N, generator=g)


def test_one_wrong_fragment_passes_the_whole_norm_but_not_the_fragment_check():
    ref = _ref(2048, 4096)
    y = ref.clone()
    y[32:64, 512:544] *= 1.05           # one 32 x 32 fragment off by 5 %
    whole = ((y - ref).norm() / ref.norm()).item()
    assert whole < 1e-2                 # hidden in the whole-matrix norm
    with pytest.raises(AssertionError, match=r"rows \[32, 64\) x cols \[512, 544\)"):
        assert_gemm_close(y.bfloat16(), ref, torch.bfloat16, "planted")


def test_rounding_only_passes_and_edges_are_covered():
    ref = _ref(1000, 520, 1)                     # ragged: edge fragments partly empty
    assert_gemm_close(ref.bfloat16(), ref, torch.bfloat16, "bf16 rounding")
    assert_gemm_close(ref.half(), ref, torch.float16, "fp16 rounding")
    fe = fragment_errors(ref.bfloat16(), ref)
    assert fe.shape == (32, 17)
    y = ref.clone()
    y[999, 519] += 1.0                           # last element of the last, partial fragment
    with pytest.raises(AssertionError, match=r"rows \[992, 1024\) x cols \[512, 544\)"):
        assert_gemm_close(y, ref, torch.bfloat16, "edge")
