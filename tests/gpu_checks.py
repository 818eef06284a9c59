"""Shared result checks of the GPU parity tests.

The GEMM bar is a relative Frobenius error against an fp32 matmul of the
oracle-dequantized weight (1e-2 bf16, 5e-3 fp16). Over a whole large output
that norm can hide a localized mistake: one wrong 32 x 256 strip of an
8192 x 14336 result moves it by only sqrt(8192 / 117.4 M) ~ 0.008. So the
check also holds every 32 x 32 fragment (the MFMA output tile) to the same
bar on its own.
"""

from __future__ import annotations

import torch

TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-3}


def fragment_errors(y: torch.Tensor, ref: torch.Tensor, frag: int = 32) -> torch.Tensor:
    """Relative Frobenius error of every frag x frag block of a 2-D result
    (edge blocks cover what is left); fp32, on the inputs' device."""
    assert y.shape == ref.shape and y.dim() == 2, (tuple(y.shape), tuple(ref.shape))
    M, N = ref.shape
    Mp, Np = -(-M // frag) * frag, -(-N // frag) * frag
    d = torch.zeros(Mp, Np, device=ref.device)
    r = torch.zeros(Mp, Np, device=ref.device)
    d[:M, :N] = y.float() - ref
    r[:M, :N] = ref
    dn = d.view(Mp // frag, frag, Np // frag, frag).square().sum((1, 3))
    rn = r.view(Mp // frag, frag, Np // frag, frag).square().sum((1, 3))
    return (dn / rn.clamp_min(1e-30)).sqrt()


def assert_gemm_close(y: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype, what: str = "") -> float:
    """Whole-matrix and per-32x32-fragment relative error within the dtype's
    tolerance; returns the whole-matrix error."""
    tol = TOL[dtype]
    y2 = y.reshape(-1, y.shape[-1])
    r2 = ref.reshape(-1, ref.shape[-1])
    whole = ((y2.float() - r2).norm() / r2.norm()).item()
    assert whole <= tol, f"{what}: relative error {whole:.3e} > {tol}"
    if y2.numel():
        fe = fragment_errors(y2, r2)
        worst = int(fe.argmax())
        fmax = fe.view(-1)[worst].item()
        fi, fj = divmod(worst, fe.shape[1])
        assert fmax <= tol, (f"{what}: fragment rows [{32 * fi}, {32 * fi + 32}) x cols [{32 * fj}, {32 * fj + 32}) "
                             f"relative error {fmax:.3e} > {tol}")
    return whole
