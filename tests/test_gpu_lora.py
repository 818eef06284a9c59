"""LoRA side products (T = s X A^T, U = s dY B, dB = dY^T T, dA = U^T X) against
fp32 torch on the same inputs: relative error within the GEMM tolerance (1e-2
bf16, 5e-3 fp16), identical bits on a repeated call (fixed-order reduction),
ragged row and column counts, every supported rank, and empty problems."""

import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-3}
SHAPES = [
    (1, 8, 8),         # one row, one chunk of columns, rank 8 (padded to 16)
    (64, 256, 16),     # one step, one column block
    (65, 264, 16),     # one row past a step, 8 columns past a block
    (300, 520, 24),    # rank 24 (padded to 32), two column blocks + 8
    (130, 4104, 32),   # rank 32, 17 column blocks
    (2000, 4096, 16),  # several row blocks
    (513, 1000, 8),    # ragged in both directions
    (16, 4104, 32),    # decode size: lora_down's one-launch kernel, 8 columns past a 2048 sweep
    (40, 14336, 24),   # decode size, rank 24, long rows
]


def seeded(shape, seed, std, dtype, dev):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype).to(dev)


def rel(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,R", SHAPES)
def test_lora_down(cuda, dtype, M, K, R):
    from stratum_amd.functional import lora_down
    x = seeded((M, K), 1, 1.0, dtype, cuda)
    a = seeded((R, K), 2, 0.05, dtype, cuda)
    t = lora_down(x, a, 2.0)
    assert t.shape == (M, R) and t.dtype == dtype
    ref = 2.0 * (x.float() @ a.float().t().contiguous())
    assert rel(t, ref) <= TOL[dtype]
    assert torch.equal(t, lora_down(x, a, 2.0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,R", SHAPES)
def test_lora_dy(cuda, dtype, M, N, R):
    from stratum_amd.functional import lora_dy
    dy = seeded((M, N), 3, 1.0, dtype, cuda)
    b = seeded((N, R), 4, 0.05, dtype, cuda)
    t = seeded((M, R), 5, 1.0, dtype, cuda)
    u, db = lora_dy(dy, b, t, 0.5)
    assert u.shape == (M, R) and db.shape == (N, R)
    assert rel(u, 0.5 * (dy.float() @ b.float())) <= TOL[dtype]
    assert rel(db, dy.float().t().contiguous() @ t.float()) <= TOL[dtype]
    u2, db2 = lora_dy(dy, b, t, 0.5)
    assert torch.equal(u, u2) and torch.equal(db, db2)
    # without T only U is computed, with the same bits
    u3, none = lora_dy(dy, b, None, 0.5)
    assert none is None and torch.equal(u, u3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,R", SHAPES)
def test_lora_da(cuda, dtype, M, K, R):
    from stratum_amd.functional import lora_da
    u = seeded((M, R), 6, 1.0, dtype, cuda)
    x = seeded((M, K), 7, 1.0, dtype, cuda)
    da = lora_da(u, x)
    assert da.shape == (R, K)
    assert rel(da, u.float().t().contiguous() @ x.float()) <= TOL[dtype]
    assert torch.equal(da, lora_da(u, x))


def test_lora_at_the_lora_step_shape(cuda):
    """X [8192, 4096], dY [8192, 14336], rank 16: the products of one LoRA step."""
    from stratum_amd.functional import lora_da, lora_down, lora_dy
    dt = torch.bfloat16
    M, N, K, R = 8192, 14336, 4096, 16
    x = seeded((M, K), 8, 1.0, dt, cuda)
    dy = seeded((M, N), 9, 1.0, dt, cuda)
    a = seeded((R, K), 10, 0.01, dt, cuda)
    b = seeded((N, R), 11, 0.01, dt, cuda)
    t = lora_down(x, a, 1.0)
    assert rel(t, x.float() @ a.float().t().contiguous()) <= 1e-2
    u, db = lora_dy(dy, b, t, 1.0)
    assert rel(u, dy.float() @ b.float()) <= 1e-2
    assert rel(db, dy.float().t().contiguous() @ t.float()) <= 1e-2
    da = lora_da(u, x)
    assert rel(da, u.float().t().contiguous() @ x.float()) <= 1e-2


def test_lora_empty_problems(cuda):
    from stratum_amd.functional import lora_da, lora_down, lora_dy
    dt = torch.bfloat16
    x0 = torch.empty((0, 256), dtype=dt, device=cuda)
    a = seeded((16, 256), 12, 0.05, dt, cuda)
    assert lora_down(x0, a).shape == (0, 16)
    # no reduction (K = 0): zeros
    t = lora_down(torch.empty((5, 0), dtype=dt, device=cuda), torch.empty((16, 0), dtype=dt, device=cuda))
    assert t.shape == (5, 16) and not t.any()
    # no rows: U is empty, dB and dA are zero
    u, db = lora_dy(torch.empty((0, 64), dtype=dt, device=cuda), seeded((64, 16), 13, 0.05, dt, cuda),
                    torch.empty((0, 16), dtype=dt, device=cuda))
    assert u.shape == (0, 16) and db.shape == (64, 16) and not db.any()
    da = lora_da(torch.empty((0, 16), dtype=dt, device=cuda), x0)
    assert da.shape == (16, 256) and not da.any()


def test_lora_entry_points_replay_correctly_in_a_hip_graph(cuda):
    """T, U + dB and dA captured into one HIP graph: every replay, with eager
    LoRA work on other inputs and synchronisations between replays, matches the
    eager results bit for bit (the partial buffers are fully overwritten; no
    memset is recorded)."""
    from stratum_amd.functional import lora_da, lora_down, lora_dy
    dt = torch.bfloat16
    M, N, K, R = 300, 520, 264, 16
    x = seeded((M, K), 20, 1.0, dt, cuda)
    dy = seeded((M, N), 21, 1.0, dt, cuda)
    a = seeded((R, K), 22, 0.05, dt, cuda)
    b = seeded((N, R), 23, 0.05, dt, cuda)
    t_e = lora_down(x, a, 2.0)
    u_e, db_e = lora_dy(dy, b, t_e, 2.0)
    da_e = lora_da(u_e, x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lora_down(x, a, 2.0)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        t_g = lora_down(x, a, 2.0)
        u_g, db_g = lora_dy(dy, b, t_g, 2.0)
        da_g = lora_da(u_g, x)
    for i in range(3):
        junk = lora_dy(dy.flip(0), b, t_e, 0.5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(t_g, t_e), i
        assert torch.equal(u_g, u_e) and torch.equal(db_g, db_e), i
        assert torch.equal(da_g, da_e), i
        del junk
