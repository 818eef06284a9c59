"""Every GEMM kernel variant on the same ragged problems.

The library picks, per call, the 256 x 256 tile (register-weight kernels, or
LDS-weight kernels for some split reductions), the 128 x 256 register-weight
tile (unsplit) or the 128 x 128 LDS-weight tile, split or not, and for a
forward of at most 64 rows a weight-streaming small-M kernel: the split-free one
(its work-group's waves split the reduction and add bias and the LoRA term
themselves) where the rows fit and the launch fills the GPU, else the one whose
reduction ranges the split-reduce kernel sums (adding bias and the LoRA term).
stm_nf4_gemm_set_tile pins the tile kind (and so skips the small-M kernel) and
a call through the C ABI without a workspace pins "unsplit", so each kernel is
reached on shapes whose rows, output columns and reduction are not multiples
of the tile:
results within the fp32-reference tolerance (1e-2 bf16, 5e-3 fp16) and, for
the same problem, within rounding of each other.
"""

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-3}
TAG = {torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16}


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def rel(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def nf4(shape, seed, bs, dtype):
    """(packed, absmax) of a seeded fp16 weight and its oracle dequantization in dtype (fp32)."""
    w = seeded(shape, seed, 0.02, torch.float16)
    bits = w.contiguous().view(torch.int16).numpy().view(np.uint16)
    rp, ra = C.quantize(bits, O.DT_F16, bs, "argmin")
    n = int(np.prod(shape))
    deq = C.dequantize(rp, ra, n, bs, TAG[dtype]).view(np.int16).reshape(shape)
    return torch.from_numpy(rp), torch.from_numpy(ra), torch.from_numpy(deq).view(dtype).float()


def ptr(t):
    return t.data_ptr() if t is not None else None


def fwd_abi(L, stream, x, packed, absmax, bias, t, lb, rank, N, K, bs, workspace=None):
    from stratum_amd.functional import _gemm_dtype
    M = x.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    nbytes = workspace.numel() * 4 if workspace is not None else 0
    rc = L.stm_nf4_gemm_fwd(x.data_ptr(), packed.data_ptr(), absmax.data_ptr(), ptr(bias), ptr(t), ptr(lb), rank,
                            y.data_ptr(), M, N, K, bs, _gemm_dtype(x), ptr(workspace), nbytes, stream)
    assert rc == 0, L.stm_last_error()
    return y


def bwd_abi(L, stream, dy, packed, absmax, u, at, rank, N, K, bs, workspace=None):
    from stratum_amd.functional import _gemm_dtype
    M = dy.shape[0]
    dx = torch.empty((M, K), dtype=dy.dtype, device=dy.device)
    nbytes = workspace.numel() * 4 if workspace is not None else 0
    rc = L.stm_nf4_gemm_bwd_dx(dy.data_ptr(), packed.data_ptr(), absmax.data_ptr(), ptr(u), ptr(at), rank,
                               dx.data_ptr(), M, N, K, bs, _gemm_dtype(dy), ptr(workspace), nbytes, stream)
    assert rc == 0, L.stm_last_error()
    return dx


TILE_KIND = {None: -1, "big": 0, "small": 1, "mid": 2, "big8": 3}


def set_tile(monkeypatch, tile):
    from stratum_amd import _lib
    _lib.lib().stm_nf4_gemm_set_tile(TILE_KIND[tile])


@pytest.fixture(autouse=True)
def _cost_model_after_each_test():
    yield
    from stratum_amd import _lib
    _lib.lib().stm_nf4_gemm_set_tile(-1)


def variants(L, M, N, K, backward, monkeypatch, dev):
    """(name, tile, workspace or None) for every kernel the problem can reach;
    tile None is the library's own choice (the small-M kernel where it applies)."""
    out = []
    for tile in (None, "big", "big8", "mid", "small"):
        set_tile(monkeypatch, tile)
        name = tile or "auto"
        out.append((name + "-unsplit", tile, None))
        nbytes = L.stm_nf4_gemm_workspace_bytes(M, N, K, int(backward))
        if nbytes > 0:
            out.append((name + "-split", tile, torch.empty(nbytes // 4, dtype=torch.float32, device=dev)))
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,bs,bias,rank", [
    (1, 64, 64, 64, False, 0),
    (257, 520, 576, 64, True, 16),     # rows and columns past a tile edge
    (300, 256, 512, 128, True, 32),    # blocksize 128
    (64, 1000, 320, 64, False, 16),    # 1000 columns: last tile 232 wide
    (33, 2048, 4096, 256, False, 0),   # small M: split reductions exist
    (16, 520, 576, 64, True, 16),      # small-M kernel: 520 columns, K % 256 == 64 (half-empty last chunk)
    (5, 4096, 1024, 128, True, 32),    # small-M kernel, blocksize 128, bias + LoRA in the reduce
    (12, 264, 4160, 64, False, 16),    # small-M kernel: 17 groups of 256 over uneven ranges
    (15, 8, 64, 64, True, 0),          # one half chunk, eight columns, unsplit with bias
    (3, 8192, 320, 64, True, 0),       # unsplit, K % 256 == 64
    (9, 8200, 1024, 256, True, 16),    # split, last block of 256 weight rows partly outside
    (7, 264, 384, 128, True, 0),       # K % 256 == 128: last group's second chunk empty
    (11, 520, 448, 64, False, 0),      # K % 256 == 192: last group's second chunk half empty
    (17, 8, 64, 64, True, 0),          # 32-row variant (256-row blocks, groups of 128): half a group, unsplit, bias
    (24, 520, 576, 64, True, 16),      # 32-row variant (256-row blocks): 5 ranges, LoRA in the reduce
    (31, 200, 448, 64, True, 0),       # 32-row variant (256-row blocks): 4 ranges, K % 128 == 64
    (32, 4104, 4160, 64, False, 16),   # 32-row variant (192-row blocks, groups of 256), uneven ranges
    (20, 4096, 4096, 128, True, 16),   # 32-row variant, 192-row blocks: 8 ranges, blocksize 128, bias + LoRA
    (28, 1000, 1536, 512, True, 0),    # 32-row variant, 192-row blocks, blocksize 512
    (26, 6152, 2048, 256, False, 32),  # 32-row variant, 256-row blocks over groups of 128, blocksize 256
    (22, 12296, 1024, 128, True, 16),  # 32-row variant, 256-row blocks: 4 ranges, blocksize 128, last block of 8 rows
    (48, 8200, 1024, 128, False, 16),  # 48-row variant, blocksize 128, 4 ranges, last block of 8 rows
    (33, 8, 64, 64, True, 0),          # 64-row variant (groups of 128): one half group, unsplit with bias
    (48, 520, 576, 64, True, 16),      # 64-row variant, K % 128 == 64, LoRA in the reduce
    (64, 264, 4160, 64, False, 16),    # 64-row variant at its row limit: 33 groups over uneven ranges
    (40, 1000, 1536, 256, True, 0),    # 64-row variant, blocksize 256 (a group is half a block)
    (56, 4104, 1024, 512, True, 32),   # 64-row variant, blocksize 512, last block of 256 rows partly outside
    (320, 520, 576, 64, True, 16),     # last 256-row tile: 64 rows (the 2-fragment short item)
    (384, 264, 640, 64, False, 0),     # last 256-row tile: 128 rows (the 4-fragment short item)
    (100, 256, 1024, 128, True, 16),   # one tile of 100 rows (4 fragments), blocksize 128
    # the split-free small-M kernel (16 T weight rows per work-group, 8 / T reduction slices)
    (1, 4096, 4096, 64, True, 16),     # T = 1: 8 slices, 2 steps; bias + LoRA in its epilogue
    (4, 3072, 1600, 64, False, 0),     # T = 1 at its row limit, 192 work-groups, 7 groups (last 64 deep)
    (2, 4096, 4160, 64, True, 0),      # T = 1: 17 groups, the third step holds one tail group
    (8, 8192, 2048, 128, True, 16),    # T = 2 at its row limit, blocksize 128
    (16, 12288, 1024, 64, True, 16),   # T = 4: 16 rows, 2 slices
    (13, 25600, 1024, 512, False, 0),  # T = 8: one slice, blocksize 512 (one scale per group)
    (2, 12288, 4096, 128, True, 16),   # T = 4, two tiles per wave, 4 slices; blocksize 128, bias + LoRA
    (4, 14336, 4160, 64, False, 0),    # two tiles per wave: 17 groups, the last step holds one
    (8, 4096, 4096, 64, True, 16),     # T = 2 at 128 work-groups (half the CUs; K <= 4096), bias + LoRA
    (1, 2048, 2048, 128, False, 0),    # T = 1 at 128 work-groups, blocksize 128
])
def test_forward_every_kernel(cuda, monkeypatch, dtype, M, N, K, bs, bias, rank):
    from stratum_amd import _lib
    L = _lib.lib()
    stream = _lib.stream_handle(cuda)
    rp, ra, wq = nf4((N, K), M + N + K + bs, bs, dtype)
    packed, absmax = rp.to(cuda), ra.to(cuda)
    x = seeded((M, K), 1, 1.0, dtype).to(cuda)
    b = seeded((N,), 2, 0.1, dtype).to(cuda) if bias else None
    t = seeded((M, rank), 3, 0.5, dtype).to(cuda) if rank else None
    lb = seeded((N, rank), 4, 0.01, dtype).to(cuda) if rank else None
    ref = x.float() @ wq.to(cuda).t().contiguous()
    if bias:
        ref = ref + b.float()
    if rank:
        ref = ref + t.float() @ lb.float().t().contiguous()
    results = {}
    for name, tile, ws in variants(L, M, N, K, False, monkeypatch, cuda):
        set_tile(monkeypatch, tile)
        y = fwd_abi(L, stream, x, packed, absmax, b, t, lb, rank, N, K, bs, ws)
        assert rel(y, ref) <= TOL[dtype], name
        results[name] = y
    first = results["big-unsplit"]
    for name, y in results.items():
        assert rel(y, first) <= TOL[dtype] / 4, name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,bs,rank", [
    (1, 64, 64, 64, 0),
    (257, 192, 320, 64, 16),           # 320 output columns: second tile 64 wide
    (300, 512, 384, 128, 32),          # blocksize 128, second tile 128 wide
    (64, 128, 960, 64, 16),            # last tile 192 wide
    (33, 4096, 2048, 64, 0),           # small M: split reductions exist
    (320, 512, 576, 64, 16),           # last 256-row tile: 64 rows (the 2-fragment short item)
    (384, 256, 640, 64, 0),            # last 256-row tile: 128 rows (the 4-fragment short item)
    (100, 1024, 256, 128, 16),         # one tile of 100 rows (4 fragments), blocksize 128
    # the small-M input gradient (256 output columns per work-group, ranges of 256 weight rows)
    (1, 4096, 4096, 64, 16),           # 16 ranges of one group, LoRA in the reduce
    (16, 14336, 1024, 64, 0),          # 16 rows, 56 groups over uneven ranges
    (5, 4160, 320, 64, 16),            # last group 64 rows (three subgroups past N); 320 columns: second block 64 wide
    (3, 4160, 384, 128, 0),            # blocksize 128 (two scales per work-group row), second block 128 wide
    (9, 448, 768, 256, 0),             # one range: groups of 256 and 192 rows; blocksize 256
    (12, 1024, 4608, 512, 16),         # blocksize 512 (one scale per work-group row), 18 column blocks
    (2, 64, 64, 64, 0),                # one subgroup of one group, one 64-column block
    (17, 64, 64, 64, 0),               # 32-row variant (groups of 128 rows): one subgroup
    (24, 4160, 320, 64, 16),           # 32-row variant: last group 64 rows, LoRA in the reduce
    (32, 14336, 1024, 128, 0),         # 32-row variant at its row limit, blocksize 128
    (20, 448, 768, 256, 16),           # 32-row variant: groups of 128 and 64 rows, blocksize 256
    (7, 2048, 512, 64, 32),            # small-M input gradient, rank 32 in the reduce
    (29, 1024, 1024, 128, 64),         # 32-row variant, rank 64 in the reduce
    (33, 64, 64, 64, 0),               # 64-row variant (two dY copies per wave): one subgroup
    (48, 4160, 320, 64, 16),           # 64-row variant: last group 64 rows, LoRA in the reduce
    (64, 14336, 1024, 128, 0),         # 64-row variant at its row limit, blocksize 128
    (57, 448, 768, 256, 32),           # 64-row variant: groups of 128 and 64 rows, blocksize 256, rank 32
])
def test_input_gradient_every_kernel(cuda, monkeypatch, dtype, M, N, K, bs, rank):
    from stratum_amd import _lib
    L = _lib.lib()
    stream = _lib.stream_handle(cuda)
    rp, ra, wq = nf4((N, K), 3 * M + N + K + bs, bs, dtype)
    packed, absmax = rp.to(cuda), ra.to(cuda)
    dy = seeded((M, N), 5, 1.0, dtype).to(cuda)
    u = seeded((M, rank), 6, 0.5, dtype).to(cuda) if rank else None
    at = seeded((K, rank), 7, 0.01, dtype).to(cuda) if rank else None
    ref = dy.float() @ wq.to(cuda)
    if rank:
        ref = ref + u.float() @ at.float().t().contiguous()
    results = {}
    for name, tile, ws in variants(L, M, N, K, True, monkeypatch, cuda):
        set_tile(monkeypatch, tile)
        dx = bwd_abi(L, stream, dy, packed, absmax, u, at, rank, N, K, bs, ws)
        assert rel(dx, ref) <= TOL[dtype], name
        results[name] = dx
    first = results["big-unsplit"]
    for name, dx in results.items():
        assert rel(dx, first) <= TOL[dtype] / 4, name


@pytest.mark.parametrize("backward", [False, True])
def test_grouped_call_with_one_expert_writes_only_its_rows(cuda, backward):
    """A grouped call with one expert of 5 rows and max_rows 16 (a bound, not
    the row count) runs a grouped kernel (the forward: the grouped form of the
    weight-streaming kernel; the input gradient: the tiles), which takes its
    rows from the offsets: the output rows past offsets[1] keep their contents,
    and the 5 rows match the fp32 reference."""
    from stratum_amd import _lib
    from stratum_amd.functional import _gemm_dtype
    L = _lib.lib()
    dtype, rows, max_rows, N, K = torch.bfloat16, 5, 16, 512, 256
    rp, ra, wq = nf4((N, K), 77, 64, dtype)
    packed, absmax = rp.to(cuda), ra.to(cuda)
    a = seeded((max_rows, K if not backward else N), 12, 1.0, dtype).to(cuda)
    out_cols = K if backward else N
    out = torch.full((max_rows, out_cols), 7.0, dtype=dtype, device=cuda)
    host = torch.tensor([0, rows], dtype=torch.int32)
    dev_off = host.to(cuda)
    fn = L.stm_nf4_grouped_gemm_bwd_dx if backward else L.stm_nf4_grouped_gemm_fwd
    rc = fn(a.data_ptr(), packed.data_ptr(), absmax.data_ptr(), dev_off.data_ptr(), host.data_ptr(), 1, max_rows,
            out.data_ptr(), N, K, 64, _gemm_dtype(a), _lib.stream_handle(cuda))
    assert rc == 0, L.stm_last_error()
    torch.cuda.synchronize()
    ref = a[:rows].float() @ (wq.to(cuda) if backward else wq.to(cuda).t().contiguous())
    assert rel(out[:rows], ref) <= TOL[dtype]
    assert bool((out[rows:] == 7.0).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("counts,N,K,bs,max_rows", [
    ([1, 0, 1, 1, 0, 1, 1, 1], 520, 576, 64, None),        # decode: one row per expert, empty experts, K % 256 == 64
    ([3, 16, 0, 7, 16, 1], 264, 1024, 128, None),          # up to 16 rows (one activation block), blocksize 128
    ([17, 0, 24, 5, 20], 1000, 320, 64, None),             # 17-32 rows: 256-row blocks over groups of 128, K % 128 == 64
    ([33, 64, 0, 2, 48, 40, 1], 264, 1536, 256, None),     # 33-64 rows, blocksize 256 (a group is half a block)
    ([9] * 40, 136, 512, 512, None),                       # 40 experts, blocksize 512
    ([40, 0, 33, 7], 264, 576, 64, None),                  # 33-48 rows: the 48-row layout
    ([1, 0, 3, 2], 264, 576, 64, 64),                      # max_rows 64 (a bound) over 0-3 rows: the 64-row layout
])
def test_grouped_forward_small_rows_per_expert(cuda, monkeypatch, dtype, counts, N, K, bs, max_rows):
    """Grouped forwards with at most 64 rows per expert run the grouped form of
    the weight-streaming small-M kernel (one work-group per block of weight rows
    and expert, rows from the offsets): every expert's rows against fp32 on the
    oracle weights, every output row written, and the tile path (pinned) on the
    same call within rounding."""
    from stratum_amd.functional import nf4_grouped_gemm
    E = len(counts)
    w = seeded((E, N, K), 81, 0.02, torch.float16)
    bits = w.reshape(-1, K).contiguous().view(torch.int16).numpy().view(np.uint16)
    rp, ra = C.quantize(bits, O.DT_F16, bs, "argmin")
    deq = C.dequantize(rp, ra, E * N * K, bs, TAG[dtype]).view(np.int16).reshape(E, N, K)
    wq = torch.from_numpy(deq).view(dtype).float().to(cuda)
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    Mt = int(off[-1])
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    x = seeded((Mt, K), 82, 1.0, dtype).to(cuda)
    set_tile(monkeypatch, None)
    y = torch.full((Mt, N), float("nan"), dtype=dtype, device=cuda)
    nf4_grouped_gemm(x, q, a, off.to(cuda), (N, K), bs, max_rows=max_rows, out=y)
    assert not bool(torch.isnan(y).any())
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi > lo:
            assert rel(y[lo:hi], x[lo:hi].float() @ wq[e].t().contiguous()) <= TOL[dtype], e
    set_tile(monkeypatch, "big")
    yt = nf4_grouped_gemm(x, q, a, off.to(cuda), (N, K), bs, max_rows=max_rows)
    assert rel(y, yt) <= TOL[dtype] / 4


@pytest.mark.parametrize("tile", ["big", "big8", "mid", "small"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_every_tile(cuda, monkeypatch, dtype, tile):
    """Expert banks with empty, tiny and tile-straddling experts; 320 columns in
    the input gradient so its last tile is partly outside the matrix."""
    from stratum_amd.functional import nf4_grouped_gemm
    set_tile(monkeypatch, tile)
    E, N, K = 6, 320, 320
    w = seeded((E, N, K), 78, 0.02, torch.float16)
    bits = w.reshape(-1, K).contiguous().view(torch.int16).numpy().view(np.uint16)
    rp, ra = C.quantize(bits, O.DT_F16, 64, "argmin")
    deq = C.dequantize(rp, ra, E * N * K, 64, TAG[dtype]).view(np.int16).reshape(E, N, K)
    wq = torch.from_numpy(deq).view(dtype).float().to(cuda)
    counts = [0, 3, 300, 1, 256, 70]
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    Mt = int(off[-1])
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    x = seeded((Mt, K), 8, 1.0, dtype).to(cuda)
    dy = seeded((Mt, N), 9, 1.0, dtype).to(cuda)
    y = nf4_grouped_gemm(x, q, a, off.to(cuda), (N, K), 64)
    dx = nf4_grouped_gemm(dy, q, a, off.to(cuda), (N, K), 64, backward=True)
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi == lo:
            continue
        assert rel(y[lo:hi], x[lo:hi].float() @ wq[e].t().contiguous()) <= TOL[dtype], e
        assert rel(dx[lo:hi], dy[lo:hi].float() @ wq[e]) <= TOL[dtype], e


@pytest.mark.parametrize("tile", [None, "big"])
@pytest.mark.parametrize("E", [512, 513])
def test_grouped_item_list_at_the_expert_limit(cuda, monkeypatch, E, tile):
    """The register-weight kernels build their grouped item list in LDS for up
    to 512 experts and enumerate max_rows slots per expert above that. Both
    sides of the limit, with empty and 1-row experts, last tiles of exactly 64,
    65, 128, 129 and 256 rows (tail / main boundaries) and multi-tile experts:
    forward and input gradient per expert against the oracle weights."""
    from stratum_amd.functional import nf4_grouped_gemm
    set_tile(monkeypatch, tile)
    N, K = 256, 128
    dtype = torch.bfloat16
    rng = np.random.default_rng(E)
    counts = rng.integers(0, 200, E)
    special = [0, 1, 64, 65, 128, 129, 256, 257, 256 + 64, 256 + 65, 256 + 128, 256 + 129, 600]
    counts[:len(special)] = special
    counts[-1] = 0
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    Mt = int(off[-1])
    w = seeded((E, N, K), 93, 0.02, torch.float16)
    bits = w.reshape(-1, K).contiguous().view(torch.int16).numpy().view(np.uint16)
    rp, ra = C.quantize(bits, O.DT_F16, 64, "argmin")
    deq = C.dequantize(rp, ra, E * N * K, 64, TAG[dtype]).view(np.int16).reshape(E, N, K)
    wq = torch.from_numpy(deq).view(dtype).float().to(cuda)
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    x = seeded((Mt, K), 94, 1.0, dtype).to(cuda)
    dy = seeded((Mt, N), 95, 1.0, dtype).to(cuda)
    y = nf4_grouped_gemm(x, q, a, off, (N, K), 64)
    dx = nf4_grouped_gemm(dy, q, a, off, (N, K), 64, backward=True)
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi == lo:
            continue
        assert rel(y[lo:hi], x[lo:hi].float() @ wq[e].t().contiguous()) <= TOL[dtype], (e, hi - lo)
        assert rel(dx[lo:hi], dy[lo:hi].float() @ wq[e]) <= TOL[dtype], (e, hi - lo)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_forward_picks_192_row_tiles_from_host_counts(cuda, monkeypatch, dtype):
    """32 experts of 180 or 190 rows (one empty, one of 1 row): one 192-row
    item each (0.81 units) against one full 256-row item (1 unit), so the
    library's own choice is the 192-row register-weight kernel (seen in the
    profile); its result matches the fp32 reference per expert and the forced
    256-row kernel."""
    from stratum_amd import _lib
    from stratum_amd.functional import nf4_grouped_gemm
    E, N, K = 32, 1536, 512
    counts = [180, 190] * 15 + [0, 1]
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    assert _lib.lib().stm_nf4_grouped_tile_rows(off.data_ptr(), E) == 192
    w = seeded((E, N, K), 91, 0.02, torch.float16)
    bits = w.reshape(-1, K).contiguous().view(torch.int16).numpy().view(np.uint16)
    rp, ra = C.quantize(bits, O.DT_F16, 64, "argmin")
    deq = C.dequantize(rp, ra, E * N * K, 64, TAG[dtype]).view(np.int16).reshape(E, N, K)
    wq = torch.from_numpy(deq).view(dtype).float().to(cuda)
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    x = seeded((int(off[-1]), K), 92, 1.0, dtype).to(cuda)
    set_tile(monkeypatch, None)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        y = nf4_grouped_gemm(x, q, a, off, (N, K), 64)
        torch.cuda.synchronize()
    names = [e.key for e in prof.key_averages()]
    if any("k_gemm" in n for n in names):  # the profiler saw device kernels
        assert any("k_gemm_fwd_rw" in n and "192" in n for n in names), names
    set_tile(monkeypatch, "big")
    y256 = nf4_grouped_gemm(x, q, a, off, (N, K), 64)
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi == lo:
            continue
        assert rel(y[lo:hi], x[lo:hi].float() @ wq[e].t().contiguous()) <= TOL[dtype], e
    assert rel(y, y256) <= TOL[dtype] / 4
