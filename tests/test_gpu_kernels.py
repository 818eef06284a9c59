"""GPU parity of the HIP kernels against the CPU oracle.

Bar: quantize (packed codes + absmax) and dequantize are bit-exact; fused GEMMs
are within a relative Frobenius error of 1e-2 (bf16) / 5e-3 (fp16) of an fp32
matmul on the oracle-dequantized weight (the path's stated GEMM tolerances).
"""

import glob
import os

import numpy as np
import pytest
import torch

from gpu_checks import assert_gemm_close
from oracle import c_oracle as C
from oracle import nf4_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-3}
TAG = {torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16, torch.float32: O.DT_F32}


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def host_bits(t):
    """CPU numpy view of a tensor's raw bits (uint16 for 16-bit, uint32 for fp32)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def oracle_quant(x, bs, rule="argmin"):
    return C.quantize(host_bits(x) if x.dtype != torch.float32 else x.numpy(), TAG[x.dtype], bs, rule)


def oracle_deq_tensor(packed, absmax, shape, bs, dtype):
    n = int(np.prod(shape))
    bits = C.dequantize(packed, absmax, n, bs, TAG[dtype])
    if dtype == torch.float32:
        return torch.from_numpy(bits.view(np.float32).reshape(shape))
    return torch.from_numpy(bits.view(np.int16).reshape(shape)).view(dtype)


# -------------------------------------------------------------- quantize
@pytest.mark.parametrize("rule", ["argmin", "threshold"])
@pytest.mark.parametrize("dtype,shape,bs", [
    (torch.float16, (5632, 2048), 64),      # TinyLlama gate_proj, the CPU-runnable reference case
    (torch.float16, (8192, 4096), 64),      # 2^19 blocks: the launch's larger per-wave work size
    (torch.bfloat16, (1024, 1024), 64),
    (torch.float32, (256, 1024), 64),
    (torch.float16, (64, 1024), 128),
    (torch.float16, (32, 2048), 256),
    (torch.bfloat16, (16, 4096), 512),
    (torch.float16, (8, 4096), 1024),
    (torch.float32, (4, 8192), 4096),
    (torch.float16, (1001,), 64),           # odd length, partial last block
    (torch.float16, (3, 100), 64),          # n % 8 != 0
])
def test_quantize_bit_exact(cuda, rule, dtype, shape, bs):
    from stratum_amd.functional import quantize_4bit
    x = seeded(shape, 100 + bs, 0.02 if dtype != torch.float32 else 1.0, dtype)
    packed, state = quantize_4bit(x.to(cuda), blocksize=bs, rounding=rule)
    ref_p, ref_a = oracle_quant(x, bs, rule)
    assert packed.shape == ((x.numel() + 1) // 2, 1) and packed.dtype == torch.uint8
    assert state.absmax.dtype == torch.float32 and state.shape == x.shape and state.dtype == dtype
    np.testing.assert_array_equal(host_bits(state.absmax), ref_a.view(np.uint32))
    np.testing.assert_array_equal(packed.cpu().numpy().ravel(), ref_p)


@pytest.mark.parametrize("rule", ["argmin", "threshold"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_quantize_special_blocks_bit_exact(cuda, rule, dtype):
    """Blocks holding NaN, +-inf, only zeros (with -0.0), a subnormal absmax
    whose reciprocal overflows (bf16/fp32), values of both signs at exactly
    +-absmax, and an ordinary block -- codes bit-exact and absmax equal (NaN
    where the oracle has NaN) against the C oracle."""
    from stratum_amd.functional import quantize_4bit
    bs = 64
    blocks = []
    g = torch.Generator().manual_seed(77)
    base = torch.randn(bs, generator=g) * 0.02
    b = base.clone(); b[5] = float("nan"); blocks.append(b)
    b = base.clone(); b[9] = float("inf"); blocks.append(b)
    b = base.clone(); b[17] = float("-inf"); blocks.append(b)
    b = torch.zeros(bs); b[::3] = -0.0; blocks.append(b)
    tiny = {torch.float16: 6e-8, torch.bfloat16: 1e-39, torch.float32: 1e-40}[dtype]
    b = torch.zeros(bs); b[::2] = tiny; b[1::4] = -tiny; blocks.append(b)
    b = base.clone(); b[0] = b.abs().max() * 2; b[1] = -b[0]; blocks.append(b)
    b = base.clone(); b[2] = float("nan"); b[3] = float("inf"); blocks.append(b)
    blocks.append(base.clone())
    x = torch.cat(blocks).to(dtype)
    packed, state = quantize_4bit(x.to(cuda), blocksize=bs, rounding=rule)
    ref_p, ref_a = oracle_quant(x, bs, rule)
    np.testing.assert_array_equal(packed.cpu().numpy().ravel(), ref_p)
    got = state.absmax.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref_a))
    np.testing.assert_array_equal(got[~np.isnan(got)].view(np.uint32), ref_a[~np.isnan(ref_a)].view(np.uint32))


@pytest.mark.parametrize("rule", ["argmin", "threshold"])
@pytest.mark.parametrize("n", [64 * 64, 64 * 9 + 37])  # whole blocks; a partial block (one-thread kernel)
def test_quantize_fp32_nan_payloads_give_code_zero(cuda, rule, n):
    """fp32 NaNs whose payload bits fall in the kernel's cell-index bits
    (quiet and signalling, both signs): their blocks quantize to code 0 with a
    NaN absmax, bit-exact against the oracle, and the other blocks are intact."""
    from stratum_amd.functional import quantize_4bit
    x = seeded((n,), 31, 1.0, torch.float32)
    bits = x.view(torch.int32)
    payloads = [0x7FC003FC, 0x7FC00004, 0x7FC00100, 0xFFC003F8, 0x7F8003FF, 0xFF800201, 0x7FFFFFFF]
    for i, pl in enumerate(payloads):
        pos = (2 * i) * 64 + 5 * i + 1 if (2 * i) * 64 + 5 * i + 1 < n else n - 1 - i
        bits[pos] = torch.tensor(pl, dtype=torch.int64).to(torch.int32)  # wraps to the signed value
    packed, state = quantize_4bit(x.to(cuda), blocksize=64, rounding=rule)
    ref_p, ref_a = oracle_quant(x, 64, rule)
    np.testing.assert_array_equal(packed.cpu().numpy().ravel(), ref_p)
    got = state.absmax.cpu().numpy()
    assert np.isnan(ref_a).sum() >= 4 and np.array_equal(np.isnan(got), np.isnan(ref_a))
    np.testing.assert_array_equal(got[~np.isnan(got)].view(np.uint32), ref_a[~np.isnan(ref_a)].view(np.uint32))


def test_quantize_unaligned_input_and_cpu_input(cuda):
    from stratum_amd import _lib
    from stratum_amd.functional import quantize_4bit
    base = seeded((4097,), 9, 0.02, torch.float16)
    x = base[1:].contiguous()
    rp, ra = oracle_quant(x, 64)
    # a pointer 2 bytes past an allocation takes the library's unaligned path
    xg = base.to(cuda)[1:]
    p = torch.empty(2048, dtype=torch.uint8, device=cuda)
    a = torch.empty(64, dtype=torch.float32, device=cuda)
    rc = _lib.lib().stm_nf4_quantize(xg.data_ptr(), _lib.STM_F16, 4096, 64, _lib.STM_NF4_ARGMIN, p.data_ptr(),
                                     a.data_ptr(), _lib.stream_handle(cuda))
    assert rc == 0
    np.testing.assert_array_equal(p.cpu().numpy(), rp)
    np.testing.assert_array_equal(host_bits(a), ra.view(np.uint32))
    # a CPU input is quantized on the GPU and returned on the CPU, like bitsandbytes
    p2, s2 = quantize_4bit(x, blocksize=64)
    assert p2.device.type == "cpu" and s2.absmax.device.type == "cpu"
    np.testing.assert_array_equal(p2.numpy().ravel(), rp)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))))
def test_kernels_reproduce_golden_fixtures(cuda, path):
    from stratum_amd.functional import dequantize_4bit, quantize_4bit
    f = np.load(path)
    x, tag, bs = f["x"], int(f["dtype_tag"]), int(f["blocksize"])
    if tag == O.DT_F16:
        xt = torch.from_numpy(x)
    elif tag == O.DT_BF16:
        xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(x)
    for rule in ("argmin", "threshold"):
        p, s = quantize_4bit(xt.to(cuda), blocksize=bs, rounding=rule)
        np.testing.assert_array_equal(p.cpu().numpy().ravel(), f[f"packed_{rule}"])
        np.testing.assert_array_equal(host_bits(s.absmax), f[f"absmax_{rule}"].view(np.uint32))
    n = x.size
    q = torch.from_numpy(f["packed_argmin"]).to(cuda)
    a = torch.from_numpy(f["absmax_argmin"]).to(cuda)
    for dt, key in ((torch.float16, "deq_f16"), (torch.bfloat16, "deq_bf16"), (torch.float32, "deq_f32")):
        out = dequantize_4bit(q, absmax=a, shape=(n,), blocksize=bs, dtype=dt)
        want = f[key].view(np.uint32) if dt == torch.float32 else f[key]
        np.testing.assert_array_equal(host_bits(out), want)


# ------------------------------------------------------------ dequantize
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape,bs", [((5632, 2048), 64), ((4096, 6144), 64), ((14336, 4096), 64),
                                      ((128, 4096), 4096), ((1001,), 64), ((7, 9), 64)])
def test_dequantize_bit_exact(cuda, out_dtype, shape, bs):
    """Bit-exact against the oracle; the sizes take each per-thread work size of
    the kernel (2, 4 and 8 groups of 8 elements: under 2^24, 2^24..2^25, over)
    and the one-element-per-thread tail."""
    from stratum_amd.functional import dequantize_4bit
    x = seeded(shape, 7, 0.02, torch.float16)
    rp, ra = oracle_quant(x, bs)
    q = torch.from_numpy(rp).reshape(-1, 1).to(cuda)
    a = torch.from_numpy(ra).to(cuda)
    out = dequantize_4bit(q, absmax=a, shape=shape, blocksize=bs, dtype=out_dtype)
    assert out.shape == torch.Size(shape) and out.dtype == out_dtype and out.is_contiguous()
    want = C.dequantize(rp, ra, x.numel(), bs, TAG[out_dtype])
    np.testing.assert_array_equal(host_bits(out).ravel(), want.view(np.uint32) if out_dtype == torch.float32 else want)


def test_dequantize_into_misaligned_out(cuda):
    from stratum_amd.functional import dequantize_4bit
    x = seeded((4096,), 8, 0.02, torch.float16)
    rp, ra = oracle_quant(x, 64)
    buf = torch.empty(4097, dtype=torch.float16, device=cuda)
    out = buf[1:]
    dequantize_4bit(torch.from_numpy(rp).to(cuda), absmax=torch.from_numpy(ra).to(cuda), shape=(4096,),
                    blocksize=64, dtype=torch.float16, out=out)
    np.testing.assert_array_equal(host_bits(out), C.dequantize(rp, ra, 4096, 64, O.DT_F16))


def test_all_zero_block_dequantizes_to_negative_zero(cuda):
    from stratum_amd.functional import dequantize_4bit, quantize_4bit
    x = torch.zeros(2, 64, dtype=torch.float16)
    x[1, 3] = 0.5
    p, s = quantize_4bit(x.to(cuda))
    assert s.absmax[0].item() == 0.0
    out = dequantize_4bit(p, s)
    bits = host_bits(out)
    assert np.all(bits[0] == 0x8000)  # code 0 (-1.0) * 0.0 = -0.0, as the reference computes it


# ------------------------------------------------- many tensors per launch
MANY_SHAPES = [(5632, 2048), (256, 2048), (2048, 5632), (1001,), (3, 100), (64, 1024), (8,), (7,), (0,),
               (129, 64)]


@pytest.mark.parametrize("dtype,bs", [(torch.float16, 64), (torch.bfloat16, 64), (torch.float32, 128),
                                      (torch.float16, 256), (torch.bfloat16, 4096)])
def test_quantize_many_matches_the_oracle_per_tensor(cuda, dtype, bs):
    """Ragged sizes (partial last blocks, odd lengths, an empty tensor) and 44
    tensors (two launches of at most 32): every packed array and absmax
    bit-exact against the C oracle."""
    from stratum_amd.functional import quantize_4bit_many
    shapes = MANY_SHAPES + [(64 * (i + 1),) for i in range(34)]
    xs = [seeded(sh, 500 + i, 0.02 if dtype != torch.float32 else 1.0, dtype) for i, sh in enumerate(shapes)]
    got = quantize_4bit_many([x.to(cuda) for x in xs], blocksize=bs)
    assert len(got) == len(xs)
    for i, (x, (p, st)) in enumerate(zip(xs, got)):
        if x.numel() == 0:
            assert p.numel() == 0 and st.absmax.numel() == 0
            continue
        rp, ra = oracle_quant(x, bs)
        assert st.shape == x.shape and st.dtype == dtype and st.blocksize == bs
        np.testing.assert_array_equal(p.cpu().numpy().ravel(), rp, err_msg=f"tensor {i} {tuple(x.shape)}")
        np.testing.assert_array_equal(host_bits(st.absmax), ra.view(np.uint32), err_msg=f"tensor {i}")


def test_quantize_many_unaligned_input_through_the_abi(cuda):
    """A tensor 2 bytes past its allocation (no whole-block batching) beside
    aligned ones: all bit-exact."""
    import ctypes
    from stratum_amd import _lib
    base = seeded((4097,), 9, 0.02, torch.float16)
    others = [seeded((2048,), 10, 0.02, torch.float16), seeded((1000,), 11, 0.02, torch.float16)]
    srcs = [base.to(cuda)[1:]] + [o.to(cuda) for o in others]
    ns = [4096, 2048, 1000]
    ps = [torch.empty((n + 1) // 2, dtype=torch.uint8, device=cuda) for n in ns]
    As = [torch.empty(-(-n // 64), dtype=torch.float32, device=cuda) for n in ns]
    arr = lambda v, t=ctypes.c_void_p: (t * len(v))(*v)
    rc = _lib.lib().stm_nf4_quantize_many(3, arr([x.data_ptr() for x in srcs]), arr(ns, ctypes.c_int64),
                                          _lib.STM_F16, 64, _lib.STM_NF4_ARGMIN, arr([p.data_ptr() for p in ps]),
                                          arr([a.data_ptr() for a in As]), _lib.stream_handle(cuda))
    assert rc == 0, _lib.lib().stm_last_error()
    for x, p, a in zip([base[1:].contiguous()] + others, ps, As):
        rp, ra = oracle_quant(x, 64)
        np.testing.assert_array_equal(p.cpu().numpy(), rp)
        np.testing.assert_array_equal(host_bits(a), ra.view(np.uint32))


@pytest.mark.parametrize("out_dtype,bs", [(torch.float16, 64), (torch.bfloat16, 64), (torch.float32, 256),
                                          (torch.bfloat16, 4096)])
def test_dequantize_many_matches_the_oracle_per_tensor(cuda, out_dtype, bs):
    """The same ragged set (and 44 tensors) dequantized in batched launches,
    into fresh outputs and into given ones, one of them misaligned: bit-exact
    against the C oracle."""
    from stratum_amd.functional import QuantState, dequantize_4bit_many
    shapes = MANY_SHAPES + [(64 * (i + 1),) for i in range(34)]
    xs = [seeded(sh, 700 + i, 0.02, torch.float16) for i, sh in enumerate(shapes)]
    items, want = [], []
    for x in xs:
        rp, ra = oracle_quant(x, bs)
        st = QuantState(absmax=torch.from_numpy(ra).to(cuda), shape=x.shape, code=None, blocksize=bs,
                        quant_type="nf4", dtype=torch.float16)
        items.append((torch.from_numpy(rp).reshape(-1, 1).to(cuda), st))
        w = C.dequantize(rp, ra, x.numel(), bs, TAG[out_dtype])
        want.append(w.view(np.uint32) if out_dtype == torch.float32 else w)
    outs = dequantize_4bit_many(items, dtype=out_dtype)
    for i, (o, w) in enumerate(zip(outs, want)):
        assert o.dtype == out_dtype and o.shape == shapes[i]
        np.testing.assert_array_equal(host_bits(o).ravel(), w, err_msg=f"tensor {i} {shapes[i]}")
    buf = torch.empty(5632 * 2048 + 1, dtype=out_dtype, device=cuda)
    given = [buf[1:].view(5632, 2048)] + [torch.empty(sh, dtype=out_dtype, device=cuda) for sh in shapes[1:]]
    dequantize_4bit_many(items, dtype=out_dtype, out=given)
    for i, (o, w) in enumerate(zip(given, want)):
        np.testing.assert_array_equal(host_bits(o).ravel(), w, err_msg=f"given output {i}")


def test_ensure_weights_dequantizes_a_layer_in_one_launch(cuda):
    """A module with four NF4 projections (and a small plain parameter):
    ensure_weights places all of them with one batched dequantize launch, each
    weight bit-exact against the oracle."""
    import torch.nn as nn
    from stratum_amd.upload import ensure_weights, free_weights, prepare_nf4
    m = nn.Module()
    shapes = {"q": (512, 256), "k": (128, 256), "up": (1024, 256), "down": (256, 1024)}
    for seed, (name, (n, k)) in enumerate(shapes.items()):
        lin = nn.Linear(k, n, bias=False, dtype=torch.float16)
        with torch.no_grad():
            lin.weight.copy_(seeded((n, k), 900 + seed, 0.02, torch.float16))
        setattr(m, name, lin)
    m.norm = nn.Parameter(torch.ones(256, dtype=torch.float16))
    m.requires_grad_(False)
    want = {name: C.dequantize(*oracle_quant(getattr(m, name).weight.data, 64), n * k, 64, O.DT_F16)
            for name, (n, k) in shapes.items()}
    prepare_nf4(m, verbose=False, min_numel=4096)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        ensure_weights(m, 0)
        torch.cuda.synchronize()
    names = [e.name for e in prof.events() if "k_dequantize" in e.name]
    if names:  # the profiler saw device kernels
        assert len(names) == 1 and "k_dequantize_many" in names[0], names
    for name in shapes:
        np.testing.assert_array_equal(host_bits(getattr(m, name).weight).ravel(), want[name], err_msg=name)
    free_weights(m)


def test_roundtrip_is_idempotent_at_8b_mlp_size(cuda):
    """quantize(dequantize(quantize(W))) == quantize(W) at the full [14336, 4096] size."""
    from stratum_amd.functional import dequantize_4bit, quantize_4bit
    w = seeded((14336, 4096), 42, 0.02, torch.float16).to(cuda)
    p1, s1 = quantize_4bit(w)
    d1 = dequantize_4bit(p1, s1)
    p2, s2 = quantize_4bit(d1)
    assert torch.equal(p1, p2)
    assert torch.equal(s1.absmax, s2.absmax)


# ------------------------------------------------------------- fused GEMM
def _rel(y, ref):
    y = y.float()
    return ((y - ref).norm() / ref.norm()).item()


def _nf4_weight(N, K, seed, bs=64, src=torch.float16):
    w = seeded((N, K), seed, 0.02, src)
    rp, ra = oracle_quant(w, bs)
    return rp, ra


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,bias,rank", [
    (1, 128, 64, False, 0), (37, 200, 192, True, 0), (128, 128, 128, False, 16), (300, 520, 576, True, 16),
    (4096, 2048, 1024, False, 0), (512, 14336, 4096, False, 16), (129, 1024, 3072, True, 32),
])
def test_gemm_fwd_matches_fp32_reference(cuda, dtype, M, N, K, bias, rank):
    from stratum_amd.functional import nf4_gemm_fwd
    rp, ra = _nf4_weight(N, K, M + N + K)
    wq = oracle_deq_tensor(rp, ra, (N, K), 64, dtype).to(cuda)
    x = seeded((M, K), 1, 1.0, dtype).to(cuda)
    b = seeded((N,), 2, 0.1, dtype).to(cuda) if bias else None
    t = seeded((M, rank), 3, 0.5, dtype).to(cuda) if rank else None
    lb = seeded((N, rank), 4, 0.01, dtype).to(cuda) if rank else None
    y = nf4_gemm_fwd(x, torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda), (N, K), 64, bias=b,
                     lora_t=t, lora_b=lb)
    ref = x.float() @ wq.float().t().contiguous()
    if bias:
        ref = ref + b.float()
    if rank:
        ref = ref + t.float() @ lb.float().t().contiguous()
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel(y, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,rank", [
    (1, 64, 64, 0), (37, 192, 128, 0), (300, 576, 512, 16), (4096, 1024, 2048, 0), (512, 14336, 4096, 16),
    (129, 3072, 1024, 32),
])
def test_gemm_bwd_dx_matches_fp32_reference(cuda, dtype, M, N, K, rank):
    from stratum_amd.functional import nf4_gemm_bwd_dx
    rp, ra = _nf4_weight(N, K, M * 3 + N + K)
    wq = oracle_deq_tensor(rp, ra, (N, K), 64, dtype).to(cuda)
    dy = seeded((M, N), 5, 1.0, dtype).to(cuda)
    u = seeded((M, rank), 6, 0.5, dtype).to(cuda) if rank else None
    at = seeded((K, rank), 7, 0.01, dtype).to(cuda) if rank else None
    dx = nf4_gemm_bwd_dx(dy, torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda), (N, K), 64,
                         lora_u=u, lora_at=at)
    ref = dy.float() @ wq.float()
    if rank:
        ref = ref + u.float() @ at.float().t().contiguous()
    assert dx.shape == (M, K) and dx.dtype == dtype
    assert _rel(dx, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,backward", [
    (16, 14336, 4096, False), (1, 4096, 14336, False), (7, 2048, 1024, False),
    (16, 14336, 4096, True), (3, 4096, 14336, True), (64, 3072, 1024, True),
])
def test_split_reduction_matches_fp32_and_unsplit(cuda, dtype, M, N, K, backward):
    """Small M splits the reduction over work-groups (fp32 partials in a
    workspace, summed by a second kernel): same result as the reference within
    tolerance, bias added once, LoRA term once, and within rounding of the
    unsplit kernel (called through the ABI with no workspace)."""
    from stratum_amd import _lib
    from stratum_amd.functional import _gemm_dtype, nf4_gemm_bwd_dx, nf4_gemm_fwd
    L = _lib.lib()
    assert L.stm_nf4_gemm_workspace_bytes(M, N, K, int(backward)) > 0, "case must exercise the split path"
    rp, ra = _nf4_weight(N, K, M + N + K + int(backward))
    wq = oracle_deq_tensor(rp, ra, (N, K), 64, dtype).to(cuda)
    packed, absmax = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    R = 16
    if not backward:
        x = seeded((M, K), 11, 1.0, dtype).to(cuda)
        b = seeded((N,), 12, 0.1, dtype).to(cuda)
        t = seeded((M, R), 13, 0.5, dtype).to(cuda)
        lb = seeded((N, R), 14, 0.01, dtype).to(cuda)
        y = nf4_gemm_fwd(x, packed, absmax, (N, K), 64, bias=b, lora_t=t, lora_b=lb)
        ref = x.float() @ wq.float().t().contiguous() + b.float() + t.float() @ lb.float().t().contiguous()
        plain = torch.empty_like(y)
        rc = L.stm_nf4_gemm_fwd(x.data_ptr(), packed.data_ptr(), absmax.data_ptr(), b.data_ptr(), t.data_ptr(),
                                lb.data_ptr(), R, plain.data_ptr(), M, N, K, 64, _gemm_dtype(x), None, 0,
                                _lib.stream_handle(x.device))
    else:
        dy = seeded((M, N), 15, 1.0, dtype).to(cuda)
        u = seeded((M, R), 16, 0.5, dtype).to(cuda)
        at = seeded((K, R), 17, 0.01, dtype).to(cuda)
        y = nf4_gemm_bwd_dx(dy, packed, absmax, (N, K), 64, lora_u=u, lora_at=at)
        ref = dy.float() @ wq.float() + u.float() @ at.float().t().contiguous()
        plain = torch.empty_like(y)
        rc = L.stm_nf4_gemm_bwd_dx(dy.data_ptr(), packed.data_ptr(), absmax.data_ptr(), u.data_ptr(), at.data_ptr(),
                                   R, plain.data_ptr(), M, N, K, 64, _gemm_dtype(dy), None, 0,
                                   _lib.stream_handle(dy.device))
    assert rc == 0, L.stm_last_error()
    assert _rel(y, ref) <= TOL[dtype]
    assert _rel(plain, ref) <= TOL[dtype]
    # only the fp32 summation order differs: a few elements one 16-bit step apart
    assert _rel(y, plain.float()) <= TOL[dtype] / 4


@pytest.mark.parametrize("dtype", [torch.bfloat16])
def test_gemm_full_lora_step_shape(cuda, dtype):
    """W [14336, 4096], X [8192, 4096]: forward and input gradient at full size."""
    from stratum_amd.functional import nf4_gemm_bwd_dx, nf4_gemm_fwd
    N, K, M = 14336, 4096, 8192
    rp, ra = _nf4_weight(N, K, 55)
    wq = oracle_deq_tensor(rp, ra, (N, K), 64, dtype).to(cuda).float()
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    x = seeded((M, K), 1, 1.0, dtype).to(cuda)
    y = nf4_gemm_fwd(x, q, a, (N, K), 64)
    # whole matrix and every 32 x 32 fragment (persistent items past the first
    # 256 work-groups, the XCD tile walk)
    assert_gemm_close(y, x.float() @ wq.t().contiguous(), dtype, "forward")
    del y
    dy = seeded((M, N), 2, 1.0, dtype).to(cuda)
    dx = nf4_gemm_bwd_dx(dy, q, a, (N, K), 64)
    assert_gemm_close(dx, dy.float() @ wq, dtype, "input gradient")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouped_gemm_matches_per_expert_reference(cuda, dtype):
    from stratum_amd.functional import nf4_grouped_gemm
    E, N, K = 8, 256, 192
    w = seeded((E, N, K), 77, 0.02, torch.float16)
    rp, ra = oracle_quant(w.reshape(-1, K), 64)
    wq = oracle_deq_tensor(rp, ra, (E, N, K), 64, dtype).to(cuda).float()
    counts = [0, 5, 130, 64, 1, 0, 257, 33]
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    Mt = int(off[-1])
    x = seeded((Mt, K), 8, 1.0, dtype).to(cuda)
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    y = nf4_grouped_gemm(x, q, a, off.to(cuda), (N, K), 64)
    dy = seeded((Mt, N), 9, 1.0, dtype).to(cuda)
    dx = nf4_grouped_gemm(dy, q, a, off.to(cuda), (N, K), 64, backward=True)
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi == lo:
            continue
        assert _rel(y[lo:hi], x[lo:hi].float() @ wq[e].t().contiguous()) <= TOL[dtype]
        assert _rel(dx[lo:hi], dy[lo:hi].float() @ wq[e]) <= TOL[dtype]


def test_grouped_gemm_host_offsets_cached_across_streams(cuda):
    """Host (CPU) offsets are validated and uploaded once, then reused: the same
    array on the default stream, then on a side stream that starts behind a
    long sleep, then again after the cache has been filled past its size --
    every result bit-identical to the first."""
    from stratum_amd import functional as F
    E, N, K = 4, 256, 256
    w = seeded((E, N, K), 81, 0.02, torch.float16)
    rp, ra = oracle_quant(w.reshape(-1, K), 64)
    q, a = torch.from_numpy(rp).to(cuda), torch.from_numpy(ra).to(cuda)
    counts = [40, 0, 300, 17]
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    x = seeded((int(off[-1]), K), 82, 1.0, torch.bfloat16).to(cuda)
    first = F.nf4_grouped_gemm(x, q, a, off, (N, K), 64)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        torch.cuda._sleep(20_000_000)
        again = F.nf4_grouped_gemm(x, q, a, off.clone(), (N, K), 64)
    for i in range(F._OFFSETS_CACHE_SIZE + 2):  # evict the cached array
        other = torch.tensor([0, i, i, i, int(off[-1])], dtype=torch.int32)
        F.nf4_grouped_gemm(x, q, a, other, (N, K), 64)
    torch.cuda.synchronize()
    third = F.nf4_grouped_gemm(x, q, a, off, (N, K), 64)
    assert torch.equal(again, first) and torch.equal(third, first)


def test_entry_points_replay_correctly_in_a_hip_graph(cuda):
    """quantize, dequantize and a split-reduction GEMM (M = 16) captured into
    one HIP graph: every replay, with eager work and synchronisations between
    replays, matches the eager results bit for bit. (The entry points record no
    memset: the split partials are fully overwritten.)"""
    from stratum_amd.functional import dequantize_4bit, nf4_gemm_fwd, quantize_4bit
    w = seeded((1024, 2048), 91, 0.02, torch.float16).to(cuda)
    x = seeded((16, 2048), 92, 1.0, torch.bfloat16).to(cuda)
    p_e, s_e = quantize_4bit(w)
    d_e = dequantize_4bit(p_e, s_e, dtype=torch.bfloat16)
    y_e = nf4_gemm_fwd(x, p_e, s_e.absmax, (1024, 2048), 64)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        quantize_4bit(w)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        p_g, s_g = quantize_4bit(w)
        d_g = dequantize_4bit(p_g, s_g, dtype=torch.bfloat16)
        y_g = nf4_gemm_fwd(x, p_g, s_g.absmax, (1024, 2048), 64)
    for i in range(3):
        # eager work between replays that touches the same kind of kernels
        junk = nf4_gemm_fwd(x.flip(0), p_e, s_e.absmax, (1024, 2048), 64)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(p_g, p_e), i
        assert torch.equal(s_g.absmax, s_e.absmax), i
        assert torch.equal(d_g, d_e), i
        assert torch.equal(y_g, y_e), i
        del junk
