"""The C ABI library on the CPU: it loads, exports every symbol the header
declares, rejects bad arguments before touching a GPU, and its host-side
decision tables agree with the oracle (exhaustively over fp32)."""

import ctypes
import os
import re

import numpy as np
import pytest

from oracle import c_oracle as C
from oracle import nf4_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "stratum_nf4.h")


@pytest.fixture(scope="module")
def L():
    from stratum_amd import _lib
    return _lib.lib()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(stm_\w+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = header_functions()
    for n in ("stm_nf4_quantize", "stm_nf4_dequantize", "stm_nf4_gemm_fwd", "stm_nf4_gemm_bwd_dx",
              "stm_nf4_grouped_gemm_fwd", "stm_nf4_grouped_gemm_bwd_dx", "stm_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol(L):
    from stratum_amd import _lib
    missing = [n for n in header_functions() if not hasattr(L, n)]
    assert not missing, missing
    assert set(header_functions()) == set(_lib.SIGNATURES)


def test_abi_version(L):
    assert L.stm_nf4_abi_version() == 5


@pytest.mark.parametrize("rule,code", [("argmin", 0), ("threshold", 1)])
def test_boundaries_match_oracle(L, rule, code):
    out = np.zeros(15, np.float32)
    assert L.stm_nf4_decision_boundaries(code, out.ctypes.data) == 0
    np.testing.assert_array_equal(out.view(np.uint32), O.decision_boundaries(rule).view(np.uint32))


@pytest.mark.parametrize("rule,code", [("argmin", 0), ("threshold", 1)])
def test_cell_table_is_exact_over_all_fp32(L, rule, code):
    """Every fp32 s in [-1, 1] (plus NaN, +-inf, values just outside) gets the
    same level from the kernel's 65-cell table as from the C restatement."""
    bound = np.zeros(65, np.float32)
    base = np.zeros(65, np.uint8)
    assert L.stm_nf4_cell_table(code, bound.ctypes.data, base.ctypes.data) == 0
    bad, first = C.check_cells(bound, base, rule)
    assert bad == 0, f"first mismatch at bits {first:#010x}"


def _err(L):
    return L.stm_last_error().decode()


def test_invalid_arguments_are_rejected_without_a_gpu(L):
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    assert L.stm_nf4_quantize(p, 0, 128, 100, 0, p, p, None) == -1
    assert "blocksize" in _err(L)
    assert L.stm_nf4_quantize(p, 9, 128, 64, 0, p, p, None) == -1
    assert L.stm_nf4_quantize(p, 0, 128, 64, 5, p, p, None) == -1
    assert L.stm_nf4_quantize(None, 0, 128, 64, 0, p, p, None) == -1
    assert L.stm_nf4_quantize(None, 0, 0, 64, 0, None, None, None) == 0  # empty input is a no-op
    assert L.stm_nf4_dequantize(p, p, -1, 64, p, 0, None) == -1
    assert L.stm_nf4_dequantize(p, p, 16, 64, p, 7, None) == -1
    assert L.stm_nf4_dequantize(None, None, 0, 64, None, 0, None) == 0
    # K not a multiple of 64 -> unsupported
    assert L.stm_nf4_gemm_fwd(p, p, p, None, None, None, 0, p, 4, 8, 100, 64, 1, None, 0, None) == -2
    assert "multiple of 64" in _err(L)
    # fp32 GEMM is not a thing
    assert L.stm_nf4_gemm_fwd(p, p, p, None, None, None, 0, p, 4, 8, 64, 64, 2, None, 0, None) == -1
    # bad LoRA rank
    assert L.stm_nf4_gemm_fwd(p, p, p, None, p, p, 8, p, 4, 8, 64, 64, 1, None, 0, None) == -1
    # backward needs N % 64 == 0
    assert L.stm_nf4_gemm_bwd_dx(p, p, p, None, None, 0, p, 4, 40, 64, 64, 1, None, 0, None) == -2
    # misaligned pointer
    assert L.stm_nf4_gemm_fwd(p + 2, p, p, None, None, None, 0, p, 4, 8, 64, 64, 1, None, 0, None) == -1
    assert L.stm_nf4_grouped_gemm_fwd(p, p, p, None, None, 4, 16, p, 8, 64, 64, 1, None) == -1
    assert L.stm_nf4_grouped_gemm_fwd(p, p, p, p, None, 0, 16, p, 8, 64, 64, 1, None) == -1
    # batched (de)quantize: argument checks before any launch
    i64 = (ctypes.c_int64 * 1)(-1)
    ptrs = (ctypes.c_void_p * 1)(p)
    assert L.stm_nf4_quantize_many(-1, None, None, 0, 64, 0, None, None, None) == -1
    assert L.stm_nf4_quantize_many(0, None, None, 0, 64, 0, None, None, None) == 0   # nothing to do
    assert L.stm_nf4_quantize_many(1, None, None, 0, 64, 0, None, None, None) == -1  # NULL arrays
    assert L.stm_nf4_quantize_many(1, ptrs, i64, 0, 64, 0, ptrs, ptrs, None) == -1   # n < 0
    assert L.stm_nf4_quantize_many(1, ptrs, i64, 0, 96, 0, ptrs, ptrs, None) == -1   # blocksize
    assert L.stm_nf4_quantize_many(1, ptrs, i64, 0, 64, 7, ptrs, ptrs, None) == -1   # rule
    assert L.stm_nf4_dequantize_many(-1, None, None, None, 64, None, 0, None) == -1
    assert L.stm_nf4_dequantize_many(0, None, None, None, 64, None, 0, None) == 0
    assert L.stm_nf4_dequantize_many(1, ptrs, ptrs, i64, 64, ptrs, 0, None) == -1    # n < 0
    assert L.stm_nf4_dequantize_many(1, ptrs, ptrs, i64, 64, ptrs, 9, None) == -1    # dtype
    nulls = (ctypes.c_void_p * 1)(None)
    i64[0] = 64
    assert L.stm_nf4_dequantize_many(1, nulls, ptrs, i64, 64, ptrs, 0, None) == -1   # NULL tensor pointer
    assert "NULL pointer for tensor 0" in _err(L)
    assert L.stm_nf4_grouped_tile_rows(None, 4) == -1
    assert L.stm_nf4_grouped_tile_rows(p, 0) == -1
    assert L.stm_nf4_decision_boundaries(3, p) == -1


def test_python_wrapper_raises_value_error_on_bad_arguments():
    import torch
    from stratum_amd import functional as F
    with pytest.raises(NotImplementedError):
        F.quantize_4bit(torch.zeros(64, 64), quant_type="fp4")
    with pytest.raises(ValueError):
        F.quantize_4bit(torch.zeros(64, 64), blocksize=100)
    with pytest.raises(NotImplementedError):
        F.quantize_4bit(torch.zeros(64, 64), compress_statistics=True)
    with pytest.raises(RuntimeError):
        F.dequantize_4bit(torch.zeros(32, 1, dtype=torch.uint8), absmax=torch.ones(1), shape=(8, 8))
    # batched forms: argument checks before any GPU work
    assert F.quantize_4bit_many([]) == [] and F.dequantize_4bit_many([]) == []
    with pytest.raises(ValueError):
        F.quantize_4bit_many([torch.zeros(64, dtype=torch.float16)], rounding="nearest")
    with pytest.raises(ValueError):
        F.quantize_4bit_many([torch.zeros(64, dtype=torch.float16), torch.zeros(64, dtype=torch.bfloat16)])
    st64 = F.QuantState(absmax=torch.ones(1), shape=(8, 8), blocksize=64, dtype=torch.float16)
    st128 = F.QuantState(absmax=torch.ones(1), shape=(8, 16), blocksize=128, dtype=torch.float16)
    q = torch.zeros(32, 1, dtype=torch.uint8)
    with pytest.raises(ValueError):
        F.dequantize_4bit_many([(q, st64), (torch.zeros(64, 1, dtype=torch.uint8), st128)])
    with pytest.raises(RuntimeError):
        F.dequantize_4bit_many([(q, st64)])  # packed bytes on the CPU


def test_swiglu_rejects_bad_arguments(L):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails before any launch
    assert L.stm_swiglu_fwd(None, fake, 4, 8, 1, None) == -1
    assert L.stm_swiglu_fwd(fake, fake, 4, 8, 2, None) == -1  # fp32 is not a SwiGLU dtype
    assert L.stm_swiglu_fwd(fake, fake, -1, 8, 1, None) == -1
    assert L.stm_swiglu_bwd(fake, None, fake, 4, 8, 0, None) == -1
    assert L.stm_swiglu_bwd(fake, fake, fake, 4, -8, 0, None) == -1
    assert b"swiglu" in L.stm_last_error()


def test_swiglu_empty_is_a_no_op(L):
    fake = ctypes.c_void_p(4096)
    assert L.stm_swiglu_fwd(fake, fake, 0, 8, 1, None) == 0
    assert L.stm_swiglu_bwd(fake, fake, fake, 16, 0, 0, None) == 0


def test_swiglu_empty_accepts_null_pointers(L):
    assert L.stm_swiglu_fwd(None, None, 0, 8, 1, None) == 0
    assert L.stm_swiglu_bwd(None, None, None, 5, 0, 0, None) == 0



def test_gemm_workspace_sizing(L):
    # large problems fill the GPU with output tiles: no split, no workspace
    assert L.stm_nf4_gemm_workspace_bytes(8192, 14336, 4096, 0) == 0
    assert L.stm_nf4_gemm_workspace_bytes(8192, 14336, 4096, 1) == 0
    # M = 33, W [14336, 4096]: the small-M forward's 56 blocks of 256 weight
    # rows x 32 groups of 128 split 4 ways (224 work-groups, one round; the
    # tile path would split 2 ways); M = 16: the input gradient's 16 big tiles
    # (4096 output columns) split 16 ways over the 224 steps of its 14336-long
    # reduction
    assert L.stm_nf4_gemm_workspace_bytes(33, 14336, 4096, 0) == 4 * 33 * 14336 * 4
    assert L.stm_nf4_gemm_workspace_bytes(16, 14336, 4096, 1) == 16 * 16 * 4096 * 4
    # forward with M <= 16 where the split-free small-M kernel applies (the rows
    # fit and it fills the GPU): no partials of its own, so the workspace is
    # what a pinned tile kind would split: 16 rows of W [14336, 4096] -> the
    # 128 x 128 tiles' 2 ways; 1 row of W [4096, 14336] -> 8 ways
    assert L.stm_nf4_gemm_workspace_bytes(16, 14336, 4096, 0) == 2 * 16 * 14336 * 4
    assert L.stm_nf4_gemm_workspace_bytes(1, 4096, 14336, 0) == 8 * 1 * 4096 * 4
    # 16 rows of W [4096, 14336] do not fit it (16 rows need 4 tiles per
    # work-group: 64 work-groups): the split small-M kernel's ranges (blocks of
    # 256 weight rows, one per CU; groups of 256 along K; least estimated
    # time): 16 blocks x 56 groups -> 14 ranges of 4
    assert L.stm_nf4_gemm_workspace_bytes(16, 4096, 14336, 0) == 14 * 16 * 4096 * 4
    # a short reduction over few blocks still splits: W [3072, 1024] at 16
    # rows -> 12 blocks x 4 groups -> 4 ranges of 1
    assert L.stm_nf4_gemm_workspace_bytes(16, 3072, 1024, 0) == 4 * 16 * 3072 * 4
    # 17..32 rows, the faster of two estimated layouts: here 256 weight rows
    # over groups of 128 (56 blocks x 32 groups -> 4 ranges of 8, 224
    # work-groups) beats 192 rows over groups of 256 (3 ranges of 6)
    assert L.stm_nf4_gemm_workspace_bytes(17, 14336, 4096, 0) == 4 * 17 * 14336 * 4
    # ... and on W [4096, 4096] the 192-row layout's 8 ranges of 2 groups
    assert L.stm_nf4_gemm_workspace_bytes(20, 4096, 4096, 0) == 8 * 20 * 4096 * 4
    assert L.stm_nf4_gemm_workspace_bytes(24, 4096, 4096, 0) == 8 * 24 * 4096 * 4
    # W [28672, 4096] at 17 rows: 112 blocks of 256 rows -> 2 ranges (224 work-groups)
    assert L.stm_nf4_gemm_workspace_bytes(17, 28672, 4096, 0) == 2 * 17 * 28672 * 4
    # 64 rows (groups of 128): W [4096, 4096] -> 16 blocks x 32 groups -> 11 ranges of 3
    assert L.stm_nf4_gemm_workspace_bytes(64, 4096, 4096, 0) == 11 * 64 * 4096 * 4
    # input gradient at 64 rows of W [1024, 4096]: 8 groups of 128 weight rows;
    # counting the partials' bytes keeps it at 4 ranges (the rule without them
    # took 8)
    assert L.stm_nf4_gemm_workspace_bytes(64, 1024, 4096, 1) == 4 * 64 * 4096 * 4
    # one block of weight rows over 4 groups: the small-M kernel's 4 ranges of
    # one group (estimated below one work-group walking all 4), which is more
    # than the tile path's 2 (pinned tile kinds, 8 steps per range); one group:
    # one range, no workspace
    assert L.stm_nf4_gemm_workspace_bytes(16, 256, 1024, 0) == 4 * 16 * 256 * 4
    assert L.stm_nf4_gemm_workspace_bytes(16, 256, 256, 0) == 0
    assert L.stm_nf4_gemm_workspace_bytes(0, 256, 4096, 0) == 0
    assert L.stm_nf4_gemm_workspace_bytes(-1, 256, 256, 0) < 0


def test_gemm_rejects_small_workspace(L):
    p = ctypes.c_void_p(4096)
    need = L.stm_nf4_gemm_workspace_bytes(16, 14336, 4096, 0)
    assert L.stm_nf4_gemm_fwd(p, p, p, None, None, None, 0, p, 16, 14336, 4096, 64, 1, p, need - 4, None) == -1
    assert b"workspace" in L.stm_last_error()


def test_lora_arguments_are_rejected_without_a_gpu(L):
    buf = ctypes.create_string_buffer(4096)
    p = (ctypes.addressof(buf) + 15) & ~15
    ws_need = L.stm_lora_workspace_bytes(64, 256, 16, 0)
    # rank outside {8, 16, 24, 32}
    assert L.stm_lora_down(p, p, p, 64, 256, 12, 1.0, 1, p, ws_need, None) == -2
    assert "rank" in _err(L)
    assert L.stm_lora_down(p, p, p, 64, 256, 64, 1.0, 1, p, ws_need, None) == -2
    # columns not a multiple of 8
    assert L.stm_lora_down(p, p, p, 64, 250, 16, 1.0, 1, p, ws_need, None) == -2
    # fp32 and unknown dtypes
    assert L.stm_lora_down(p, p, p, 64, 256, 16, 1.0, 2, p, ws_need, None) == -1
    # misaligned operand, null operand
    assert L.stm_lora_down(p + 2, p, p, 64, 256, 16, 1.0, 1, p, ws_need, None) == -1
    assert L.stm_lora_dy(p, None, p, p, p, 64, 256, 16, 1.0, 1, p, 1 << 30, None) == -1
    assert L.stm_lora_da(p, p, None, 64, 256, 16, 1, p, 1 << 30, None) == -1
    # workspace too small or missing
    assert L.stm_lora_down(p, p, p, 64, 256, 16, 1.0, 1, p, ws_need - 16, None) == -1
    assert "workspace" in _err(L)
    assert L.stm_lora_da(p, p, p, 64, 256, 16, 1, None, 0, None) == -1
    # no rows: nothing to do for the forward product
    assert L.stm_lora_down(None, None, None, 0, 256, 16, 1.0, 1, None, 0, None) == 0
    # too large for one buffer range: 4M + 8 columns, or 2^24 + 64 rows
    assert L.stm_lora_down(p, p, p, 64, (1 << 22) + 8, 16, 1.0, 1, p, 1 << 40, None) == -2
    assert L.stm_lora_down(p, p, p, (1 << 24) + 64, 256, 16, 1.0, 1, p, 1 << 40, None) == -2
    assert L.stm_lora_workspace_bytes(64, 256, 16, 3) < 0
    assert L.stm_lora_workspace_bytes(64, 256, 40, 0) < 0
    # widths beyond the kernels' limits are refused by the sizing call too
    # (2^25 columns once divided by zero while planning the row blocks)
    assert L.stm_lora_workspace_bytes(5, 1 << 25, 16, 0) == -2
    assert L.stm_lora_workspace_bytes(5, (1 << 22) + 8, 16, 1) == -2
    assert L.stm_lora_workspace_bytes((1 << 24) + 64, 256, 16, 2) == -2
    assert L.stm_lora_workspace_bytes(64, 250, 16, 0) == -2


def test_lora_workspace_sizing(L):
    """fp32 partials: [column blocks of 256][rows][RP] for the row-direction sums
    and [row blocks][cols][RP] for the column-direction sums, RP = rank rounded
    up to 16; about 512 work-groups (row blocks of whole 64-row steps), 768 for
    the two-direction pass at RP = 16."""
    # lora_dy at the 8192 x 14336 shape: 56 column blocks, 13 row blocks of 640 rows
    assert L.stm_lora_workspace_bytes(8192, 14336, 16, 1) == 56 * 8192 * 16 * 4 + 13 * 14336 * 16 * 4
    # rank 32 (RP = 32): two work-groups per CU, 10 row blocks of 832 rows
    assert L.stm_lora_workspace_bytes(8192, 14336, 32, 1) == 56 * 8192 * 32 * 4 + 10 * 14336 * 32 * 4
    # lora_down / lora_da on X [8192, 4096]: 16 column blocks, 32 row blocks of 256 rows
    assert L.stm_lora_workspace_bytes(8192, 4096, 16, 0) == 16 * 8192 * 16 * 4
    assert L.stm_lora_workspace_bytes(8192, 4096, 16, 2) == 32 * 4096 * 16 * 4
    # rank 8 is padded to 16, rank 24 to 32
    assert L.stm_lora_workspace_bytes(8192, 4096, 8, 0) == 16 * 8192 * 16 * 4
    assert L.stm_lora_workspace_bytes(8192, 4096, 24, 0) == 16 * 8192 * 32 * 4
    # ragged: 1000 columns = 4 blocks; 65 rows = 2 steps, one row block each
    assert L.stm_lora_workspace_bytes(65, 1000, 16, 1) == 4 * 65 * 16 * 4 + 2 * 1000 * 16 * 4
    assert L.stm_lora_workspace_bytes(0, 1000, 16, 1) == 0
    # row blocks are capped so that one block of dY spans at most 2^31 bytes:
    # 1M rows x 14336 columns -> 1170 steps of 64 rows per block, 15 row blocks
    per = (1 << 31) // (14336 * 2 * 64)
    nrb = -(-(1 << 20) // (per * 64))
    assert L.stm_lora_workspace_bytes(1 << 20, 14336, 16, 2) == nrb * 14336 * 16 * 4
    # no columns: nothing to reduce (a zero-width X gives T = 0)
    assert L.stm_lora_workspace_bytes(5, 0, 16, 0) == 0
    assert L.stm_lora_workspace_bytes(5, 0, 16, 2) == 0


def test_lora_eligibility_matches_the_library_limits(L):
    """functional.lora_supported routes to the kernels exactly the problems the
    library accepts (checked against the library's own answer on the CPU)."""
    from stratum_amd.functional import lora_supported
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) & ~15
    cases = [(16, 14336, 8192), (8, 8, 1), (24, 4104, 130), (32, 1 << 22, 1), (16, (1 << 22) + 8, 1),
             (16, 256, 1 << 24), (16, 256, (1 << 24) + 64), (12, 256, 64), (64, 256, 64), (16, 250, 64)]
    for rank, cols, rows in cases:
        rc = L.stm_lora_down(p, p, p, rows, cols, rank, 1.0, 1, p, 0, None)
        # -1 here means only "workspace too small": the shape itself was accepted
        accepted = rc in (0, -1)
        assert lora_supported(rank, cols, rows) == accepted, (rank, cols, rows, rc)


@pytest.mark.parametrize("offsets,max_rows,match", [
    ([1, 4, 10], None, "start at 0"),           # does not start at 0
    ([0, 6, 4, 10], None, "non-decreasing"),    # an expert with negative rows
    ([0, 4, 12], None, "end at"),               # past the last row of x
    ([0, 4, 8], None, "end at"),                # short of the last row
    ([0, 4, 10], 5, "max_rows"),                # max_rows below the largest expert (6 rows)
    ([0], None, "two entries"),                 # no expert
])
def test_grouped_gemm_rejects_bad_offsets_before_launch(offsets, max_rows, match):
    """The grouped GEMM indexes X and Y with the offsets: a bad array must be a
    ValueError on the host, never a launch (these tensors are on the CPU, so a
    launch would touch host memory from the GPU)."""
    import torch
    from stratum_amd.functional import nf4_grouped_gemm
    E = max(len(offsets) - 1, 1)
    x = torch.zeros(10, 64, dtype=torch.bfloat16)
    packed = torch.zeros(E * 64 * 64 // 2, dtype=torch.uint8)
    absmax = torch.ones(E * 64, dtype=torch.float32)
    with pytest.raises(ValueError, match=match):
        nf4_grouped_gemm(x, packed, absmax, torch.tensor(offsets, dtype=torch.int32), (64, 64), 64,
                         max_rows=max_rows)


def test_grouped_gemm_rejects_a_short_payload_and_cpu_operands():
    import torch
    from stratum_amd.functional import nf4_grouped_gemm
    x = torch.zeros(10, 64, dtype=torch.bfloat16)
    off = torch.tensor([0, 4, 10], dtype=torch.int32)
    with pytest.raises(ValueError, match="packed holds"):
        nf4_grouped_gemm(x, torch.zeros(64 * 64 // 2, dtype=torch.uint8), torch.ones(128), off, (64, 64), 64)
    with pytest.raises(ValueError, match="absmax holds"):
        nf4_grouped_gemm(x, torch.zeros(64 * 64, dtype=torch.uint8), torch.ones(64), off, (64, 64), 64)
    with pytest.raises(RuntimeError, match="GPU"):
        nf4_grouped_gemm(x, torch.zeros(64 * 64, dtype=torch.uint8), torch.ones(128), off, (64, 64), 64)


def test_noalloc_forward_refuses_oversized_problems_before_touching_a_gpu(L):
    """stm_nf4_gemm_fwd_noalloc checks the partials of the split plan against its
    16 MiB static scratch on the host: an oversized problem is refused with a
    clear error before any device call (host pointers here)."""
    buf = ctypes.create_string_buffer(256)
    p = (ctypes.addressof(buf) + 15) & ~15
    assert L.stm_nf4_gemm_workspace_bytes(512, 4096, 14336, 0) > 16 << 20
    assert L.stm_nf4_gemm_fwd_noalloc(p, p, p, None, None, None, 0, p, 512, 4096, 14336, 64, 1, None) == -2
    assert "static scratch" in _err(L)
    # the same argument checks as stm_nf4_gemm_fwd
    assert L.stm_nf4_gemm_fwd_noalloc(p, p, p, None, None, None, 0, p, 16, 4096, 100, 64, 1, None) == -2
    assert L.stm_nf4_gemm_fwd_noalloc(None, p, p, None, None, None, 0, p, 16, 4096, 128, 64, 1, None) == -1
    assert L.stm_nf4_gemm_fwd_noalloc(p, p, p, None, None, None, 8, p, 16, 4096, 128, 64, 1, None) == -1


@pytest.mark.parametrize("counts, rows", [
    # top-8 of 8192 tokens over 128 experts: ~512 rows each, half just above 512.
    # 256-row tiles: 64 * (2 + 0.45) + 64 * 2 = 284.8 units; 192-row tiles
    # 128 * 3 * 0.81 = 311: the 256-row tile with a short last item
    ([540] * 64 + [490] * 64, 256),
    ([512] * 16, 256),          # 32 units against 38.9
    ([256] * 8, 256),           # exact 256-row tiles
    ([100] * 8, 256),           # one 128-row short item each (0.6) against one 192-row item (0.81)
    ([180, 190] * 4, 192),      # 192-row items (0.81) against full 256-row items (1)
    ([0, 0, 0], 256),           # nothing to compute: the default
    ([0, 520, 0, 515], 192),    # empty experts skipped: 4.9 units against 4.86
    ([576] * 4, 192),           # 3 * 0.81 = 2.43 against 2 + 0.45 = 2.45
    ([700], 256),               # 3 units against 3.24
])
def test_grouped_tile_rows_picks_the_fewest_padded_rows(L, counts, rows):
    import numpy as np
    off = np.zeros(len(counts) + 1, dtype=np.int32)
    off[1:] = np.cumsum(counts)
    assert L.stm_nf4_grouped_tile_rows(off.ctypes.data, len(counts)) == rows


@pytest.mark.parametrize("offsets, max_rows, msg", [
    ([0, 5, 3], 16, "decrease at expert 1"),
    ([2, 5, 9], 16, "offsets[0] = 2"),
    ([0, 5, 30], 16, "expert 1 has 25 rows, above max_rows 16"),
    ([0, 0, -4], 16, "decrease at expert 1"),
])
def test_grouped_calls_refuse_bad_host_offsets_before_any_launch(L, offsets, max_rows, msg):
    """Host offsets that break the contract (start at 0, never decrease, no
    expert above max_rows) are refused by every grouped entry point before a
    kernel is launched (these calls would otherwise need a GPU)."""
    off = np.asarray(offsets, dtype=np.int32)
    E = len(offsets) - 1
    p = 4096  # a non-NULL, 256-byte aligned stand-in: never dereferenced
    rc = L.stm_nf4_grouped_gemm_fwd(p, p, p, p, off.ctypes.data, E, max_rows, p, 64, 64, 64, 1, None)
    assert rc == -1 and msg in _err(L)
    rc = L.stm_nf4_grouped_gemm_bwd_dx(p, p, p, p, off.ctypes.data, E, max_rows, p, 64, 64, 64, 1, None)
    assert rc == -1 and msg in _err(L)
    if "max_rows" not in msg:  # the tile planner has no row bound
        assert L.stm_nf4_grouped_tile_rows(off.ctypes.data, E) == -1 and msg in _err(L)


def test_stack_nf4_equals_quantizing_the_stacked_weight():
    """Byte-concatenated payloads of weights sharing K are the payload of the
    row-stacked weight (checked through the C oracle); mismatched K or
    blocksize is refused."""
    import torch
    from stratum_amd.functional import QuantState, stack_nf4
    g = torch.Generator().manual_seed(5)
    ws = [(torch.randn(n, 320, generator=g) * 0.02).half() for n in (64, 8, 128)]

    def payload(w, bs=64):
        p, a = C.quantize(w.view(torch.int16).numpy().view(np.uint16), O.DT_F16, bs)
        return torch.from_numpy(p).reshape(-1, 1), QuantState(absmax=torch.from_numpy(a), shape=w.shape,
                                                              blocksize=bs, dtype=torch.float16)
    p, st = stack_nf4([payload(w) for w in ws])
    rp, ra = C.quantize(torch.cat(ws).view(torch.int16).numpy().view(np.uint16), O.DT_F16, 64)
    np.testing.assert_array_equal(p.numpy().ravel(), rp)
    np.testing.assert_array_equal(st.absmax.numpy(), ra)
    assert tuple(st.shape) == (200, 320) and st.blocksize == 64 and st.dtype == torch.float16
    with pytest.raises(ValueError):
        stack_nf4([payload(ws[0]), payload((torch.randn(8, 256) * 0.02).half())])
    with pytest.raises(ValueError):
        stack_nf4([payload(ws[0]), payload(ws[1], bs=128)])
    with pytest.raises(ValueError):
        stack_nf4([])


@pytest.mark.parametrize("name,kind", [("big", 0), ("small", 1), ("mid", 2), ("big8", 3), ("bogus", -1)])
def test_tile_env_names_map_to_tile_kinds(name, kind):
    """STRATUM_NF4_GEMM_TILE, read once when the library loads, pins the tile
    kind that stm_nf4_gemm_set_tile reports back (each documented name; any
    other value leaves the cost model in charge)."""
    import subprocess
    import sys
    code = ("from stratum_amd import _lib; L = _lib.lib(); "
            "print(L.stm_nf4_gemm_set_tile(-1))")
    env = dict(os.environ, STRATUM_NF4_GEMM_TILE=name)
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    assert int(out.stdout.strip().splitlines()[-1]) == kind


@pytest.mark.parametrize("fn", ["fwd", "bwd"])
def test_gemm_wrappers_reject_short_or_mistyped_weights_before_launch(fn):
    """nf4_gemm_fwd / nf4_gemm_bwd_dx check the packed codes, absmax (and bias)
    against the weight shape on the host: a short tensor would otherwise be read
    past its end by the kernels (CPU tensors here, so nothing is launched)."""
    import torch
    from stratum_amd.functional import nf4_gemm_bwd_dx, nf4_gemm_fwd
    N, K = 128, 64
    x = torch.zeros(4, K if fn == "fwd" else N, dtype=torch.bfloat16)
    call = (lambda p, a, **kw: nf4_gemm_fwd(x, p, a, (N, K), 64, **kw)) if fn == "fwd" else \
        (lambda p, a, **kw: nf4_gemm_bwd_dx(x, p, a, (N, K), 64, **kw))
    good_p, good_a = torch.zeros(N * K // 2, dtype=torch.uint8), torch.ones(N * K // 64)
    with pytest.raises(ValueError, match="packed holds"):
        call(good_p[:-1], good_a)
    with pytest.raises(ValueError, match="absmax holds"):
        call(good_p, good_a[:-1])
    with pytest.raises(ValueError, match="uint8"):
        call(good_p.to(torch.int16), good_a)
    with pytest.raises(ValueError, match="float32"):
        call(good_p, good_a.double())
    if fn == "fwd":
        with pytest.raises(ValueError, match="bias"):
            call(good_p, good_a, bias=torch.zeros(N - 1, dtype=torch.bfloat16))


def test_wrappers_refuse_operands_on_another_device():
    """A host pointer handed to a kernel beside device ones is refused on the host
    (here every operand but one is on the meta device, so nothing can launch)."""
    import torch
    from stratum_amd.functional import _on_device
    dev = torch.device("meta")
    _on_device(dev, a=torch.empty(2, device=dev), b=None)
    with pytest.raises(ValueError, match="b is on cpu"):
        _on_device(dev, a=torch.empty(2, device=dev), b=torch.zeros(2))
