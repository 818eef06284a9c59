"""Pins the CPU oracle (oracle/) with checks that do not restate its formulas:
the published construction of the codebook, brute force in float64, special
values, known-answer bytes, torch's own rounding, a second independently written
C restatement, and the committed golden fixtures."""

import glob
import os

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import nf4_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def seeded(shape, seed, std, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def as_np(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16), O.DT_BF16
    if t.dtype == torch.float16:
        return t.numpy(), O.DT_F16
    return t.numpy(), O.DT_F32


# --------------------------------------------------------------- codebook
def test_codebook_is_the_qlora_normal_quantile_construction():
    """QLoRA (arXiv 2305.14314, App. E): 8 positive quantiles of N(0,1) from
    linspace(offset, 0.5, 9), 7 negative from linspace(offset, 0.5, 8), plus 0,
    normalised by the max; offset = 0.9677083. With the float32 linspace this
    reproduces every literal bit for bit."""
    from scipy.stats import norm
    offset = 0.9677083
    pos = norm.ppf(torch.linspace(offset, 0.5, 9)[:-1].numpy())
    neg = -norm.ppf(torch.linspace(offset, 0.5, 8)[:-1].numpy())
    v = np.sort(np.concatenate([pos, [0.0], neg]))
    v = (v / v.max()).astype(np.float32)
    np.testing.assert_array_equal(v, O.NF4_CODE)


def test_codebook_invariants():
    c = O.NF4_CODE
    assert c.dtype == np.float32 and c.size == 16
    assert np.all(np.diff(c) > 0)
    assert c[0] == -1.0 and c[7] == 0.0 and c[15] == 1.0


def test_product_codebook_matches_oracle():
    from stratum_amd.functional import NF4_LEVELS, get_4bit_type
    np.testing.assert_array_equal(np.array(NF4_LEVELS, np.float32), O.NF4_CODE)
    np.testing.assert_array_equal(get_4bit_type("nf4").numpy(), O.NF4_CODE)


# ----------------------------------------------------------------- absmax
def test_absmax_brute_force_with_partial_block():
    x = seeded((300,), 7, 1.0, torch.float32).numpy()
    am = O.block_absmax(x, 64)
    expect = [max(abs(float(v)) for v in x[i:i + 64]) for i in range(0, 300, 64)]
    assert am.tolist() == pytest.approx(expect, abs=0, rel=0)
    assert am.size == 5


def test_absmax_nan_propagates_and_zero_block():
    x = np.zeros(128, np.float32)
    x[70] = np.nan
    am = O.block_absmax(x, 64)
    assert am[0] == 0.0 and np.isnan(am[1])


# ------------------------------------------------------------ code choice
@pytest.mark.parametrize("rule", O.ROUNDINGS)
def test_codes_equal_float64_nearest_level_away_from_midpoints(rule):
    x = seeded((64, 512), 11, 0.02, torch.float16).numpy()
    xf = x.astype(np.float64).ravel()
    _, absmax, codes = O.quantize(x, O.DT_F16, 64, rule)
    s = xf / np.repeat(absmax.astype(np.float64), 64)
    d = np.abs(s[:, None] - O.NF4_CODE.astype(np.float64)[None, :])
    nearest = d.argmin(1)
    srt = np.sort(d, 1)
    clear = (srt[:, 1] - srt[:, 0]) > 1e-5  # not within rounding distance of a midpoint
    assert clear.mean() > 0.999
    np.testing.assert_array_equal(codes[clear], nearest[clear])


@pytest.mark.parametrize("rule", O.ROUNDINGS)
def test_special_values(rule):
    a = np.float32(0.37)
    x = np.array([a, -a, 0.0, a / 2] + [0.0] * 60 + [0.0] * 64, np.float32)
    _, absmax, codes = O.quantize(x, O.DT_F32, 64, rule)
    assert absmax[0] == a and absmax[1] == 0.0
    assert codes[0] == 15 and codes[1] == 0 and codes[2] == 7
    assert codes[3] == 12  # 0.5 lies between 0.4407 and 0.5626, nearer 0.4407
    assert np.all(codes[64:] == 0)  # zero block: 0 * inf = NaN -> code 0 under both rules


def test_rules_differ_only_at_fp32_midpoints():
    """The threshold rule maps an exact fp32 midpoint down; the argmin rule's
    choice there depends on the two fp32 distances. Away from midpoints they agree."""
    t = O.midpoint_thresholds()
    thr = O.nearest_codes(t, "threshold")
    np.testing.assert_array_equal(thr, np.arange(15))
    arg = O.nearest_codes(t, "argmin")
    assert set(np.unique(arg - thr)) <= {0, 1}
    up = np.array([np.nextafter(v, np.float32(2)) for v in t], np.float32)
    dn = np.array([np.nextafter(v, np.float32(-2)) for v in t], np.float32)
    np.testing.assert_array_equal(O.nearest_codes(up, "threshold"), np.arange(1, 16))
    np.testing.assert_array_equal(O.nearest_codes(dn, "argmin"), np.arange(15))


def test_decision_boundaries_characterise_the_rules():
    """Each boundary b_i is where the rule switches from level i to i+1:
    argmin compares fp32 distances, threshold is the next float above the midpoint."""
    c = O.NF4_CODE
    b = O.decision_boundaries("argmin")
    for i in range(15):
        lo = np.nextafter(b[i], np.float32(-2))
        assert np.abs(np.float32(b[i]) - c[i + 1]) < np.abs(np.float32(b[i]) - c[i])
        assert not (np.abs(lo - c[i + 1]) < np.abs(lo - c[i]))
    bt = O.decision_boundaries("threshold")
    t = ((c[:-1].astype(np.float64) + c[1:].astype(np.float64)) / 2).astype(np.float32)
    np.testing.assert_array_equal(bt, np.nextafter(t, np.float32(2)))


@pytest.mark.parametrize("shape,seed", [
    ((5632, 2048), 0),     # the round-trip matrix
    ((14336, 4096), 1),    # 8B gate / up projection, the LoRA-step weight
    ((4096, 14336), 2),    # 8B down projection
    ((3072, 1024), 3),     # Qwen3-0.6B gate / up
    ((16 * 1536, 2048), 4),  # 16 experts of the MoE gate_up bank
])
def test_rules_differ_only_at_exact_midpoints_on_the_workload_matrices(shape, seed):
    """The two published assignment rules (bitsandbytes' torch/CPU argmin and
    its CUDA threshold tree) on every workload matrix (fp16 N(0, 0.02)): the
    same absmax, and codes that differ only for elements whose scaled value is
    exactly an fp32 midpoint between two levels, where the threshold rule takes
    the lower level. There are a handful of such elements per matrix (one
    -0.0368042 / 0.060272217 pair of fp16 values lands on the midpoint between
    levels 1 and 2), not none."""
    x = seeded(shape, seed, 0.02, torch.float16).numpy().view(np.uint16)
    threads = min(8, os.cpu_count() or 1)
    pa, aa = C.quantize(x, O.DT_F16, 64, "argmin", threads)
    pt, at = C.quantize(x, O.DT_F16, 64, "threshold", threads)
    np.testing.assert_array_equal(aa, at)
    bytes_ = np.nonzero(pa != pt)[0]
    assert bytes_.size <= 32, bytes_.size
    if bytes_.size == 0:
        return
    elems = np.concatenate([2 * bytes_, 2 * bytes_ + 1])
    xf = O.to_f32(x.ravel()[elems].view(np.float16), O.DT_F16)
    s = O.scaled_values(xf, aa[elems // 64], 1)
    mids = O.midpoint_thresholds()
    code_a, code_t = O.nearest_codes(s, "argmin"), O.nearest_codes(s, "threshold")
    differ = code_a != code_t
    assert differ.any()
    np.testing.assert_array_equal(np.isin(s[differ], mids), True)
    np.testing.assert_array_equal(code_t[differ], np.searchsorted(mids, s[differ]))
    # the packed bytes carry exactly these codes (high nibble = even element)
    for rule_codes, packed in ((code_a, pa), (code_t, pt)):
        nib = np.where(elems % 2 == 0, packed[elems // 2] >> 4, packed[elems // 2] & 15)
        np.testing.assert_array_equal(nib, rule_codes)


# ---------------------------------------------------------------- packing
def test_pack_known_answers():
    np.testing.assert_array_equal(O.pack_nibbles([1, 2, 3, 4]), np.array([0x12, 0x34], np.uint8))
    np.testing.assert_array_equal(O.pack_nibbles([15, 0, 7]), np.array([0xF0, 0x70], np.uint8))
    np.testing.assert_array_equal(O.unpack_nibbles(np.array([0xAB, 0x5C], np.uint8), 3), [10, 11, 5])


# ------------------------------------------------------------- dequantize
@pytest.mark.parametrize("out_dtype,tag", [(torch.float16, O.DT_F16), (torch.bfloat16, O.DT_BF16)])
def test_dequant_rounding_matches_torch_conversion(out_dtype, tag):
    x = seeded((32, 256), 3, 0.02, torch.float16).numpy()
    packed, absmax, _ = O.quantize(x, O.DT_F16, 64)
    prod = O.dequantize_f32(packed, absmax, x.size, 64)
    ref = torch.from_numpy(prod).to(out_dtype)
    got = O.dequantize(packed, absmax, x.size, 64, tag)
    ref_bits = ref.view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got.view(np.uint16), ref_bits)


def test_dequant_endpoints_and_signed_zero():
    a = np.float32(0.0123)
    packed = O.pack_nibbles([15, 0, 7, 0] + [7] * 60 + [0] * 64)
    absmax = np.array([a, 0.0], np.float32)
    v = O.dequantize(packed, absmax, 128, 64, O.DT_F32)
    assert v[0] == a and v[1] == -a and v[2] == 0.0 and not np.signbit(v[2])
    assert np.all(v[64:] == 0) and np.all(np.signbit(v[64:]))  # -1 * 0 = -0.0


def test_roundtrip_error_bounded_by_half_gap():
    x = seeded((16, 1024), 5, 0.02, torch.float32).numpy()
    packed, absmax, _ = O.quantize(x, O.DT_F32, 64)
    v = O.dequantize_f32(packed, absmax, x.size, 64)
    half_gap = np.diff(O.NF4_CODE.astype(np.float64)).max() / 2
    bound = np.repeat(absmax.astype(np.float64), 64) * (half_gap + 1e-6)
    assert np.all(np.abs(v.astype(np.float64) - x.ravel()) <= bound)


# ------------------------------------------------ C restatement cross-check
@pytest.mark.parametrize("rule", O.ROUNDINGS)
@pytest.mark.parametrize("dtype,bs,shape", [
    (torch.float16, 64, (37, 128)), (torch.bfloat16, 128, (16, 256)), (torch.float32, 256, (3, 1000)),
    (torch.float16, 4096, (2, 4096)), (torch.float32, 64, (1001,)),
])
def test_c_restatement_agrees(rule, dtype, bs, shape):
    x, tag = as_np(seeded(shape, 21, 0.5, dtype))
    p, a, _ = O.quantize(x, tag, bs, rule)
    pc, ac = C.quantize(x, tag, bs, rule)
    np.testing.assert_array_equal(p, pc)
    np.testing.assert_array_equal(a.view(np.uint32), ac.view(np.uint32))
    for out_tag in (O.DT_F16, O.DT_BF16, O.DT_F32):
        d = O.dequantize(p, a, x.size, bs, out_tag)
        dc = C.dequantize(p, a, x.size, bs, out_tag)
        np.testing.assert_array_equal(d.view(np.uint16 if out_tag != O.DT_F32 else np.uint32),
                                      dc.view(np.uint16 if out_tag != O.DT_F32 else np.uint32))


def test_c_restatement_on_edge_values():
    x = np.load(os.path.join(GOLDEN, "nf4_f32_edge_bs64.npz"))["x"]
    for rule in O.ROUNDINGS:
        p, a, _ = O.quantize(x, O.DT_F32, 64, rule)
        pc, ac = C.quantize(x, O.DT_F32, 64, rule)
        np.testing.assert_array_equal(p, pc)


# ---------------------------------------------------------- golden vectors
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))))
def test_oracle_reproduces_golden_fixture(path):
    f = np.load(path)
    x, tag, bs = f["x"], int(f["dtype_tag"]), int(f["blocksize"])
    for rule in O.ROUNDINGS:
        p, a, _ = O.quantize(x, tag, bs, rule)
        np.testing.assert_array_equal(p, f[f"packed_{rule}"])
        np.testing.assert_array_equal(a.view(np.uint32), f[f"absmax_{rule}"].view(np.uint32))
    n = x.size
    np.testing.assert_array_equal(O.dequantize(f["packed_argmin"], f["absmax_argmin"], n, bs, O.DT_F16).view(np.uint16),
                                  f["deq_f16"])
    np.testing.assert_array_equal(O.dequantize(f["packed_argmin"], f["absmax_argmin"], n, bs, O.DT_BF16), f["deq_bf16"])
