"""NumPy restatement of the NF4 blockwise quantize / pack / dequantize path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker for the HIP
kernels, never the thing measured or shipped.

Reference behaviour restated here (the reference itself holds no arithmetic;
it calls the third-party ``bitsandbytes.functional``, version unpinned in
``pyproject.toml:19`` / ``Dockerfile:51``, absent from the reference tree):

* ``quantize_4bit(weight, blocksize=64, compress_statistics=False,
  quant_type="nf4")`` at ``stratum/upload.py:367-369`` and ``:725-727`` on a
  CPU, contiguous, 2-D (``[-1, last]`` for stacked experts, ``:365-366``)
  tensor. Published algorithm: flatten row-major; per block of ``blocksize``
  elements ``absmax = max|x|`` kept in fp32; ``s = fp32(x) * fp32(1/absmax)``;
  code = nearest NF4 level; two codes per byte, even element in the high nibble.
* ``dequantize_4bit(q, QuantState(...))`` at ``stratum/upload.py:221,946,1038``
  and ``stratum/nf4_linear.py:46``: ``out = dtype(fp32(code[q]) * absmax)`` with
  one fp32 product followed by a round-to-nearest-even conversion.

bitsandbytes has two published rules for "nearest level":

* ``"argmin"``: the torch/CPU backend: ``clamp(s, -1, 1)`` then
  ``argmin(|s - code|)`` over fp32 distances, first index on ties. This is what
  the reference runs, since it quantizes CPU tensors (``stratum/upload.py:360``).
* ``"threshold"``: the CUDA kernel: a comparison tree on the fp32-rounded
  midpoints of adjacent levels with a strict ``>``.

Both give code 0 for NaN scales (an all-zero block has ``absmax = 0`` and
``0 * inf = NaN``).
"""

from __future__ import annotations

import numpy as np

# NF4 levels (QLoRA, arXiv 2305.14314, Appendix E), the fp32 table that
# bitsandbytes returns as QuantState.code and the reference stores in
# NF4Payload.code (stratum/upload.py:78,372,733).
NF4_CODE = np.array(
    [
        -1.0,
        -0.6961928009986877,
        -0.5250730514526367,
        -0.39491748809814453,
        -0.28444138169288635,
        -0.18477343022823334,
        -0.09105003625154495,
        0.0,
        0.07958029955625534,
        0.16093020141124725,
        0.24611230194568634,
        0.33791524171829224,
        0.44070982933044434,
        0.5626170039176941,
        0.7229568362236023,
        1.0,
    ],
    dtype=np.float32,
)

ROUNDINGS = ("argmin", "threshold")

# dtype tags shared with the C restatement
DT_F16, DT_BF16, DT_F32 = 0, 1, 2


def midpoint_thresholds() -> np.ndarray:
    """fp32-rounded midpoints of adjacent levels (the CUDA comparison tree's constants)."""
    c = NF4_CODE.astype(np.float64)
    return ((c[:-1] + c[1:]) / 2.0).astype(np.float32)


# ---------------------------------------------------------------- bf16 helpers
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | np.uint32(0x40)).astype(np.uint16)  # quiet NaN
    return out


def to_f32(x: np.ndarray, dtype_tag: int) -> np.ndarray:
    """Exact widening of fp16 / bf16 (uint16 bits) / fp32 input to fp32."""
    if dtype_tag == DT_F16:
        return np.asarray(x, dtype=np.float16).astype(np.float32).ravel()
    if dtype_tag == DT_BF16:
        return bf16_bits_to_f32(np.asarray(x).ravel())
    if dtype_tag == DT_F32:
        return np.asarray(x, dtype=np.float32).ravel()
    raise ValueError(f"unknown dtype tag {dtype_tag}")


# ------------------------------------------------------------------- quantize
def block_absmax(xf: np.ndarray, blocksize: int) -> np.ndarray:
    """Per-block max|x| in fp32; the last block may be partial; NaN propagates
    (torch ``abs().max(dim=-1)`` semantics)."""
    n = xf.size
    nb = -(-n // blocksize)
    pad = nb * blocksize - n
    a = np.abs(np.concatenate([xf, np.zeros(pad, np.float32)])).reshape(nb, blocksize)
    return a.max(axis=1).astype(np.float32)  # np.max propagates NaN


def scaled_values(xf: np.ndarray, absmax: np.ndarray, blocksize: int) -> np.ndarray:
    """s = fp32(x) * fp32(1 / absmax) with one rounding per operation."""
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        inv = np.float32(1.0) / absmax
        blk = np.arange(xf.size) // blocksize
        return (xf * inv[blk]).astype(np.float32)


def nearest_codes(s: np.ndarray, rounding: str = "argmin", chunk: int = 1 << 20) -> np.ndarray:
    if rounding == "argmin":
        out = np.empty(s.size, np.uint8)
        for i in range(0, s.size, chunk):
            part = np.clip(s[i:i + chunk], np.float32(-1), np.float32(1))
            with np.errstate(invalid="ignore"):
                d = np.abs(part[:, None] - NF4_CODE[None, :])
            out[i:i + chunk] = np.argmin(d, axis=1)  # NaN rows -> index 0; ties -> first
        return out
    if rounding == "threshold":
        t = midpoint_thresholds()
        out = np.empty(s.size, np.uint8)
        for i in range(0, s.size, chunk):
            with np.errstate(invalid="ignore"):
                out[i:i + chunk] = (s[i:i + chunk, None] > t[None, :]).sum(axis=1)
        return out
    raise ValueError(f"unknown rounding {rounding!r}")


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """Two codes per byte, even element in the high nibble; odd length pads a zero low nibble."""
    c = np.asarray(codes, dtype=np.uint8).ravel()
    if c.size % 2:
        c = np.concatenate([c, np.zeros(1, np.uint8)])
    return ((c[0::2] << 4) | c[1::2]).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray, n: int) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8).ravel()
    c = np.empty(p.size * 2, np.uint8)
    c[0::2] = p >> 4
    c[1::2] = p & 0x0F
    return c[:n]


def quantize(x: np.ndarray, dtype_tag: int, blocksize: int = 64, rounding: str = "argmin"):
    """Returns (packed uint8 [(n+1)//2], absmax fp32 [ceil(n/blocksize)], codes uint8 [n])."""
    xf = to_f32(x, dtype_tag)
    absmax = block_absmax(xf, blocksize)
    s = scaled_values(xf, absmax, blocksize)
    codes = nearest_codes(s, rounding)
    return pack_nibbles(codes), absmax, codes


# ----------------------------------------------------------------- dequantize
def dequantize_f32(packed: np.ndarray, absmax: np.ndarray, n: int, blocksize: int = 64) -> np.ndarray:
    """fp32 products code[q] * absmax (before the output-dtype rounding)."""
    codes = unpack_nibbles(packed, n)
    blk = np.arange(n) // blocksize
    return (NF4_CODE[codes] * np.asarray(absmax, np.float32)[blk]).astype(np.float32)


def dequantize(packed: np.ndarray, absmax: np.ndarray, n: int, blocksize: int, out_tag: int) -> np.ndarray:
    """fp16 -> np.float16 array; bf16 -> uint16 bit patterns; fp32 -> np.float32."""
    v = dequantize_f32(packed, absmax, n, blocksize)
    if out_tag == DT_F16:
        with np.errstate(over="ignore"):
            return v.astype(np.float16)  # numpy's float->half is round-to-nearest-even
    if out_tag == DT_BF16:
        return f32_to_bf16_bits(v)
    if out_tag == DT_F32:
        return v
    raise ValueError(f"unknown dtype tag {out_tag}")


# ------------------------------------------------ decision boundaries (fp32)
def _f32_next(x: np.float32) -> np.float32:
    return np.nextafter(np.float32(x), np.float32(np.inf), dtype=np.float32)


def decision_boundaries(rounding: str) -> np.ndarray:
    """For each i in 0..14 the smallest fp32 ``s`` that the rule maps to a code
    > i. Found by scanning fp32 values outward from the midpoint and applying
    ``nearest_codes`` itself, so it is a consequence of the rule, not a restatement."""
    out = np.empty(15, np.float32)
    mids = midpoint_thresholds()
    for i in range(15):
        m = mids[i]
        # window of +-4096 ulps around the midpoint holds the switch point
        bits = m.view(np.int32) if m != 0 else np.int32(0)
        if m >= 0:
            cand_bits = np.arange(int(bits) - 4096, int(bits) + 4096, dtype=np.int64)
            cand = cand_bits.astype(np.int32).view(np.float32)
        else:
            cand_bits = np.arange(int(bits) + 4096, int(bits) - 4096, -1, dtype=np.int64)
            cand = cand_bits.astype(np.int32).view(np.float32)
        cand = np.sort(cand)
        codes = nearest_codes(cand, rounding)
        first = np.argmax(codes > i)
        assert codes[first] == i + 1 and codes[0] <= i, (i, rounding)
        out[i] = cand[first]
    return out
